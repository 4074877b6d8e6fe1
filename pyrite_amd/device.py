"""Device-resident entry points over torch tensors (buffer ownership only).

Weights are GGUF block bytes uploaded verbatim into HBM as uint8 tensors;
activations and outputs are fp32 tensors on the same device.  Every call is
queued on torch's current stream and goes through the C ABI of
include/pyrite_hip.h.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from .ggml_types import spec


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def upload(payload, device: str | torch.device = "cuda") -> torch.Tensor:
    """Copy GGUF block bytes verbatim into device memory."""
    host = torch.frombuffer(bytearray(payload), dtype=torch.uint8) if not isinstance(payload, torch.Tensor) else payload
    return host.to(device=device, dtype=torch.uint8).contiguous()


def _ld(t: torch.Tensor) -> int:
    """Leading dimension of a [batch, n] tensor (size-1 batches may carry any stride)."""
    return t.stride(0) if t.shape[0] > 1 else t.shape[1]


def _check_weights(type_id: int, w: torch.Tensor, rows: int, cols: int) -> None:
    t = spec(type_id)
    if w.dtype != torch.uint8 or not w.is_cuda or not w.is_contiguous():
        raise ValueError("weights must be a contiguous uint8 CUDA tensor")
    if cols % t.block_size:
        raise ValueError(f"{t.name} needs cols divisible by {t.block_size}")


def _activations(x: torch.Tensor, device: torch.device, cols: int, name: str = "x") -> torch.Tensor:
    """x as a [batch, cols] view: fp32, on ``device``, rows contiguous.

    The kernels dereference the pointer on the GPU, so a host tensor or a
    tensor on another device is refused here, before any launch."""
    if not isinstance(x, torch.Tensor) or not x.is_cuda or x.device != device:
        raise ValueError(f"{name} must be a CUDA tensor on {device}")
    x2 = x.reshape(1, -1) if x.dim() == 1 else x
    if x2.dim() != 2 or x2.dtype != torch.float32 or x2.shape[1] != cols or x2.stride(1) != 1:
        raise ValueError(f"{name} must be fp32 [batch, {cols}] with contiguous rows")
    if x2.shape[0] < 1:
        raise ValueError(f"{name} has no vectors")
    return x2


def _output(y: torch.Tensor, device: torch.device, batch: int, n: int, name: str = "out") -> torch.Tensor:
    """An output as a [batch, n] view of the caller's own memory (never a copy).

    1-D outputs are accepted for batch 1.  Rows must be contiguous and must
    not overlap (stride(0) >= n), so every kernel write lands in ``y``."""
    if not isinstance(y, torch.Tensor) or not y.is_cuda or y.device != device:
        raise ValueError(f"{name} must be a CUDA tensor on {device}")
    if y.dtype != torch.float32:
        raise ValueError(f"{name} must be fp32")
    if y.dim() == 1 and batch == 1 and y.shape[0] == n and (n == 1 or y.stride(0) == 1):
        return y.view(1, n)
    if (y.dim() == 2 and tuple(y.shape) == (batch, n) and (n == 1 or y.stride(1) == 1)
            and (batch == 1 or y.stride(0) >= n)):
        return y
    raise ValueError(f"{name} must be fp32 [{batch}, {n}] (or [{n}] for one vector) with contiguous rows")


def matvec(type_id: int, w: torch.Tensor, x: torch.Tensor, rows: int, cols: int,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """y[b] = dequant(w) @ x[b]; x is [cols] or [batch, cols] fp32 (last dim contiguous)."""
    _check_weights(type_id, w, rows, cols)
    squeeze = x.dim() == 1
    x2 = _activations(x, w.device, cols)
    batch = x2.shape[0]
    if out is None:
        out = torch.empty(batch, rows, dtype=torch.float32, device=w.device)
    y2 = _output(out, w.device, batch, rows)
    lib = _lib.load()
    code = lib.pyrite_dev_matvec(type_id, w.data_ptr(), w.numel(), rows, cols, x2.data_ptr(), _ld(x2),
                                 y2.data_ptr(), _ld(y2), batch, _stream_ptr(w.device))
    _lib.check(code, "pyrite_dev_matvec")
    return out.reshape(rows) if squeeze else out


class _MatvecDesc(ctypes.Structure):
    """pyrite_matvec_desc (include/pyrite_hip.h)."""
    _fields_ = [("w", ctypes.c_void_p), ("w_len", ctypes.c_size_t), ("rows", ctypes.c_size_t),
                ("cols", ctypes.c_size_t), ("x", ctypes.c_void_p), ("ldx", ctypes.c_size_t),
                ("y", ctypes.c_void_p), ("ldy", ctypes.c_size_t)]


def matvec_grouped(type_id: int, mats: list[tuple[torch.Tensor, int, int]], x: torch.Tensor,
                   outs: list[torch.Tensor] | None = None) -> list[torch.Tensor]:
    """Same-type matrices (w, rows, cols) times the same x in one launch per 16 matrices
    (a layer's q/k/v or gate/up, pyrite/executor.py:689-697, 672-683).  Each output equals
    matvec() of that matrix alone, bit for bit."""
    if not mats:
        return []
    squeeze = x.dim() == 1
    dev = mats[0][0].device
    x2 = _activations(x, dev, x.shape[-1])
    batch = x2.shape[0]
    if outs is None:
        outs = [torch.empty(batch, rows, dtype=torch.float32, device=w.device) for w, rows, _ in mats]
    if len(outs) != len(mats):
        raise ValueError(f"{len(mats)} matrices but {len(outs)} outputs")
    descs = (_MatvecDesc * len(mats))()
    for i, ((w, rows, cols), y) in enumerate(zip(mats, outs)):
        _check_weights(type_id, w, rows, cols)
        if w.device != dev:
            raise ValueError(f"matrix {i} is on {w.device}, matrix 0 on {dev}")
        if x2.shape[1] != cols:
            raise ValueError(f"matrix {i}: x has {x2.shape[1]} columns, the matrix {cols}")
        y2 = _output(y, dev, batch, rows, f"outs[{i}]")
        descs[i] = _MatvecDesc(w.data_ptr(), w.numel(), rows, cols, x2.data_ptr(), _ld(x2), y2.data_ptr(), _ld(y2))
    lib = _lib.load()
    code = lib.pyrite_dev_matvec_grouped(type_id, descs, len(mats), batch, _stream_ptr(mats[0][0].device))
    _lib.check(code, "pyrite_dev_matvec_grouped")
    return [y.reshape(y.shape[-1]) if squeeze else y for y in outs]


def dequantize(type_id: int, w: torch.Tensor, rows: int, cols: int,
               dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Exact dequantization to fp32 or fp64 (fp64 is bit-identical to the reference)."""
    _check_weights(type_id, w, rows, cols)
    if dtype not in (torch.float32, torch.float64):
        raise ValueError("dtype must be float32 or float64")
    out = torch.empty(rows, cols, dtype=dtype, device=w.device)
    lib = _lib.load()
    code = lib.pyrite_dev_dequantize(type_id, w.data_ptr(), w.numel(), rows, cols, out.data_ptr(),
                                     int(dtype == torch.float64), _stream_ptr(w.device))
    _lib.check(code, "pyrite_dev_dequantize")
    return out


def lm_head_argmax(type_id: int, w: torch.Tensor, x: torch.Tensor, rows: int, cols: int,
                   logits: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """LM head: fp32 logits and the exact greedy token per vector.

    ``x`` is [cols] or [batch, cols] fp32.  Returns (logits [batch, rows] fp32,
    ids [batch] int32); ids equal the first index of the maximum of the
    reference's fp64 logits (pyrite/executor.py:852-875, pyrite/sampler.py:12-15).
    """
    _check_weights(type_id, w, rows, cols)
    x2 = _activations(x, w.device, cols)
    batch = x2.shape[0]
    if logits is None:
        logits = torch.empty(batch, rows, dtype=torch.float32, device=w.device)
    l2 = _output(logits, w.device, batch, rows, "logits")
    ids = torch.empty(batch, dtype=torch.int32, device=w.device)
    lib = _lib.load()
    code = lib.pyrite_dev_lm_head_argmax(type_id, w.data_ptr(), w.numel(), rows, cols, x2.data_ptr(),
                                         _ld(x2), l2.data_ptr(), _ld(l2), ids.data_ptr(),
                                         batch, _stream_ptr(w.device))
    _lib.check(code, "pyrite_dev_lm_head_argmax")
    return logits, ids


def rms_norm(x: torch.Tensor, weight: torch.Tensor | None = None, eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm over the last dim of fp32 x (pyrite/tensor_ops.py:502-506), fp64 inside."""
    if not isinstance(x, torch.Tensor) or not x.is_cuda:
        raise ValueError("x must be an fp32 CUDA tensor with contiguous rows")
    x2 = _activations(x, x.device, x.shape[-1])
    n = x2.shape[1]
    if weight is not None and (weight.dtype != torch.float32 or weight.numel() != n or not weight.is_contiguous()
                               or weight.device != x2.device):
        raise ValueError("weight must be a contiguous fp32 tensor of x's last dim on x's device")
    y = torch.empty_like(x2)
    lib = _lib.load()
    code = lib.pyrite_dev_rms_norm(x2.data_ptr(), _ld(x2), weight.data_ptr() if weight is not None else None,
                                   n, float(eps), y.data_ptr(), _ld(y), x2.shape[0], _stream_ptr(x2.device))
    _lib.check(code, "pyrite_dev_rms_norm")
    return y.reshape(x.shape)


class _MoeLayerC(ctypes.Structure):
    _fields_ = [
        ("router_type", ctypes.c_int), ("router", ctypes.c_void_p), ("router_len", ctypes.c_size_t),
        ("gate_type", ctypes.c_int), ("gate", ctypes.c_void_p), ("gate_len", ctypes.c_size_t),
        ("up_type", ctypes.c_int), ("up", ctypes.c_void_p), ("up_len", ctypes.c_size_t),
        ("down_type", ctypes.c_int), ("down", ctypes.c_void_p), ("down_len", ctypes.c_size_t),
        ("n_experts", ctypes.c_size_t), ("hidden", ctypes.c_size_t), ("inter", ctypes.c_size_t),
        ("k", ctypes.c_size_t), ("norm_topk_prob", ctypes.c_int), ("scale", ctypes.c_double),
    ]


@dataclass
class MoeLayer:
    """One Qwen3-MoE FFN layer's tensors in device memory (verbatim GGUF bytes).

    ``router`` is ffn_gate_inp [n_experts][hidden]; ``gate``/``up`` are the
    stacked [n_experts][inter][hidden] tensors and ``down`` [n_experts][hidden][inter]
    (pyrite/qwen3_moe.py:364-398, 432-443).
    """
    router_type: int
    router: torch.Tensor
    gate_type: int
    gate: torch.Tensor
    up_type: int
    up: torch.Tensor
    down_type: int
    down: torch.Tensor
    n_experts: int
    hidden: int
    inter: int
    k: int
    norm_topk_prob: bool = True
    scale: float = 1.0

    def _c(self) -> _MoeLayerC:
        for t in (self.router, self.gate, self.up, self.down):
            if t.dtype != torch.uint8 or not t.is_cuda or not t.is_contiguous():
                raise ValueError("MoE tensors must be contiguous uint8 CUDA tensors")
            if t.device != self.router.device:
                raise ValueError("MoE tensors must be on one device")
        return _MoeLayerC(self.router_type, self.router.data_ptr(), self.router.numel(),
                          self.gate_type, self.gate.data_ptr(), self.gate.numel(),
                          self.up_type, self.up.data_ptr(), self.up.numel(),
                          self.down_type, self.down.data_ptr(), self.down.numel(),
                          self.n_experts, self.hidden, self.inter, self.k, int(self.norm_topk_prob),
                          float(self.scale))


def moe_ffn(layer: MoeLayer, x: torch.Tensor, out: torch.Tensor | None = None
            ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Qwen3-MoE FFN for fp32 tokens x [batch, hidden] (pyrite/executor.py:757-793).

    Returns (out [batch, hidden] fp32, ids [batch, k] int32 in rank order,
    weights [batch, k] fp32); the ids equal the reference's expert choice.
    """
    dev = layer.router.device
    x2 = _activations(x, dev, layer.hidden)
    batch = x2.shape[0]
    if out is None:
        out = torch.empty(batch, layer.hidden, dtype=torch.float32, device=dev)
    o2 = _output(out, dev, batch, layer.hidden)
    ids = torch.empty(batch, layer.k, dtype=torch.int32, device=dev)
    wts = torch.empty(batch, layer.k, dtype=torch.float32, device=dev)
    c = layer._c()
    lib = _lib.load()
    code = lib.pyrite_dev_moe_ffn(ctypes.addressof(c), x2.data_ptr(), _ld(x2), o2.data_ptr(), _ld(o2),
                                  ids.data_ptr(), wts.data_ptr(), batch, _stream_ptr(dev))
    _lib.check(code, "pyrite_dev_moe_ffn")
    return out, ids, wts


def add_rms_norm(h: torch.Tensor, delta: torch.Tensor, weight: torch.Tensor | None, eps: float,
                 h_out: torch.Tensor | None = None, normed: torch.Tensor | None = None
                 ) -> tuple[torch.Tensor, torch.Tensor]:
    """Residual add and RMSNorm in one launch: h_out = h + delta (fp32) and
    normed = rms_norm(h_out) * weight (pyrite/executor.py:795-811).  h_out may be h."""
    n = h.shape[-1]
    h2 = _activations(h, h.device, n, "h")
    d2 = _activations(delta, h.device, n, "delta")
    batch = h2.shape[0]
    if d2.shape[0] != batch:
        raise ValueError("h and delta need the same number of vectors")
    if weight is not None and (weight.dtype != torch.float32 or weight.numel() != n or not weight.is_contiguous()
                               or weight.device != h.device):
        raise ValueError("weight must be a contiguous fp32 tensor of h's last dim on h's device")
    h_out = torch.empty_like(h2) if h_out is None else h_out
    normed = torch.empty_like(h2) if normed is None else normed
    o2 = _output(h_out, h.device, batch, n, "h_out")
    n2 = _output(normed, h.device, batch, n, "normed")
    lib = _lib.load()
    code = lib.pyrite_dev_add_rms_norm(h2.data_ptr(), _ld(h2), d2.data_ptr(), _ld(d2),
                                       weight.data_ptr() if weight is not None else None, n, float(eps),
                                       o2.data_ptr(), _ld(o2), n2.data_ptr(), _ld(n2), batch, _stream_ptr(h.device))
    _lib.check(code, "pyrite_dev_add_rms_norm")
    return h_out, normed


def matvec_swiglu(type_id: int, w: torch.Tensor, gate: torch.Tensor, up: torch.Tensor, rows: int, cols: int,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """y[b] = dequant(w) @ (silu(gate[b]) * up[b]): the dense FFN's down projection with its
    activation formed while the input is staged (pyrite/dense.py:473-495)."""
    _check_weights(type_id, w, rows, cols)
    squeeze = gate.dim() == 1
    g2 = _activations(gate, w.device, cols, "gate")
    u2 = _activations(up, w.device, cols, "up")
    if u2.shape != g2.shape or _ld(u2) != _ld(g2):
        raise ValueError("gate and up need the same shape and row stride")
    batch = g2.shape[0]
    if out is None:
        out = torch.empty(batch, rows, dtype=torch.float32, device=w.device)
    y2 = _output(out, w.device, batch, rows)
    lib = _lib.load()
    code = lib.pyrite_dev_matvec_swiglu(type_id, w.data_ptr(), w.numel(), rows, cols, g2.data_ptr(), u2.data_ptr(),
                                        _ld(g2), y2.data_ptr(), _ld(y2), batch, _stream_ptr(w.device))
    _lib.check(code, "pyrite_dev_matvec_swiglu")
    return out.reshape(rows) if squeeze else out


class _AttnLayerC(ctypes.Structure):
    """pyrite_attention_layer (include/pyrite_hip.h)."""
    _fields_ = [("n_heads", ctypes.c_size_t), ("n_kv_heads", ctypes.c_size_t), ("head_dim", ctypes.c_size_t),
                ("value_dim", ctypes.c_size_t), ("rotary_dim", ctypes.c_size_t), ("rope_theta", ctypes.c_double),
                ("eps", ctypes.c_double), ("q_norm", ctypes.c_void_p), ("k_norm", ctypes.c_void_p),
                ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p), ("capacity", ctypes.c_size_t)]


@dataclass
class AttentionCache:
    """One layer's attention geometry and its fp32 KV cache in device memory
    (the reference's LayerKV, pyrite/executor.py:79-141, as a ring of
    ``capacity`` slots; capacity = max_kv_tokens keeps the oldest-first
    eviction of LayerKV.truncate)."""
    n_heads: int
    n_kv_heads: int
    head_dim: int
    value_dim: int
    capacity: int
    rope_theta: float = 10000.0
    rotary_dim: int = 0
    eps: float = 1e-6
    q_norm: torch.Tensor | None = None
    k_norm: torch.Tensor | None = None
    device: str | torch.device = "cuda"
    tokens: int = 0  # tokens appended so far

    def __post_init__(self):
        self.k_cache = torch.zeros(self.capacity, self.n_kv_heads * self.head_dim, device=self.device)
        self.v_cache = torch.zeros(self.capacity, self.n_kv_heads * self.value_dim, device=self.device)
        for t in (self.q_norm, self.k_norm):
            if t is not None and (t.dtype != torch.float32 or t.numel() != self.head_dim or not t.is_contiguous()
                                  or t.device != self.k_cache.device):
                raise ValueError("QK-norm weights must be contiguous fp32 [head_dim] on the cache's device")

    def _c(self) -> _AttnLayerC:
        return _AttnLayerC(self.n_heads, self.n_kv_heads, self.head_dim, self.value_dim, self.rotary_dim,
                           float(self.rope_theta), float(self.eps),
                           self.q_norm.data_ptr() if self.q_norm is not None else None,
                           self.k_norm.data_ptr() if self.k_norm is not None else None,
                           self.k_cache.data_ptr(), self.v_cache.data_ptr(), self.capacity)


def attention_decode(cache: AttentionCache, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, position: int,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """One token's attention (pyrite/executor.py:685-755): QK-norm and RoPE at
    ``position``, the key and value appended to the cache, softmax-weighted values of
    every head over the cached tokens.  Returns [n_heads * value_dim] fp32."""
    dev = cache.k_cache.device
    nq, nk, nv = cache.n_heads * cache.head_dim, cache.n_kv_heads * cache.head_dim, cache.n_kv_heads * cache.value_dim
    for name, t, n in (("q", q, nq), ("k", k, nk), ("v", v, nv)):
        if (not isinstance(t, torch.Tensor) or not t.is_cuda or t.device != dev or t.dtype != torch.float32
                or t.numel() != n or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous fp32 tensor of {n} values on {dev}")
    if out is None:
        out = torch.empty(cache.n_heads * cache.value_dim, dtype=torch.float32, device=dev)
    elif (out.dtype != torch.float32 or out.device != dev or out.numel() != cache.n_heads * cache.value_dim
          or not out.is_contiguous()):
        raise ValueError("out must be a contiguous fp32 tensor of n_heads * value_dim values")
    slot = cache.tokens % cache.capacity
    n_ctx = min(cache.tokens + 1, cache.capacity)
    c = cache._c()
    lib = _lib.load()
    code = lib.pyrite_dev_attention_decode(ctypes.addressof(c), q.data_ptr(), k.data_ptr(), v.data_ptr(), position,
                                           slot, n_ctx, out.data_ptr(), _stream_ptr(dev))
    _lib.check(code, "pyrite_dev_attention_decode")
    cache.tokens += 1
    return out
