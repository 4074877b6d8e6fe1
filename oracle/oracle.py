"""ctypes bindings for the CPU oracle and for the reference's own C library.

TEST INFRASTRUCTURE ONLY.  ``liboracle.so`` is this repository's restatement
of the reference algorithm (oracle/pyrite_oracle.c).  ``_ref/libpyrite_ref.so``
is the reference's own pyrite/kernels/native.c compiled unmodified by
oracle/Makefile; it exports the three reference entry points
(pyrite/kernels/native.c:484-576).  Both take numpy arrays.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "liboracle.so"
REF_SO = HERE / "_ref" / "libpyrite_ref.so"

_u8p = ctypes.POINTER(ctypes.c_uint8)
_dp = ctypes.POINTER(ctypes.c_double)
_fp = ctypes.POINTER(ctypes.c_float)
_ip = ctypes.POINTER(ctypes.c_int)

#: type id -> (name, elements per block, bytes per block); pyrite/ggml_types.py:34-74
TYPES = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20),
    6: ("Q5_0", 32, 22), 7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 9: ("Q8_1", 32, 36),
    10: ("Q2_K", 256, 84), 11: ("Q3_K", 256, 110), 12: ("Q4_K", 256, 144),
    13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210), 20: ("IQ4_NL", 32, 18),
    23: ("IQ4_XS", 256, 136), 24: ("I8", 1, 1), 25: ("I16", 1, 2), 26: ("I32", 1, 4),
    27: ("I64", 1, 8), 28: ("F64", 1, 8), 30: ("BF16", 1, 2),
}


def row_bytes(type_id: int, cols: int) -> int:
    _, bs, bpb = TYPES[type_id]
    assert cols % bs == 0
    return cols // bs * bpb


def build() -> None:
    """Compile liboracle.so (and _ref when the reference checkout is present)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def _ptr(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def _declare_abi(lib: ctypes.CDLL, prefix: str) -> None:
    mv = getattr(lib, f"{prefix}_matvec")
    mv.argtypes = (ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, _dp, _dp, ctypes.c_size_t, ctypes.c_size_t)
    mv.restype = ctypes.c_int
    dq = getattr(lib, f"{prefix}_dequantize_rows")
    dq.argtypes = (ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, _dp, ctypes.c_size_t, ctypes.c_size_t)
    dq.restype = ctypes.c_int
    nt = getattr(lib, f"{prefix}_native_types")
    nt.argtypes = (_ip, ctypes.c_size_t)
    nt.restype = ctypes.c_int


class _ABI:
    """The three-function C-ABI shared by the oracle and the reference build."""

    def __init__(self, lib: ctypes.CDLL, prefix: str):
        self.lib = lib
        self.prefix = prefix
        _declare_abi(lib, prefix)
        self._mv = getattr(lib, f"{prefix}_matvec")
        self._dq = getattr(lib, f"{prefix}_dequantize_rows")
        self._nt = getattr(lib, f"{prefix}_native_types")

    def native_types(self) -> list[int]:
        n = self._nt(None, 0)
        buf = (ctypes.c_int * n)()
        w = self._nt(buf, n)
        return [buf[i] for i in range(w)]

    def matvec_raw(self, type_id, data: np.ndarray, x: np.ndarray, out: np.ndarray, rows, cols) -> int:
        return self._mv(type_id, data.ctypes.data if data is not None else None,
                        0 if data is None else data.nbytes,
                        None if x is None else _ptr(x, _dp), None if out is None else _ptr(out, _dp),
                        rows, cols)

    def matvec(self, type_id: int, data: np.ndarray, x: np.ndarray, rows: int, cols: int) -> np.ndarray:
        data = np.ascontiguousarray(data, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float64)
        out = np.zeros(rows, dtype=np.float64)
        rc = self.matvec_raw(type_id, data, x, out, rows, cols)
        if rc != 0:
            raise ValueError(f"{self.prefix}_matvec error {rc}")
        return out

    def dequantize_rows(self, type_id: int, data: np.ndarray, rows: int, cols: int) -> np.ndarray:
        data = np.ascontiguousarray(data, dtype=np.uint8)
        out = np.zeros(rows * cols, dtype=np.float64)
        rc = self._dq(type_id, data.ctypes.data, data.nbytes, _ptr(out, _dp), rows, cols)
        if rc != 0:
            raise ValueError(f"{self.prefix}_dequantize_rows error {rc}")
        return out


class Oracle(_ABI):
    def __init__(self):
        if not ORACLE_SO.is_file():
            build()
        lib = ctypes.CDLL(str(ORACLE_SO))
        super().__init__(lib, "oracle")
        lib.oracle_quantize.argtypes = (ctypes.c_int, _dp, ctypes.c_size_t, _u8p)
        lib.oracle_quantize.restype = ctypes.c_long
        lib.oracle_fill_normal.argtypes = (ctypes.c_uint64, ctypes.c_double, ctypes.c_double, _fp, ctypes.c_size_t)
        lib.oracle_fill_normal.restype = None
        lib.oracle_decode_block.argtypes = (ctypes.c_int, _u8p, _dp)
        lib.oracle_decode_block.restype = ctypes.c_int
        lib.oracle_half_to_double.argtypes = (ctypes.c_uint16,)
        lib.oracle_half_to_double.restype = ctypes.c_double
        lib.oracle_double_to_half.argtypes = (ctypes.c_double, _ip)
        lib.oracle_double_to_half.restype = ctypes.c_uint16
        lib.oracle_softmax.argtypes = (_dp, ctypes.c_size_t, _dp)
        lib.oracle_silu.argtypes = (ctypes.c_double,)
        lib.oracle_silu.restype = ctypes.c_double
        lib.oracle_rms_norm.argtypes = (_dp, _dp, ctypes.c_size_t, ctypes.c_double, _dp)
        lib.oracle_argmax_first.argtypes = (_dp, ctypes.c_size_t)
        lib.oracle_argmax_first.restype = ctypes.c_long
        lib.oracle_route.argtypes = (_dp, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_int, ctypes.c_double,
                                     _ip, _dp, _dp)
        lib.oracle_route.restype = ctypes.c_int
        lib.oracle_moe_ffn.argtypes = (
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
            ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t,
            ctypes.c_int, ctypes.c_double, _dp, _dp, _ip, _dp, _dp)
        lib.oracle_moe_ffn.restype = ctypes.c_int
        lib.oracle_rope.argtypes = (_dp, ctypes.c_size_t, ctypes.c_long, ctypes.c_double, ctypes.c_size_t)
        lib.oracle_rope.restype = None
        lib.oracle_attention.argtypes = (
            _dp, _dp, _dp, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t,
            ctypes.c_double, ctypes.c_double, _dp, _dp, ctypes.c_long, _fp, _fp, ctypes.c_size_t, _dp)
        lib.oracle_attention.restype = ctypes.c_int

    # -- inputs
    def normal(self, seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        self.lib.oracle_fill_normal(seed, mean, std, _ptr(out, _fp), n)
        return out

    def quantize(self, type_id: int, values: np.ndarray) -> np.ndarray:
        v = np.ascontiguousarray(values, dtype=np.float64)
        _, bs, bpb = TYPES[type_id]
        out = np.zeros(v.size // bs * bpb, dtype=np.uint8)
        rc = self.lib.oracle_quantize(type_id, _ptr(v, _dp), v.size, _ptr(out, _u8p))
        if rc < 0:
            raise ValueError(f"oracle_quantize({type_id}) error {rc}")
        return out

    def decode_block(self, type_id: int, block: np.ndarray) -> np.ndarray:
        _, bs, _ = TYPES[type_id]
        b = np.ascontiguousarray(block, dtype=np.uint8)
        out = np.zeros(bs, dtype=np.float64)
        rc = self.lib.oracle_decode_block(type_id, _ptr(b, _u8p), _ptr(out, _dp))
        if rc:
            raise ValueError(rc)
        return out

    def half_to_double(self, h: int) -> float:
        return self.lib.oracle_half_to_double(h)

    def double_to_half(self, v: float) -> tuple[int, bool]:
        ovf = ctypes.c_int(0)
        h = self.lib.oracle_double_to_half(v, ctypes.byref(ovf))
        return h, bool(ovf.value)

    # -- routing / activations
    def softmax(self, v: np.ndarray) -> np.ndarray:
        v = np.ascontiguousarray(v, dtype=np.float64)
        out = np.empty_like(v)
        self.lib.oracle_softmax(_ptr(v, _dp), v.size, _ptr(out, _dp))
        return out

    def silu(self, v: float) -> float:
        return self.lib.oracle_silu(v)

    def rms_norm(self, x: np.ndarray, w: np.ndarray | None = None, eps: float = 1e-6) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float64)
        w = np.ones_like(x) if w is None else np.ascontiguousarray(w, dtype=np.float64)
        out = np.empty_like(x)
        self.lib.oracle_rms_norm(_ptr(x, _dp), _ptr(w, _dp), x.size, eps, _ptr(out, _dp))
        return out

    def argmax_first(self, v: np.ndarray) -> int:
        v = np.ascontiguousarray(v, dtype=np.float64)
        return int(self.lib.oracle_argmax_first(_ptr(v, _dp), v.size))

    def rope(self, v: np.ndarray, position: int, theta: float, rotary_dim: int = 0) -> np.ndarray:
        out = np.array(v, dtype=np.float64)
        self.lib.oracle_rope(_ptr(out, _dp), out.size, position, theta, rotary_dim)
        return out

    def attention(self, q, k, v, n_heads, n_kv, head_dim, value_dim, k_cache, v_cache, n_prev, position,
                  theta=10000.0, rotary_dim=0, eps=1e-6, q_norm=None, k_norm=None) -> np.ndarray:
        """One token's attention; k_cache/v_cache (fp32, [n_prev + 1, ...]) receive its key and value."""
        q = np.ascontiguousarray(q, dtype=np.float64)
        k = np.ascontiguousarray(k, dtype=np.float64)
        v = np.ascontiguousarray(v, dtype=np.float64)
        assert k_cache.dtype == np.float32 and v_cache.dtype == np.float32
        assert k_cache.flags.c_contiguous and v_cache.flags.c_contiguous
        assert k_cache.size >= (n_prev + 1) * n_kv * head_dim and v_cache.size >= (n_prev + 1) * n_kv * value_dim
        qn = None if q_norm is None else np.ascontiguousarray(q_norm, dtype=np.float64)
        kn = None if k_norm is None else np.ascontiguousarray(k_norm, dtype=np.float64)
        out = np.zeros(n_heads * value_dim, dtype=np.float64)
        rc = self.lib.oracle_attention(_ptr(q, _dp), _ptr(k, _dp), _ptr(v, _dp), n_heads, n_kv, head_dim, value_dim,
                                       rotary_dim, theta, eps, None if qn is None else _ptr(qn, _dp),
                                       None if kn is None else _ptr(kn, _dp), position, _ptr(k_cache, _fp),
                                       _ptr(v_cache, _fp), n_prev, _ptr(out, _dp))
        if rc:
            raise ValueError(f"oracle_attention error {rc}")
        return out

    def route(self, logits: np.ndarray, k: int, norm_topk_prob: bool = True, scale: float = 1.0):
        lg = np.ascontiguousarray(logits, dtype=np.float64)
        ids = np.zeros(k, dtype=np.int32)
        w = np.zeros(k, dtype=np.float64)
        probs = np.zeros(lg.size, dtype=np.float64)
        rc = self.lib.oracle_route(_ptr(lg, _dp), lg.size, k, int(norm_topk_prob), scale,
                                   _ptr(ids, _ip), _ptr(w, _dp), _ptr(probs, _dp))
        if rc:
            raise ValueError(rc)
        return ids, w, probs

    def moe_ffn(self, router, router_type, gate, gate_type, up, up_type, down, down_type,
                n_experts, hidden, inter, k, x, norm_topk_prob=True, scale=1.0):
        x = np.ascontiguousarray(x, dtype=np.float64)
        out = np.zeros(hidden, dtype=np.float64)
        ids = np.zeros(k, dtype=np.int32)
        w = np.zeros(k, dtype=np.float64)
        logits = np.zeros(n_experts, dtype=np.float64)
        rc = self.lib.oracle_moe_ffn(
            router.ctypes.data, router.nbytes, router_type,
            gate.ctypes.data, gate.nbytes, gate_type,
            up.ctypes.data, up.nbytes, up_type,
            down.ctypes.data, down.nbytes, down_type,
            n_experts, hidden, inter, k, int(norm_topk_prob), scale,
            _ptr(x, _dp), _ptr(out, _dp), _ptr(ids, _ip), _ptr(w, _dp), _ptr(logits, _dp))
        if rc:
            raise ValueError(f"oracle_moe_ffn error {rc}")
        return out, ids, w, logits


class Reference(_ABI):
    """The reference's native.c built unmodified into oracle/_ref (if present)."""

    def __init__(self):
        if not REF_SO.is_file():
            raise FileNotFoundError(str(REF_SO))
        super().__init__(ctypes.CDLL(str(REF_SO)), "pyrite")


_ORACLE: Oracle | None = None


def oracle() -> Oracle:
    global _ORACLE
    if _ORACLE is None:
        _ORACLE = Oracle()
    return _ORACLE


def reference() -> Reference | None:
    try:
        return Reference()
    except (FileNotFoundError, OSError):
        return None


def lcg_payload(type_id: int, rows: int, cols: int, seed: int = 20240607,
                finite_half: bytes = b"\x00\x3c") -> np.ndarray:
    """Byte payload built the way tests/test_native_kernels.py:61-87 builds it.

    LCG bytes ``state = (1103515245*state + 12345) & 0x7FFFFFFF`` emitting
    ``(state >> 8) & 0xFF``, with each block's fp16 scale words overwritten by a
    finite half (pyrite test SCALE_OFFSETS, :34-49, extended with Q3_K's d at
    byte 108 and Q8_1's sum at 2, which the reference leaves random).  F32/F64
    payloads are finite LCG floats as in :61-70.
    """
    name, bs, bpb = TYPES[type_id]
    n = rows * cols
    if type_id in (0, 28):
        state = seed
        vals = np.empty(n, dtype=np.float64)
        for i in range(n):
            state = (1103515245 * state + 12345) & 0x7FFFFFFF
            vals[i] = (state / 0x7FFFFFFF) * 2.0 - 1.0
        return (vals.astype("<f4") if type_id == 0 else vals.astype("<f8")).view(np.uint8).copy()
    nbytes = rows * (cols // bs) * bpb
    raw = np.empty(nbytes, dtype=np.uint8)
    state = seed
    for i in range(nbytes):
        state = (1103515245 * state + 12345) & 0x7FFFFFFF
        raw[i] = (state >> 8) & 0xFF
    offsets = SCALE_OFFSETS.get(type_id, ())
    fh = np.frombuffer(finite_half, dtype=np.uint8)
    for blk in range(nbytes // bpb):
        for off in offsets:
            raw[blk * bpb + off: blk * bpb + off + 2] = fh
    return raw


#: fp16 scale words per block (tests/test_native_kernels.py:34-49) plus Q3_K's d.
#: F16 and BF16 are excluded on purpose: patching their only word makes every
#: element 1.0 (a degenerate case); their random words are finite-filtered instead.
SCALE_OFFSETS = {
    2: (0,), 3: (0, 2), 6: (0,), 7: (0, 2), 8: (0,), 9: (0, 2), 10: (80, 82),
    11: (108,), 12: (0, 2), 13: (0, 2), 14: (208,), 20: (0,), 23: (0,),
}


def finite_halfwords(raw: np.ndarray) -> np.ndarray:
    """Replace non-finite fp16/bf16 words of a byte payload with 0.5 / 0.5."""
    w = raw.view("<u2").copy()
    bad = (w & 0x7C00) == 0x7C00
    w[bad] = 0x3800
    return w.view(np.uint8)


def finite_bf16words(raw: np.ndarray) -> np.ndarray:
    w = raw.view("<u2").copy()
    bad = (w & 0x7F80) == 0x7F80
    w[bad] = 0x3F00
    return w.view(np.uint8)


def env_seed(default: int) -> int:
    return int(os.environ.get("PYRITE_TEST_SEED", default))
