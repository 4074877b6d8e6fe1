"""One decode step of a dense (Llama / Qwen3) or Qwen3-MoE model on the device.

The step follows the reference executor over a checkpoint's resident tensors
(pyrite/executor.py:819-875 ``logits``, the layer at :795-811 and
pyrite/dense.py:497-513): the embedding row, then per layer RMSNorm,
the q/k/v projections, attention with QK-norm and RoPE over the layer's KV
cache, the output projection and residual add, RMSNorm, the FFN (dense
SwiGLU or the MoE layer) and residual add, then the output norm, the LM head
and the greedy token.  Nothing goes back to the host in between.

Differences in form, not in what is computed:
- Each residual add is fused with the RMSNorm that follows it (the FFN norm,
  the next layer's attention norm, or the output norm): one launch
  (``device.add_rms_norm``) writes both the new hidden state and its norm.
- The dense FFN's gate and up projections run as one grouped launch and the
  down projection forms silu(gate) * up while staging its input
  (``device.matvec_swiglu``).
- q/k/v run as grouped launches per GGML type.
- Activations are fp32 between the launches (the reference keeps fp64).

GGUF tensor names are the reference's: ``token_embd.weight``,
``blk.N.attn_norm.weight``, ``blk.N.attn_{q,k,v,output}.weight``,
``blk.N.attn_{q,k}_norm.weight`` (optional), ``blk.N.ffn_norm.weight``,
``blk.N.ffn_{gate,up,down}.weight`` (dense) or ``blk.N.ffn_gate_inp.weight``
and ``blk.N.ffn_{gate,up,down}_exps.weight`` (MoE), ``output_norm.weight``
and ``output.weight`` (else the tied embedding).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import device as _dev
from .resident import ResidentTensors


@dataclass(frozen=True)
class DecoderConfig:
    """The geometry the step needs (the reference's checkpoint config fields)."""
    hidden_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    value_dim: int
    rope_theta: float
    rms_norm_eps: float
    max_kv_tokens: int
    rotary_dim: int = 0                  # 0 = head_dim
    num_experts_per_tok: int = 0         # > 0: the FFN is a Qwen3-MoE layer
    norm_topk_prob: bool = True
    expert_weights_scale: float = 1.0


class Decoder:
    """Device decode over a ``ResidentTensors`` checkpoint; ``step`` forwards one token."""

    def __init__(self, tensors: ResidentTensors, cfg: DecoderConfig):
        self.t = tensors
        self.cfg = cfg
        self.device = tensors.device
        self.layers = []
        for i in range(cfg.num_hidden_layers):
            p = f"blk.{i}."
            L = {"attn_norm": self._vector(p + "attn_norm.weight", cfg.hidden_size),
                 "ffn_norm": self._vector(p + "ffn_norm.weight", cfg.hidden_size)}
            qn = p + "attn_q_norm.weight"
            kn = p + "attn_k_norm.weight"
            L["cache"] = _dev.AttentionCache(
                cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.value_dim, cfg.max_kv_tokens,
                rope_theta=cfg.rope_theta, rotary_dim=cfg.rotary_dim, eps=cfg.rms_norm_eps,
                q_norm=self._vector(qn, cfg.head_dim) if qn in tensors.names() else None,
                k_norm=self._vector(kn, cfg.head_dim) if kn in tensors.names() else None, device=self.device)
            if cfg.num_experts_per_tok > 0:
                L["moe"] = tensors.moe_layer(p + "ffn_gate_inp.weight", p + "ffn_gate_exps.weight",
                                             p + "ffn_up_exps.weight", p + "ffn_down_exps.weight",
                                             cfg.num_experts_per_tok, cfg.norm_topk_prob, cfg.expert_weights_scale)
            self.layers.append(L)
        self.output_norm = self._vector("output_norm.weight", cfg.hidden_size)
        self.head = "output.weight" if "output.weight" in tensors.names() else "token_embd.weight"

    def _vector(self, name: str, n: int) -> torch.Tensor:
        t = self.t.tensor(name)
        if t.ggml_type != 0 or t.dims != (n,):
            raise ValueError(f"{name} must be an F32 vector of {n} values, got type {t.ggml_type} dims {t.dims}")
        return self.t.view(name).view(torch.float32)

    def _grouped(self, names: list[str], x: torch.Tensor) -> list[torch.Tensor]:
        """Rank-2 tensors times x, one grouped launch per GGML type, results in `names` order."""
        by_type: dict[int, list[int]] = {}
        for i, n in enumerate(names):
            by_type.setdefault(self.t.tensor(n).ggml_type, []).append(i)
        out: list[torch.Tensor | None] = [None] * len(names)
        for idx in by_type.values():
            for i, y in zip(idx, self.t.grouped_matvec([names[i] for i in idx], x)):
                out[i] = y
        return out

    def step(self, token_id: int, position: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Forward one token at ``position``; returns (logits [vocab] fp32, greedy id [1] int32)."""
        cfg = self.cfg
        rows = self.t.tensor("token_embd.weight").dims[1]
        if not 0 <= token_id < rows:
            raise ValueError(f"token id {token_id} outside vocabulary ({rows})")
        if position < 0:
            raise ValueError("position must be non-negative")
        h = self.t.matrix_rows("token_embd.weight", token_id, 1)  # [1, hidden] fp32
        normed = _dev.rms_norm(h, self.layers[0]["attn_norm"], cfg.rms_norm_eps) if self.layers else h
        for i, L in enumerate(self.layers):
            p = f"blk.{i}."
            q, k, v = self._grouped([p + "attn_q.weight", p + "attn_k.weight", p + "attn_v.weight"], normed)
            a = _dev.attention_decode(L["cache"], q.reshape(-1), k.reshape(-1), v.reshape(-1), position)
            o = self.t.tensor_matvec(p + "attn_output.weight", cfg.hidden_size,
                                     cfg.num_attention_heads * cfg.value_dim, a.reshape(1, -1))
            h, normed2 = _dev.add_rms_norm(h, o, L["ffn_norm"], cfg.rms_norm_eps, h_out=h)
            if "moe" in L:
                d = _dev.moe_ffn(L["moe"], normed2)[0]
            else:
                g, u = self._grouped([p + "ffn_gate.weight", p + "ffn_up.weight"], normed2)
                dt = self.t.tensor(p + "ffn_down.weight")
                d = _dev.matvec_swiglu(dt.ggml_type, self.t.view(dt.name), g, u, dt.dims[1], dt.dims[0])
            nxt = self.layers[i + 1]["attn_norm"] if i + 1 < len(self.layers) else self.output_norm
            h, normed = _dev.add_rms_norm(h, d, nxt, cfg.rms_norm_eps, h_out=h)
        if not self.layers:
            normed = _dev.rms_norm(h, self.output_norm, cfg.rms_norm_eps)
        self.hidden = h
        logits, ids = self.t.lm_head(self.head, normed)
        return logits.reshape(-1), ids
