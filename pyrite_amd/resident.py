"""GGUF tensors resident in HBM, and the executor's matvec dispatch over them.

``ResidentTensors`` uploads a checkpoint's tensors verbatim (the GGUF block
bytes, no repacking) into one device arena, each tensor at a 256-byte aligned
offset, streaming the file through two pinned host buffers so that reading
chunk i+1 overlaps the host-to-device copy of chunk i.  The weights are then
used in place by the device kernels; nothing is re-read per token.

The dispatch methods mirror the reference executor's entry points with the
same argument meaning and errors, minus its host-side chunking (a launch
covers the whole row range):

- ``matrix_matvec``  = ``_matrix_matvec``  (pyrite/executor.py:481-509)
- ``tensor_matvec``  = ``_tensor_matvec``  (pyrite/executor.py:511-543)
- ``grouped_matvec`` = the q/k/v and gate/up projections in one launch
  (pyrite/executor.py:689-697, 672-683)
- ``expert_slice``   = ``expert_slice``    (pyrite/qwen3_moe.py:364-398)
- ``slice_matvec``   = ``_slice_matvec``   (pyrite/executor.py:545-594)
- ``matrix_rows``    = the embedding-row decode (pyrite/executor.py:458-479)
- ``lm_head``        = the LM-head loop plus greedy pick (pyrite/executor.py:852-875,
  pyrite/sampler.py:12-15)
- ``moe_layer``      = the stacked expert tensors of one Qwen3-MoE layer for
  ``device.moe_ffn`` (pyrite/executor.py:757-793)

GGML dims are (cols, rows[, experts]): the first dimension is the fastest.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import device as _dev
from .ggml_types import spec as ggml_spec
from .gguf import GGUFReader, GGUFTensor

ARENA_ALIGN = 256
STAGING_BYTES = 64 << 20


@dataclass(frozen=True)
class ExpertSlice:
    """One expert's contiguous 2-D slice of a stacked 3-D tensor."""
    tensor_name: str
    block_offset: int     # bytes from the tensor's start
    byte_length: int
    element_offset: int
    element_count: int
    shape: tuple[int, int]  # GGML (cols, rows)
    ggml_type: int


class ResidentTensors:
    """A GGUF checkpoint's tensors (all, or ``names``) uploaded into HBM verbatim."""

    def __init__(self, reader: GGUFReader, names=None, device: str | torch.device = "cuda",
                 staging_bytes: int = STAGING_BYTES):
        self.reader = reader
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("ResidentTensors needs a CUDA (HIP) device")
        wanted = list(reader.tensor_index()) if names is None else [reader.tensor(n) for n in names]
        self._at: dict[str, tuple[int, GGUFTensor]] = {}
        off = 0
        for t in wanted:
            if t.name in self._at:
                continue
            off = -(-off // ARENA_ALIGN) * ARENA_ALIGN
            self._at[t.name] = (off, t)
            off += t.size
        self.nbytes = off
        self.arena = torch.empty(max(off, 1), dtype=torch.uint8, device=self.device)
        self._upload(max(4096, int(staging_bytes)))

    def _upload(self, staging: int) -> None:
        # Two pinned buffers: the file is read into one while the other's
        # copy is in flight; an event per buffer guards its reuse.
        stream = torch.cuda.current_stream(self.device)
        bufs = [torch.empty(staging, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        views = [b.numpy() for b in bufs]
        done: list[torch.cuda.Event | None] = [None, None]
        k = 0
        with self.reader.path.open("rb", buffering=0) as fh:
            for dst, t in self._at.values():
                pos = 0
                while pos < t.size:
                    n = min(staging, t.size - pos)
                    if done[k] is not None:
                        done[k].synchronize()
                    fh.seek(t.offset + pos)
                    got = fh.readinto(memoryview(views[k])[:n])
                    if got != n:
                        raise ValueError(f"truncated tensor payload: {t.name}")
                    self.arena[dst + pos:dst + pos + n].copy_(bufs[k][:n], non_blocking=True)
                    ev = torch.cuda.Event()
                    ev.record(stream)
                    done[k] = ev
                    pos += n
                    k ^= 1
        for ev in done:
            if ev is not None:
                ev.synchronize()

    # -------------------------------------------------------------- tensors
    def names(self) -> tuple[str, ...]:
        return tuple(self._at)

    def tensor(self, name: str) -> GGUFTensor:
        try:
            return self._at[name][1]
        except KeyError as exc:
            raise KeyError(f"tensor {name!r} is not resident") from exc

    def view(self, name: str) -> torch.Tensor:
        """The tensor's verbatim bytes in HBM (a uint8 view of the arena)."""
        off, t = self._at[name] if name in self._at else (None, self.tensor(name))
        return self.arena[off:off + t.size]

    # ------------------------------------------------------------- dispatch
    @staticmethod
    def _vector(x: torch.Tensor, cols: int, name: str) -> torch.Tensor:
        if x.shape[-1] != cols:
            raise ValueError(f"matrix/vector shape mismatch for {name}")
        return x

    def matrix_matvec(self, name: str, first_row: int, row_count: int, x: torch.Tensor,
                      out: torch.Tensor | None = None) -> torch.Tensor:
        """Rows [first_row, first_row + row_count) of a rank-2 tensor times x ([cols] or [batch, cols])."""
        t = self.tensor(name)
        if len(t.dims) != 2:
            raise ValueError(f"{name} must be rank-2 for matrix-vector execution")
        cols, rows = t.dims
        self._vector(x, cols, name)
        if first_row < 0 or row_count < 0 or first_row + row_count > rows:
            raise ValueError(f"row range [{first_row}, {first_row + row_count}) outside {name}")
        if row_count == 0:
            shape = (0,) if x.dim() == 1 else (x.shape[0], 0)
            return torch.empty(shape, dtype=torch.float32, device=self.device)
        rb = ggml_spec(t.ggml_type)
        row_bytes = cols // rb.block_size * rb.bytes_per_block
        w = self.view(name)[first_row * row_bytes:(first_row + row_count) * row_bytes]
        return _dev.matvec(t.ggml_type, w, x, row_count, cols, out=out)

    def tensor_matvec(self, name: str, rows: int, cols: int, x: torch.Tensor,
                      out: torch.Tensor | None = None) -> torch.Tensor:
        """The whole matrix times x in one launch; dims must be (cols, rows)."""
        t = self.tensor(name)
        if len(t.dims) != 2 or t.dims != (cols, rows):
            raise ValueError(f"{name} has shape {t.dims}; expected GGML dimensions {(cols, rows)}")
        return self.matrix_matvec(name, 0, rows, x, out=out)

    def grouped_matvec(self, names, x: torch.Tensor) -> list[torch.Tensor]:
        """Several rank-2 tensors of one type times the same x in one launch (a layer's
        q/k/v or gate/up, pyrite/executor.py:689-697, 672-683); each result equals
        tensor_matvec of that tensor, bit for bit."""
        ts = [self.tensor(n) for n in names]
        if not ts:
            return []
        if any(len(t.dims) != 2 for t in ts):
            raise ValueError("grouped matvec needs rank-2 tensors")
        if len({t.ggml_type for t in ts}) != 1:
            raise ValueError("grouped matvec needs tensors of one GGML type")
        for t in ts:
            self._vector(x, t.dims[0], t.name)
        return _dev.matvec_grouped(ts[0].ggml_type, [(self.view(t.name), t.dims[1], t.dims[0]) for t in ts], x)

    def expert_slice(self, name: str, expert: int) -> ExpertSlice:
        """Expert ``expert``'s contiguous slice of a stacked (cols, rows, experts) tensor."""
        t = self.tensor(name)
        if len(t.dims) != 3:
            raise ValueError(f"{t.name} must be a stacked 3D expert tensor, got dims {t.dims}")
        if not 0 <= expert < t.dims[2]:
            raise IndexError(expert)
        inner = t.dims[0] * t.dims[1]
        b = ggml_spec(t.ggml_type)
        if inner % b.block_size:
            raise ValueError(f"{t.name} expert slice of {inner} values is not a multiple of the {b.name} "
                             f"block size {b.block_size}")
        element_offset = expert * inner
        return ExpertSlice(t.name, element_offset // b.block_size * b.bytes_per_block,
                           inner // b.block_size * b.bytes_per_block, element_offset, inner,
                           (t.dims[0], t.dims[1]), t.ggml_type)

    def slice_matvec(self, name: str, expert: int, rows: int, cols: int, x: torch.Tensor,
                     out: torch.Tensor | None = None) -> torch.Tensor:
        """One expert's slice times x, read in place from the stacked tensor."""
        s = self.expert_slice(name, expert)
        if s.element_count != rows * cols or x.shape[-1] != cols:
            raise ValueError("expert matrix/vector shape mismatch")
        b = ggml_spec(s.ggml_type)
        if cols % b.block_size:
            raise ValueError(f"expert row width {cols} is not aligned to {b.name} blocks")
        w = self.view(name)[s.block_offset:s.block_offset + s.byte_length]
        return _dev.matvec(s.ggml_type, w, x, rows, cols, out=out)

    def matrix_rows(self, name: str, first_row: int, row_count: int,
                    dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """Exact dequantized rows [first_row, first_row + row_count) as [row_count, cols]."""
        t = self.tensor(name)
        if len(t.dims) != 2:
            raise ValueError(f"{name} must be rank-2 for row streaming")
        cols, rows = t.dims
        if first_row < 0 or row_count < 0 or first_row + row_count > rows:
            raise ValueError(f"row range [{first_row}, {first_row + row_count}) outside {name}")
        if row_count == 0:
            return torch.empty(0, cols, dtype=dtype, device=self.device)
        b = ggml_spec(t.ggml_type)
        row_bytes = cols // b.block_size * b.bytes_per_block
        w = self.view(name)[first_row * row_bytes:(first_row + row_count) * row_bytes]
        return _dev.dequantize(t.ggml_type, w, row_count, cols, dtype=dtype)

    def lm_head(self, name: str, x: torch.Tensor, logits: torch.Tensor | None = None):
        """(fp32 logits, greedy first-max ids) of a rank-2 output tensor."""
        t = self.tensor(name)
        if len(t.dims) != 2:
            raise ValueError(f"{name} must be rank-2 for the LM head")
        cols, rows = t.dims
        self._vector(x, cols, name)
        return _dev.lm_head_argmax(t.ggml_type, self.view(name), x, rows, cols, logits=logits)

    def moe_layer(self, router: str, gate: str, up: str, down: str, k: int,
                  norm_topk_prob: bool = True, scale: float = 1.0) -> _dev.MoeLayer:
        """A Qwen3-MoE layer over resident ffn_gate_inp / ffn_{gate,up,down}_exps tensors."""
        tr, tg, tu, td = (self.tensor(n) for n in (router, gate, up, down))
        if len(tr.dims) != 2 or any(len(t.dims) != 3 for t in (tg, tu, td)):
            raise ValueError("router must be rank-2 and the expert tensors stacked rank-3")
        hidden, n_experts = tr.dims
        inter = tg.dims[1]
        if tg.dims != (hidden, inter, n_experts) or tu.dims != tg.dims or td.dims != (inter, hidden, n_experts):
            raise ValueError(f"expert tensor dims {tg.dims}, {tu.dims}, {td.dims} do not match router "
                             f"{tr.dims}")
        return _dev.MoeLayer(tr.ggml_type, self.view(router), tg.ggml_type, self.view(gate), tu.ggml_type,
                             self.view(up), td.ggml_type, self.view(down), n_experts, hidden, inter, k,
                             norm_topk_prob, scale)
