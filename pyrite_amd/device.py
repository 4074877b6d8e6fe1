"""Device-resident entry points over torch tensors (buffer ownership only).

Weights are GGUF block bytes uploaded verbatim into HBM as uint8 tensors;
activations and outputs are fp32 tensors on the same device.  Every call is
queued on torch's current stream and goes through the C ABI of
include/pyrite_hip.h.
"""
from __future__ import annotations

import torch

from . import _lib
from .ggml_types import spec


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def upload(payload, device: str | torch.device = "cuda") -> torch.Tensor:
    """Copy GGUF block bytes verbatim into device memory."""
    host = torch.frombuffer(bytearray(payload), dtype=torch.uint8) if not isinstance(payload, torch.Tensor) else payload
    return host.to(device=device, dtype=torch.uint8).contiguous()


def _check_weights(type_id: int, w: torch.Tensor, rows: int, cols: int) -> None:
    t = spec(type_id)
    if w.dtype != torch.uint8 or not w.is_cuda or not w.is_contiguous():
        raise ValueError("weights must be a contiguous uint8 CUDA tensor")
    if cols % t.block_size:
        raise ValueError(f"{t.name} needs cols divisible by {t.block_size}")


def matvec(type_id: int, w: torch.Tensor, x: torch.Tensor, rows: int, cols: int,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """y[b] = dequant(w) @ x[b]; x is [cols] or [batch, cols] fp32 (last dim contiguous)."""
    _check_weights(type_id, w, rows, cols)
    squeeze = x.dim() == 1
    x2 = x.reshape(1, -1) if squeeze else x
    if x2.dtype != torch.float32 or x2.shape[1] != cols or x2.stride(1) != 1:
        raise ValueError("x must be fp32 [batch, cols] with contiguous rows")
    batch = x2.shape[0]
    if out is None:
        out = torch.empty(batch, rows, dtype=torch.float32, device=w.device)
    lib = _lib.load()
    code = lib.pyrite_dev_matvec(type_id, w.data_ptr(), w.numel(), rows, cols, x2.data_ptr(), x2.stride(0),
                                 out.data_ptr(), out.stride(0), batch, _stream_ptr(w.device))
    _lib.check(code, "pyrite_dev_matvec")
    return out.reshape(rows) if squeeze else out


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
