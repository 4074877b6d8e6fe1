"""GPU drop-in for the reference's native kernel module.

Same public names, argument meaning and errors as pyrite/kernels/native.py:
``NATIVE_TYPES``, ``native_available``, ``supports_native``,
``native_type_ids``, ``sorted_native_types``, ``matvec``, ``dequantize_rows``.
The entry points call libpyrite_hip.so through ctypes (pyrite_matvec /
pyrite_dequantize_rows, include/pyrite_hip.h), which run on the MI355X.

Differences from the reference, on purpose:
* there is no compile-on-first-use and no silent fallback to a Python
  decoder: without the HIP library ``native_available()`` is False and the
  entry points raise;
* ``matvec`` computes in fp64 on the GPU (the reference's double semantics,
  summed in a different order); ``dequantize_rows`` is bit-identical to the
  reference.  The fp32 device-resident path is pyrite_amd.device.
"""
from __future__ import annotations

import ctypes
from collections.abc import Sequence

import numpy as np

from . import _lib
from .ggml_types import type_name

#: GGML type ids with a GPU kernel; equal to the reference's table
#: (pyrite/kernels/native.py:31-53).
NATIVE_TYPES = frozenset({0, 1, 2, 3, 6, 7, 8, 9, 10, 11, 12, 13, 14, 20, 23, 24, 25, 26, 27, 28, 30})

_CHECKED: bool | None = None


def _library() -> ctypes.CDLL | None:
    """The loaded library when its type table matches NATIVE_TYPES, else None."""
    global _CHECKED
    try:
        lib = _lib.load()
    except (RuntimeError, OSError):
        return None
    if _CHECKED is None:
        count = lib.pyrite_native_types(None, 0)
        buf = (ctypes.c_int * max(count, 1))()
        written = lib.pyrite_native_types(buf, count)
        _CHECKED = frozenset(buf[i] for i in range(max(0, written))) == NATIVE_TYPES
    return lib if _CHECKED else None


def native_available() -> bool:
    return _library() is not None


def supports_native(ggml_type: int) -> bool:
    return ggml_type in NATIVE_TYPES and native_available()


def native_type_ids() -> tuple[int, ...]:
    lib = _library()
    if lib is None:
        return ()
    count = lib.pyrite_native_types(None, 0)
    buf = (ctypes.c_int * count)()
    written = lib.pyrite_native_types(buf, count)
    return tuple(buf[i] for i in range(max(0, written)))


def sorted_native_types() -> list[str]:
    return [type_name(t) for t in sorted(native_type_ids())]


def _bytes_view(payload) -> np.ndarray:
    """Borrow any buffer-protocol object as a uint8 array without copying."""
    return np.frombuffer(payload, dtype=np.uint8)


def matvec(ggml_type: int, payload, vector: Sequence[float], rows: int, cols: int) -> list[float]:
    """Fused quantized matrix-vector product on the GPU (pyrite/kernels/native.py:206-236)."""
    lib = _library()
    if ggml_type not in NATIVE_TYPES or lib is None:
        raise ValueError(f"no native kernel for GGML type {ggml_type}")
    if len(vector) != cols or rows <= 0 or cols <= 0:
        raise ValueError("matrix/vector shape mismatch")
    data = _bytes_view(payload)
    x = np.ascontiguousarray(vector, dtype=np.float64)
    out = np.zeros(rows, dtype=np.float64)
    dp = ctypes.POINTER(ctypes.c_double)
    code = lib.pyrite_matvec(ggml_type, data.ctypes.data, data.nbytes, x.ctypes.data_as(dp),
                             out.ctypes.data_as(dp), rows, cols)
    _lib.check(code, "native matvec")
    return out.tolist()


def dequantize_rows(ggml_type: int, payload, rows: int, cols: int) -> list[float]:
    """Dequantize a bounded row range (pyrite/kernels/native.py:239-265)."""
    lib = _library()
    if ggml_type not in NATIVE_TYPES or lib is None:
        raise ValueError(f"no native kernel for GGML type {ggml_type}")
    if rows <= 0 or cols <= 0 or rows > (1 << 62) // cols:
        raise ValueError("invalid or overflowing matrix shape")
    data = _bytes_view(payload)
    out = np.zeros(rows * cols, dtype=np.float64)
    dp = ctypes.POINTER(ctypes.c_double)
    code = lib.pyrite_dequantize_rows(ggml_type, data.ctypes.data, data.nbytes, out.ctypes.data_as(dp), rows, cols)
    _lib.check(code, "native dequantize")
    return out.tolist()
