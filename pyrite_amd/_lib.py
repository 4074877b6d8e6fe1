"""Loader for libpyrite_hip.so (the HIP kernels behind include/pyrite_hip.h).

The library is built in-tree by ``python -m pyrite_amd.build``.  There is no
CPU fallback: when the library is missing every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("PYRITE_HIP_LIB", Path(__file__).resolve().parent / "libpyrite_hip.so"))

_c = ctypes
_sz = _c.c_size_t
_vp = _c.c_void_p
_dp = _c.POINTER(_c.c_double)

#: (name, restype, argtypes) for every symbol of include/pyrite_hip.h
SIGNATURES: list[tuple[str, object, tuple]] = [
    ("pyrite_native_types", _c.c_int, (_c.POINTER(_c.c_int), _sz)),
    ("pyrite_matvec", _c.c_int, (_c.c_int, _vp, _sz, _dp, _dp, _sz, _sz)),
    ("pyrite_dequantize_rows", _c.c_int, (_c.c_int, _vp, _sz, _dp, _sz, _sz)),
    ("pyrite_hip_last_error", _c.c_char_p, ()),
    ("pyrite_dev_matvec", _c.c_int, (_c.c_int, _vp, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _sz, _vp)),
    ("pyrite_dev_matvec_grouped", _c.c_int, (_c.c_int, _vp, _sz, _sz, _vp)),
    ("pyrite_dev_matvec_grouped_timed", _c.c_int, (_c.c_int, _vp, _sz, _sz, _vp, _vp, _vp)),
    ("pyrite_dev_dequantize", _c.c_int, (_c.c_int, _vp, _sz, _sz, _sz, _vp, _c.c_int, _vp)),
    ("pyrite_dev_lm_head_argmax", _c.c_int, (_c.c_int, _vp, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp)),
    ("pyrite_dev_lm_head_argmax_noalloc", _c.c_int,
     (_c.c_int, _vp, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp)),
    ("pyrite_dev_moe_ffn", _c.c_int, (_vp, _vp, _sz, _vp, _sz, _vp, _vp, _sz, _vp)),
    ("pyrite_dev_rms_norm", _c.c_int, (_vp, _sz, _vp, _sz, _c.c_double, _vp, _sz, _sz, _vp)),
    ("pyrite_dev_add_rms_norm", _c.c_int,
     (_vp, _sz, _vp, _sz, _vp, _sz, _c.c_double, _vp, _sz, _vp, _sz, _sz, _vp)),
    ("pyrite_dev_matvec_swiglu", _c.c_int, (_c.c_int, _vp, _sz, _sz, _sz, _vp, _vp, _sz, _vp, _sz, _sz, _vp)),
    ("pyrite_dev_attention_decode", _c.c_int, (_vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp, _vp)),
]

_LIB: ctypes.CDLL | None = None
_ERROR: str | None = None


def load() -> ctypes.CDLL:
    """Load and declare the library; raise RuntimeError when it is unavailable."""
    global _LIB, _ERROR
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.is_file():
        _ERROR = f"{LIB_PATH} is not built (run `python -m pyrite_amd.build`)"
        raise RuntimeError(_ERROR)
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, restype, argtypes in SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _LIB = lib
    return lib


def last_error() -> str:
    lib = load()
    msg = lib.pyrite_hip_last_error()
    return msg.decode() if msg else ""


class KernelError(ValueError):
    """A nonzero return code from the C ABI."""

    def __init__(self, code: int, operation: str):
        detail = ""
        if code == -4:
            detail = f": {last_error()}"
        super().__init__(f"{operation} rejected the matrix buffer/shape (error {code}){detail}")
        self.code = code


def check(code: int, operation: str) -> None:
    if code != 0:
        raise KernelError(code, operation)
