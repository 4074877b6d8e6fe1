"""The C-ABI library loads, exports every symbol include/pyrite_hip.h declares,
and validates arguments with the reference's codes (pyrite/kernels/native.c:496-525,
562-566) before touching a device.  No kernel is launched here."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER_DIR = ROOT / "include"


def _declared_functions() -> list[str]:
    names = []
    for header in HEADER_DIR.glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names += re.findall(r"\b(pyrite_\w+)\s*\(", text)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    from pyrite_amd import _lib

    if not _lib.LIB_PATH.is_file():
        from pyrite_amd.build import build

        build()
    return _lib.load()


def test_every_declared_symbol_is_exported(lib):
    names = _declared_functions()
    assert {"pyrite_native_types", "pyrite_matvec", "pyrite_dequantize_rows"} <= set(names)
    for name in names:
        assert hasattr(lib, name), name


def test_bindings_cover_the_header():
    from pyrite_amd import _lib

    assert sorted(n for n, _, _ in _lib.SIGNATURES) == _declared_functions()


def test_native_type_table_matches_reference_order(lib):
    n = lib.pyrite_native_types(None, 0)
    assert n == 21
    buf = (ctypes.c_int * 21)()
    assert lib.pyrite_native_types(buf, 21) == 21
    assert list(buf) == [0, 1, 2, 3, 6, 7, 8, 9, 10, 11, 12, 13, 14, 20, 23, 24, 25, 26, 27, 28, 30]
    small = (ctypes.c_int * 3)()
    assert lib.pyrite_native_types(small, 3) == 3 and list(small) == [0, 1, 2]


def test_python_mirror_surface():
    from pyrite_amd import native

    for name in ("NATIVE_TYPES", "native_available", "supports_native", "native_type_ids",
                 "sorted_native_types", "matvec", "dequantize_rows"):
        assert hasattr(native, name)
    assert native.NATIVE_TYPES == frozenset(native.native_type_ids())
    assert native.supports_native(21) is False and native.supports_native(35) is False
    assert "Q4_K" in native.sorted_native_types()


def _dp(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


def test_validation_codes_match_the_reference(lib):
    rows, cols = 2, 256
    data = np.zeros(2 * 144, np.uint8)
    x = np.zeros(cols)
    out = np.zeros(rows)
    mv = lib.pyrite_matvec
    assert mv(99, data.ctypes.data, data.nbytes, _dp(x), _dp(out), rows, cols) == -1
    assert mv(12, data.ctypes.data, data.nbytes, _dp(x), _dp(out), 0, cols) == -2
    assert mv(12, data.ctypes.data, data.nbytes, _dp(x), _dp(out), rows, 0) == -2
    assert mv(12, data.ctypes.data, data.nbytes, _dp(x), _dp(out), rows, 100) == -2
    assert mv(12, data.ctypes.data, data.nbytes - 1, _dp(x), _dp(out), rows, cols) == -3
    assert mv(12, None, data.nbytes, _dp(x), _dp(out), rows, cols) == -3
    assert mv(12, data.ctypes.data, data.nbytes, None, _dp(out), rows, cols) == -3
    assert mv(12, data.ctypes.data, data.nbytes, _dp(x), None, rows, cols) == -3
    dq = lib.pyrite_dequantize_rows
    big = np.zeros(rows * cols)
    assert dq(99, data.ctypes.data, data.nbytes, _dp(big), rows, cols) == -1
    assert dq(12, data.ctypes.data, data.nbytes, _dp(big), 0, cols) == -2
    assert dq(12, data.ctypes.data, data.nbytes + 1, _dp(big), rows, cols) == -3
    assert dq(12, data.ctypes.data, data.nbytes, None, rows, cols) == -3
    dev = lib.pyrite_dev_matvec
    assert dev(99, 1, 10, 1, 32, 16, 32, 16, 1, 1, None) == -1
    assert dev(12, 16, 144, 1, 100, 16, 100, 16, 1, 1, None) == -2
    assert dev(12, 16, 143, 1, 256, 16, 256, 16, 1, 1, None) == -3
    assert dev(12, 16, 144, 1, 256, 18, 256, 16, 1, 1, None) == -3  # x not 16-byte aligned
    assert dev(12, 16, 144, 1, 256, 16, 256, 16, 1, 0, None) == -2  # empty batch


def test_mirror_raises_like_the_reference():
    from pyrite_amd import native

    with pytest.raises(ValueError):
        native.matvec(21, b"", [0.0], 1, 1)
    with pytest.raises(ValueError):
        native.matvec(12, bytes(144), [0.0] * 10, 1, 256)
    with pytest.raises(ValueError):
        native.dequantize_rows(12, bytes(144), 0, 256)
