"""The device's exp (pyrite_amd/csrc/libm_exp.h) equals the host libm's exp.

The MoE routing order depends on exact fp64 probabilities exp(l - peak) / total
(pyrite/tensor_ops.py:513-521, where exp is Python's math.exp, the host libm's).
libm_exp.h restates glibc's table-driven exp; it is plain C++ apart from the
__host__/__device__ markers, so this test compiles it for the host with g++ and
compares it bit for bit with the libm exp and with math.exp over millions of
arguments spread over the routing range (l - peak <= 0), the subnormal range,
tiny arguments, large positive arguments and the special values.
"""
from __future__ import annotations

import ctypes
import math
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "pyrite_amd" / "csrc" / "libm_exp.h"

SRC = r"""
#include <cmath>
#include "libm_exp.h"
extern "C" void both(const double* x, double* mine, double* libm, long n) {
    for (long i = 0; i < n; ++i) { mine[i] = pyrite::libm_exp(x[i]); libm[i] = std::exp(x[i]); }
}
"""


@pytest.fixture(scope="module")
def lib(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    d = tmp_path_factory.mktemp("libm_exp")
    (d / "t.cpp").write_text(SRC)
    so = d / "t.so"
    # -ffp-contract=off: only the fma() calls of the header fuse, as on the device
    subprocess.run([gxx, "-O2", "-std=c++17", "-ffp-contract=off", "-Wno-unknown-pragmas", "-D__host__=",
                    "-D__device__=", "-fPIC", "-shared", "-I", str(HEADER.parent), str(d / "t.cpp"), "-o",
                    str(so)], check=True)
    h = ctypes.CDLL(str(so))
    dp = ctypes.POINTER(ctypes.c_double)
    h.both.argtypes = (dp, dp, dp, ctypes.c_long)
    return h


def _run(lib, x):
    x = np.ascontiguousarray(x, dtype=np.float64)
    mine, libm = np.empty_like(x), np.empty_like(x)
    dp = ctypes.POINTER(ctypes.c_double)
    lib.both(x.ctypes.data_as(dp), mine.ctypes.data_as(dp), libm.ctypes.data_as(dp), x.size)
    return mine, libm


def _args(n, seed):
    rng = np.random.default_rng(seed)
    u = rng.random(n)
    parts = [
        -u[0::6] * 50.0,                 # softmax arguments of ordinary routers
        -u[1::6],                        # near the peak
        -u[2::6] * 745.5,                # down to the subnormal and zero results
        -(512.0 + u[3::6] * 234.0),      # the scaled branch for large |x|
        (u[4::6] - 0.5) * 1e-10,         # tiny arguments
        (u[5::6] - 0.5) * 1420.0,        # overflow to inf and underflow to 0
    ]
    return np.concatenate(parts)


def test_libm_exp_equals_host_exp(lib):
    x = np.concatenate([_args(3_000_000, 20261202),
                        np.array([0.0, -0.0, 1.0, -1.0, 709.78, 709.79, -708.39, -708.4, -745.13, -745.14,
                                  -745.2, 2.0 ** -54, -(2.0 ** -54), 2.0 ** -55, 512.0, -512.0, 1024.0,
                                  -1024.0, np.inf, -np.inf, np.nan, 5e-324, -5e-324])])
    mine, libm = _run(lib, x)
    same = (mine.view(np.uint64) == libm.view(np.uint64)) | (np.isnan(mine) & np.isnan(libm))
    bad = np.flatnonzero(~same)
    assert bad.size == 0, f"{bad.size} mismatches, first x={x[bad[0]]!r}: {mine[bad[0]]!r} vs {libm[bad[0]]!r}"


def test_libm_exp_equals_math_exp(lib):
    """math.exp is what the reference calls; it is the same libm function."""
    x = _args(300_000, 7)
    mine, _ = _run(lib, x)

    def py_exp(v):
        try:
            return math.exp(v)
        except OverflowError:
            return math.inf

    ref = np.array([py_exp(v) for v in x.tolist()])
    assert np.array_equal(mine.view(np.uint64), ref.view(np.uint64))


def test_libm_exp_not_correctly_rounded_somewhere(lib):
    """The restatement is the libm's method, not a correctly rounded exp: it
    reproduces the libm's misrounded results too (a correctly rounded exp
    would differ from the libm on these arguments)."""
    from decimal import Decimal, getcontext
    from fractions import Fraction
    getcontext().prec = 50
    x = -np.random.default_rng(11).random(20000) * 20.0
    mine, libm = _run(lib, x)
    assert np.array_equal(mine.view(np.uint64), libm.view(np.uint64))
    misrounded = 0
    for v, m in zip(x.tolist(), mine.tolist()):
        f = Fraction(v)
        exact = float(Fraction((Decimal(f.numerator) / Decimal(f.denominator)).exp()))
        misrounded += exact != m
    assert misrounded > 0
