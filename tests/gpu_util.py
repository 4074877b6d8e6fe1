"""Helpers shared by the GPU parity tests (imported only by tests marked gpu)."""
from __future__ import annotations

import sys

import numpy as np

# Sizes and seeds named by every parity case, printed before the GPU step so a
# failing run identifies its case from the log alone.


def announce(*parts) -> None:
    print("[gpu-case]", *parts, file=sys.stderr, flush=True)


def f64_bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    """Bit equality with all NaNs treated as equal (payload/sign of NaN differ by platform)."""
    a = np.ascontiguousarray(a, dtype=np.float64)
    b = np.ascontiguousarray(b, dtype=np.float64)
    na, nb = np.isnan(a), np.isnan(b)
    if not np.array_equal(na, nb):
        return False
    return np.array_equal(a[~na].view(np.uint64), b[~nb].view(np.uint64))


def f32_bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    if not np.array_equal(na, nb):
        return False
    return np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def matvec_tolerance(x: np.ndarray, row_maxabs: np.ndarray) -> np.ndarray:
    """The parity bound for fp32 accumulation: 1e-4 * ||x||_2 * max|row| (per row)."""
    return 1e-4 * float(np.linalg.norm(np.asarray(x, dtype=np.float64))) * np.asarray(row_maxabs, dtype=np.float64)


def assert_matvec_close(got, ref, x, row_maxabs, what: str = "") -> None:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    tol = matvec_tolerance(x, row_maxabs)
    finite = np.isfinite(ref)
    err = np.abs(got - ref)
    bad = finite & ~(err <= tol)
    assert not bad.any(), (
        f"{what}: {int(bad.sum())} rows outside 1e-4*||x||*max|row|; worst row {int(np.argmax(np.where(finite, err - tol, -np.inf)))} "
        f"err {float(np.max(np.where(finite, err, 0)))}")
    assert np.array_equal(np.isnan(got[~finite]), np.isnan(ref[~finite]))
