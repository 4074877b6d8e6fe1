"""Helpers shared by the parity tests and the fixture script (no GPU, no torch here)."""
from __future__ import annotations

import sys

import numpy as np

from oracle.oracle import TYPES, finite_bf16words, finite_halfwords

# byte offsets of fp16 words inside one block (scale, min, sum words)
HALF_WORDS = {1: (0,), 2: (0,), 3: (0, 2), 6: (0,), 7: (0, 2), 8: (0,), 9: (0, 2),
              10: (80, 82), 11: (108,), 12: (0, 2), 13: (0, 2), 14: (208,), 20: (0,),
              23: (0,), 30: (0,)}


def random_payload(rng, type_id: int, rows: int, cols: int) -> np.ndarray:
    """Random block bytes (every code, scale and bit pattern) with the fp16 words
    that scale a block kept finite, so that outputs are comparable numbers."""
    _, bs, bpb = TYPES[type_id]
    if type_id == 0:
        return rng.standard_normal(rows * cols).astype("<f4").view(np.uint8).copy()
    if type_id == 28:
        return rng.standard_normal(rows * cols).astype("<f8").view(np.uint8).copy()
    raw = rng.integers(0, 256, size=rows * (cols // bs) * bpb, dtype=np.uint8)
    if type_id == 30:
        return finite_bf16words(raw)
    if type_id == 1:
        return finite_halfwords(raw)
    for blk in range(raw.size // bpb):
        for off in HALF_WORDS.get(type_id, ()):
            w = int(raw[blk * bpb + off]) | (int(raw[blk * bpb + off + 1]) << 8)
            if (w & 0x7C00) == 0x7C00:
                raw[blk * bpb + off + 1] &= 0x3B
    return raw


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
