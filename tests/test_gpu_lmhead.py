"""GPU parity of the LM head (fp32 logits + exact greedy id) and of RMSNorm.

The reference path is pyrite/executor.py:852-875 (logits via pyrite_matvec in
fp64, pyrite/kernels/native.c:518-555) followed by Sampler.greedy
(pyrite/sampler.py:12-15): the first index of the maximum.  The oracle
restates both (oracle_matvec, oracle_argmax_first); ids must be identical and
logits within the matvec tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest

from tests.gpu_util import announce, assert_matvec_close

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from pyrite_amd import _lib
    _lib.load()  # fail loudly when the HIP library is missing
    return torch.device("cuda:0")


def _row_maxabs(orc, t, payload, rows, cols):
    return np.abs(orc.dequantize_rows(t, payload, rows, cols).reshape(rows, cols)).max(axis=1)


def _random_q(rng, t, rows, cols):
    from tests.gpu_util import random_payload
    return random_payload(rng, t, rows, cols)


def _quantized(orc, t, rows, cols, seed):
    from pyrite_amd.quantize import quantize
    w = orc.normal(seed, rows * cols, 0.0, 0.02).astype(np.float64)
    return quantize(t, w)


def _check(orc, dev, t, payload, rows, cols, xs, what):
    from pyrite_amd import device
    w = torch.from_numpy(payload).to(dev)
    x = torch.from_numpy(np.ascontiguousarray(xs, dtype=np.float32)).to(dev)
    announce("lm_head", what, f"type={t}", f"{rows}x{cols}", f"batch={xs.shape[0]}")
    logits, ids = device.lm_head_argmax(t, w, x, rows, cols)
    torch.cuda.synchronize()
    logits = logits.cpu().numpy()
    ids = ids.cpu().numpy()
    maxabs = None
    for b in range(xs.shape[0]):
        ref = orc.matvec(t, payload, xs[b].astype(np.float64), rows, cols)
        want = orc.argmax_first(ref)
        assert int(ids[b]) == want, f"{what} b={b}: id {int(ids[b])} != reference {want}"
        if np.isfinite(ref).all():
            if maxabs is None:
                maxabs = _row_maxabs(orc, t, payload, rows, cols)
            assert_matvec_close(logits[b], ref, xs[b], maxabs, f"{what} b={b}")
    return ids


@pytest.mark.parametrize("t", [14, 8, 12, 13, 2, 23, 11, 10, 3, 7, 20])
def test_lm_head_random_types(orc, dev, t):
    rng = np.random.default_rng(100 + t)
    rows, cols = 3000, 1024
    payload = _random_q(rng, t, rows, cols)
    xs = np.stack([orc.normal(7000 + t + 10 * b, cols) for b in range(3)])
    _check(orc, dev, t, payload, rows, cols, xs, "random")


@pytest.mark.parametrize("t", [14, 8, 12, 13, 2, 23, 11, 10, 3, 7, 20])
def test_lm_head_random_types_one_vector(orc, dev, t):
    """One vector: the argmax is decided inside the bound matvec (its own kernel)."""
    rng = np.random.default_rng(200 + t)
    rows, cols = 5000, 1024
    payload = _random_q(rng, t, rows, cols)
    x = orc.normal(7100 + t, cols)
    _check(orc, dev, t, payload, rows, cols, x[None, :], "random one vector")


@pytest.mark.parametrize("t", [0, 1, 30, 24])
def test_lm_head_plain_types(orc, dev, t):
    """Float and integer heads from seeded N(0, 0.02) weights (x 100 for I8)."""
    rows, cols = 2000, 512
    from pyrite_amd.quantize import quantize
    w = orc.normal(8000 + t, rows * cols, 0.0, 0.02).astype(np.float64) * (100.0 if t == 24 else 1.0)
    payload = quantize(t, w)
    xs = np.stack([orc.normal(8100 + t + b, cols) for b in range(2)])
    _check(orc, dev, t, payload, rows, cols, xs, "plain")


def test_lm_head_quantized_q6k(orc, dev):
    rows, cols = 8192, 1024
    payload = _quantized(orc, 14, rows, cols, 20243000)
    x = orc.normal(20243100, cols).astype(np.float64)
    x = (x / np.sqrt(np.mean(x * x) + 1e-6)).astype(np.float32)
    xs = np.stack([x, orc.normal(20243101, cols)])
    _check(orc, dev, 14, payload, rows, cols, xs, "quantized")


def _row(payload, r, rb):
    return payload[r * rb:(r + 1) * rb]


def test_lm_head_exact_ties_pick_first(orc, dev):
    """Duplicate the winning row earlier in the matrix: equal fp64 logits, the first index wins."""
    rng = np.random.default_rng(5)
    t, rows, cols = 14, 4096, 1024
    rb = cols // 256 * 210
    payload = _random_q(rng, t, rows, cols)
    x = orc.normal(31, cols)
    win = orc.argmax_first(orc.matvec(t, payload, x.astype(np.float64), rows, cols))
    for dst in (0, 777, 2000, rows - 1):
        if dst == win:
            continue
        p = payload.copy()
        p[dst * rb:(dst + 1) * rb] = _row(payload, win, rb)
        ids = _check(orc, dev, t, p, rows, cols, x[None, :], f"tie dst={dst}")
        assert int(ids[0]) == min(dst, win)


def test_lm_head_near_ties_need_recompute(orc, dev):
    """Copies of the winning row with one code changed by one step: logits differ by
    about one weight quantum times one activation, near fp32 rounding noise."""
    rng = np.random.default_rng(9)
    t, rows, cols = 8, 4096, 1024
    rb = cols // 32 * 34
    payload = _random_q(rng, t, rows, cols)
    x = orc.normal(41, cols)
    x[5] = np.float32(1e-6)  # a tiny activation: changing its weight moves the logit a hair
    win = orc.argmax_first(orc.matvec(t, payload, x.astype(np.float64), rows, cols))
    p = payload.copy()
    for k, dst in enumerate((10, 500, 3000)):
        if dst == win:
            continue
        p[dst * rb:(dst + 1) * rb] = _row(payload, win, rb)
        q = int(p[dst * rb + 2 + 5])  # block 0, code of column 5
        p[dst * rb + 2 + 5] = (q + (1 if k % 2 == 0 else 255)) % 256
    _check(orc, dev, t, p, rows, cols, x[None, :], "near-tie")


def test_lm_head_many_candidates(orc, dev):
    """600 copies of the winner (more than the deciding workgroup lists) and one
    workgroup range full of them (more than a workgroup lists)."""
    rng = np.random.default_rng(11)
    t, rows, cols = 8, 4096, 256
    rb = cols // 32 * 34
    payload = _random_q(rng, t, rows, cols)
    x = orc.normal(51, cols)
    win = orc.argmax_first(orc.matvec(t, payload, x.astype(np.float64), rows, cols))
    p = payload.copy()
    for dst in list(range(100, 700)):
        p[dst * rb:(dst + 1) * rb] = _row(payload, win, rb)
    ids = _check(orc, dev, t, p, rows, cols, x[None, :], "many")
    assert int(ids[0]) == min(100, win)


def test_lm_head_zero_activations(orc, dev):
    rng = np.random.default_rng(13)
    t, rows, cols = 14, 2048, 512
    payload = _random_q(rng, t, rows, cols)
    xs = np.zeros((2, cols), dtype=np.float32)
    ids = _check(orc, dev, t, payload, rows, cols, xs, "zero-x")
    assert list(ids) == [0, 0]
    ids = _check(orc, dev, t, payload, rows, cols, xs[:1], "zero-x one vector")
    assert list(ids) == [0]


def test_lm_head_nonfinite_activation(orc, dev):
    """An infinite activation: every path falls back to the reference's own max() scan."""
    rng = np.random.default_rng(17)
    t, rows, cols = 8, 256, 64
    payload = _random_q(rng, t, rows, cols)
    x = orc.normal(61, cols)
    x[3] = np.float32(np.inf)
    _check(orc, dev, t, payload, rows, cols, x[None, :], "inf-x")


def test_lm_head_full_vocab_151936(orc, dev):
    """The Qwen3 LM-head shape: Q6_K 151936 x 1024, RMS-normalised N(0, 1) input."""
    t, rows, cols = 14, 151936, 1024
    rng = np.random.default_rng(20243)
    bpb = 210
    raw = rng.integers(0, 256, size=rows * (cols // 256) * bpb, dtype=np.uint8).reshape(-1, bpb)
    # finite, moderate d (fp16 at bytes 208..209): exponent below 0x3C
    raw[:, 209] &= 0x3B
    payload = raw.reshape(-1)
    x = orc.normal(20243200, cols).astype(np.float64)
    x = (x / np.sqrt(np.mean(x * x) + 1e-6)).astype(np.float32)
    _check(orc, dev, t, payload, rows, cols, x[None, :], "vocab 151936")


@pytest.mark.parametrize("n,batch", [(1024, 1), (2048, 3), (1000, 2)])
def test_rms_norm(orc, dev, n, batch):
    from pyrite_amd import device
    xs = np.stack([orc.normal(900 + n + b, n, 0.0, 3.0) for b in range(batch)])
    wt = orc.normal(950 + n, n, 1.0, 0.1)
    announce("rms_norm", f"n={n}", f"batch={batch}")
    for w in (None, wt):
        got = device.rms_norm(torch.from_numpy(xs).to(dev), None if w is None else torch.from_numpy(w).to(dev),
                              eps=1e-6).cpu().numpy()
        for b in range(batch):
            ref = orc.rms_norm(xs[b].astype(np.float64), None if w is None else w.astype(np.float64), 1e-6)
            ref32 = ref.astype(np.float32)
            # fp64 inside, one rounding to fp32: equal to the reference rounded, or one ulp away
            # when the tree-ordered sum of squares moves the fp64 value across a rounding boundary
            ulps = np.abs(got[b].view(np.int32).astype(np.int64) - ref32.view(np.int32).astype(np.int64))
            assert ulps.max() <= 1, f"n={n} b={b}: {ulps.max()} ulp"
            assert np.mean(ulps == 0) > 0.99
