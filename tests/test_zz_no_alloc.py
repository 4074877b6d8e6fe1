"""pyrite_dev_lm_head_argmax_noalloc (the LM head over a fixed device scratch
array, no allocation) against pyrite_dev_lm_head_argmax through the C ABI.

Two calls in a row, the second on a smaller input, each compared bit for bit
(logits) and exactly (ids) with the allocating entry point on the same inputs;
a graph captured around the allocation-free call replays to the same results
with eager work between the replays; inputs beyond the scratch's limits are
refused with -2 before anything is launched.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from tests.gpu_util import announce

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from pyrite_amd import _lib
    return _lib.load()


def _payload(rng, t, rows, cols):
    """Random block bytes with finite, moderate fp16 block scales."""
    bpb = {12: 144, 14: 210}[t]
    raw = rng.integers(0, 256, size=rows * (cols // 256) * bpb, dtype=np.uint8).reshape(-1, bpb)
    for off in {12: (0, 2), 14: (208,)}[t]:
        raw[:, off + 1] &= 0x3B
    return raw.reshape(-1)


def _call(lib, fn, t, w, rows, cols, x, logits, ids):
    stream = torch.cuda.current_stream().cuda_stream
    return getattr(lib, fn)(t, w.data_ptr(), w.numel(), rows, cols, x.data_ptr(), x.stride(0),
                            logits.data_ptr(), logits.stride(0), ids.data_ptr(), x.shape[0], stream)


def _both(lib, t, w, rows, cols, x):
    dev = x.device
    out = {}
    for fn in ("pyrite_dev_lm_head_argmax", "pyrite_dev_lm_head_argmax_noalloc"):
        logits = torch.full((x.shape[0], rows), float("nan"), device=dev)
        ids = torch.full((x.shape[0],), -7, dtype=torch.int32, device=dev)
        rc = _call(lib, fn, t, w, rows, cols, x, logits, ids)
        assert rc == 0, f"{fn}: {rc} {lib.pyrite_hip_last_error()}"
        torch.cuda.synchronize()
        out[fn] = (logits.cpu(), ids.cpu())
    return out


def test_noalloc_equals_allocating_entry_point(lib, orc):
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(7001)
    # 1: a 151936-row Q6_K vocabulary, 8 vectors (the scratch's largest batch)
    rows, cols, batch = 151936, 1024, 8
    w = torch.from_numpy(_payload(rng, 14, rows, cols)).to(dev)
    x = torch.from_numpy(np.stack([orc.normal(7100 + b, cols) for b in range(batch)])).to(dev)
    announce("noalloc lm head", "Q6_K", rows, cols, batch)
    r = _both(lib, 14, w, rows, cols, x)
    (la, ia), (lb, ib) = r["pyrite_dev_lm_head_argmax"], r["pyrite_dev_lm_head_argmax_noalloc"]
    assert torch.equal(la.view(torch.int32), lb.view(torch.int32)) and torch.equal(ia, ib)
    # 2: smaller: 30000 Q4_K rows, 2 vectors; ids also against the oracle
    rows2, cols2, batch2 = 30000, 512, 2
    p2 = orc.quantize(12, orc.normal(7200, rows2 * cols2, 0.0, 0.02).astype(np.float64))
    w2 = torch.from_numpy(p2).to(dev)
    xs2 = np.stack([orc.normal(7300 + b, cols2) for b in range(batch2)])
    x2 = torch.from_numpy(xs2).to(dev)
    announce("noalloc lm head", "Q4_K", rows2, cols2, batch2)
    r = _both(lib, 12, w2, rows2, cols2, x2)
    (la, ia), (lb, ib) = r["pyrite_dev_lm_head_argmax"], r["pyrite_dev_lm_head_argmax_noalloc"]
    assert torch.equal(la.view(torch.int32), lb.view(torch.int32)) and torch.equal(ia, ib)
    for b in range(batch2):
        ref = orc.matvec(12, p2, xs2[b].astype(np.float64), rows2, cols2)
        assert int(ib[b]) == orc.argmax_first(ref)


def test_noalloc_graph_replays(lib, orc):
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(7400)
    rows, cols = 20000, 1024
    w = torch.from_numpy(_payload(rng, 14, rows, cols)).to(dev)
    x = torch.from_numpy(np.stack([orc.normal(7500 + b, cols) for b in range(3)])).to(dev)
    xe = torch.from_numpy(np.stack([orc.normal(7600 + b, cols) for b in range(5)])).to(dev)
    announce("noalloc lm head", "graph", rows, cols, 3)
    ref = _both(lib, 14, w, rows, cols, x)["pyrite_dev_lm_head_argmax"]
    refe = _both(lib, 14, w, rows, cols, xe)["pyrite_dev_lm_head_argmax"]
    logits = torch.empty(3, rows, device=dev)
    ids = torch.empty(3, dtype=torch.int32, device=dev)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        rc = _call(lib, "pyrite_dev_lm_head_argmax_noalloc", 14, w, rows, cols, x, logits, ids)
    assert rc == 0
    le = torch.empty(5, rows, device=dev)
    ie = torch.empty(5, dtype=torch.int32, device=dev)
    for _ in range(3):
        logits.fill_(float("nan"))
        ids.fill_(-7)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(logits.cpu().view(torch.int32), ref[0].view(torch.int32))
        assert torch.equal(ids.cpu(), ref[1])
        # eager allocation-free work on the same scratch between the replays
        assert _call(lib, "pyrite_dev_lm_head_argmax_noalloc", 14, w, rows, cols, xe, le, ie) == 0
        torch.cuda.synchronize()
        assert torch.equal(ie.cpu(), refe[1])


def test_noalloc_limits(lib, orc):
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(7700)
    rows, cols = 256, 256
    w = torch.from_numpy(_payload(rng, 14, rows, cols)).to(dev)
    announce("noalloc lm head", "limits")
    x9 = torch.ones(9, cols, device=dev)
    l9 = torch.empty(9, rows, device=dev)
    i9 = torch.empty(9, dtype=torch.int32, device=dev)
    assert _call(lib, "pyrite_dev_lm_head_argmax_noalloc", 14, w, rows, cols, x9, l9, i9) == -2
    assert b"at most 8 vectors" in lib.pyrite_hip_last_error()
    # a leading dimension that would put the last vector's bounds past the scratch
    x2 = torch.ones(2, cols, device=dev)
    wide = torch.empty(2, 1894336, device=dev)
    i2 = torch.empty(2, dtype=torch.int32, device=dev)
    assert _call(lib, "pyrite_dev_lm_head_argmax_noalloc", 14, w, rows, cols, x2, wide, i2) == -2
    torch.cuda.synchronize()
