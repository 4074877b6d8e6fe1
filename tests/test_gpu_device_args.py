"""Argument checks of the device entry points and workspace growth around graphs.

pyrite_amd.device refuses activations and outputs that the kernels could not
use (a host tensor, another dtype, a short output, overlapping or non-contiguous
rows) with ValueError before anything is launched.  The per-device workspaces
grow on demand; a block they replace stays allocated, so a HIP graph captured
before the growth still replays correctly, and growth during a capture is
refused with an error instead of allocating.
"""
from __future__ import annotations

import numpy as np
import pytest

from tests.gpu_util import announce

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from pyrite_amd import _lib
    _lib.load()
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def q4k(orc, dev):
    rows, cols = 64, 512
    payload = orc.quantize(12, orc.normal(31, rows * cols, 0.0, 0.02).astype(np.float64))
    return torch.from_numpy(payload).to(dev), rows, cols


def test_matvec_refuses_bad_activations(q4k, dev):
    from pyrite_amd import device
    w, rows, cols = q4k
    announce("device args", "matvec activations")
    with pytest.raises(ValueError, match="CUDA tensor"):
        device.matvec(12, w, torch.ones(cols), rows, cols)                      # host x
    with pytest.raises(ValueError, match="fp32"):
        device.matvec(12, w, torch.ones(cols, dtype=torch.float16, device=dev), rows, cols)
    with pytest.raises(ValueError, match="fp32"):
        device.matvec(12, w, torch.ones(2, cols + 32, device=dev), rows, cols)  # wrong width
    with pytest.raises(ValueError, match="contiguous"):
        device.matvec(12, w, torch.ones(cols, 2, device=dev).t(), rows, cols)   # strided rows


def test_matvec_refuses_bad_outputs(q4k, dev):
    from pyrite_amd import device
    w, rows, cols = q4k
    x = torch.ones(2, cols, device=dev)
    announce("device args", "matvec outputs")
    with pytest.raises(ValueError):
        device.matvec(12, w, x, rows, cols, out=torch.empty(2, rows))                      # host out
    with pytest.raises(ValueError, match="fp32"):
        device.matvec(12, w, x, rows, cols, out=torch.empty(2, rows, dtype=torch.float16, device=dev))
    with pytest.raises(ValueError):
        device.matvec(12, w, x, rows, cols, out=torch.empty(1, rows, device=dev))          # short batch
    with pytest.raises(ValueError):
        device.matvec(12, w, x, rows, cols, out=torch.empty(2, rows - 1, device=dev))      # short rows
    with pytest.raises(ValueError):
        device.matvec(12, w, x, rows, cols, out=torch.empty(rows, 2, device=dev).t())      # strided rows
    with pytest.raises(ValueError):
        device.matvec(12, w, x, rows, cols, out=torch.empty(rows, device=dev).expand(2, rows))  # overlapping
    with pytest.raises(ValueError):
        device.lm_head_argmax(12, w, x, rows, cols, logits=torch.empty(2, rows, dtype=torch.float64, device=dev))


def test_matvec_outputs_land_in_the_callers_tensor(q4k, dev, orc):
    """1-D outputs at batch 1, padded rows and grouped outputs are written in
    place (no hidden copies)."""
    from pyrite_amd import device
    w, rows, cols = q4k
    x = torch.from_numpy(orc.normal(32, 2 * cols)).to(dev).reshape(2, cols)
    announce("device args", "in-place outputs")
    ref = device.matvec(12, w, x, rows, cols)
    # batch 1 has a kernel of its own (another summation order than batch 2)
    ref1 = device.matvec(12, w, x[:1], rows, cols)
    y1 = torch.zeros(rows, device=dev)
    device.matvec(12, w, x[0], rows, cols, out=y1)
    assert torch.equal(y1, ref1[0])
    padded = torch.zeros(2, rows + 8, device=dev)
    device.matvec(12, w, x, rows, cols, out=padded[:, :rows])
    assert torch.equal(padded[:, :rows], ref) and not padded[:, rows:].any()
    outs = [torch.zeros(2, rows, device=dev), torch.zeros(2, rows + 8, device=dev)[:, :rows]]
    device.matvec_grouped(12, [(w, rows, cols), (w, rows, cols)], x, outs=outs)
    assert torch.equal(outs[0], ref) and torch.equal(outs[1], ref)
    with pytest.raises(ValueError):
        device.matvec_grouped(12, [(w, rows, cols)], x, outs=[torch.zeros(rows, 2, device=dev).t()])
    with pytest.raises(ValueError):
        device.matvec_grouped(12, [(w, rows, cols)], x.cpu())


def test_lm_head_graph_survives_workspace_growth(orc, dev):
    """A graph captured at batch 1 keeps working after an eager call at a
    larger batch has grown the LM-head workspace (the old block is retained),
    and a capture that would need a larger workspace is refused."""
    from pyrite_amd import device
    rows, cols = 5000, 512
    payload = orc.quantize(14, orc.normal(41, rows * cols, 0.0, 0.02).astype(np.float64))
    w = torch.from_numpy(payload).to(dev)
    x1 = torch.from_numpy(orc.normal(42, cols)).to(dev).reshape(1, cols)
    announce("workspace", "lm head graph across growth", rows, cols)
    logits0, ids0 = device.lm_head_argmax(14, w, x1, rows, cols)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    logits = torch.empty(1, rows, device=dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        _, ids = device.lm_head_argmax(14, w, x1, rows, cols, logits=logits)
    xb = torch.from_numpy(orc.normal(43, 24 * cols)).to(dev).reshape(24, cols)
    lb, idb = device.lm_head_argmax(14, w, xb, rows, cols)  # grows the workspace
    torch.cuda.synchronize()
    for _ in range(3):
        logits.zero_()
        ids.fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(logits, logits0) and torch.equal(ids, ids0)
        assert torch.equal(device.lm_head_argmax(14, w, xb, rows, cols)[1], idb)
    big = torch.from_numpy(orc.normal(44, 200 * cols)).to(dev).reshape(200, cols)
    g2 = torch.cuda.CUDAGraph()
    with pytest.raises(ValueError, match="capture"):
        with torch.cuda.graph(g2, stream=s):
            device.lm_head_argmax(14, w, big, rows, cols)
    torch.cuda.synchronize()
    assert torch.equal(device.lm_head_argmax(14, w, x1, rows, cols)[1], ids0)


def test_moe_graph_survives_workspace_growth(orc, dev):
    """The same for the MoE layer's workspace: a batch-1 graph, then an eager
    batch of 64 tokens, then replays."""
    from tests.test_gpu_moe import _layer
    from pyrite_amd import device
    rng = np.random.default_rng(45)
    layer, _ = _layer(orc, rng, 16, 256, 256, 4, seed=46)
    x1 = torch.from_numpy(orc.normal(47, 256)).to(dev).reshape(1, 256)
    announce("workspace", "moe graph across growth")
    out0, ids0, _ = device.moe_ffn(layer, x1)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    out = torch.empty_like(out0)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        device.moe_ffn(layer, x1, out=out)
    x64 = torch.from_numpy(orc.normal(48, 64 * 256)).to(dev).reshape(64, 256)
    out64 = device.moe_ffn(layer, x64)[0].clone()
    torch.cuda.synchronize()
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, out0)
        assert torch.equal(device.moe_ffn(layer, x64)[0], out64)
