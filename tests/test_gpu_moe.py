"""GPU parity of the Qwen3-MoE FFN layer (pyrite/executor.py:757-793, 672-683).

The oracle (oracle_moe_ffn) restates the reference's fp64 layer: router matvec,
softmax, (-p, e) ranking, top-k, renormalisation, scale, SwiGLU experts and the
weighted sum in rank order.  The expert ids must be identical; the routing
weights match to fp32 rounding; the output is within 1e-4 of its largest
magnitude (fp32 matvecs against the fp64 reference).
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


def _payload(rng, t, n_rows, cols):
    from tests.gpu_util import random_payload
    return random_payload(rng, t, n_rows, cols)


def _fast_random(rng, t, rows, cols):
    """Random block bytes with finite, moderate fp16 scales (vectorised)."""
    from oracle.oracle import TYPES
    _, bs, bpb = TYPES[t]
    raw = rng.integers(0, 256, size=rows * (cols // bs) * bpb, dtype=np.uint8).reshape(-1, bpb)
    halves = {12: (0, 2), 13: (0, 2), 14: (208,), 10: (80, 82), 11: (108,), 23: (0,), 2: (0,), 8: (0,)}[t]
    for off in halves:
        raw[:, off + 1] &= 0x3B  # exponent field below 0x1E: finite and at most ~1
    return raw.reshape(-1)


def _layer(orc, rng, E, H, I, k, types=(0, 12, 12, 14), seed=1, norm=True, scale=1.0):
    from pyrite_amd import device
    rt, gt, ut, dt = types
    router = orc.normal(seed, E * H, 0.0, 0.02).astype(np.float32).view(np.uint8).copy() if rt == 0 else \
        _fast_random(rng, rt, E, H)
    gate = _fast_random(rng, gt, E * I, H)
    up = _fast_random(rng, ut, E * I, H)
    down = _fast_random(rng, dt, E * H, I)
    d = torch.device("cuda:0")
    layer = device.MoeLayer(rt, torch.from_numpy(router).to(d), gt, torch.from_numpy(gate).to(d),
                            ut, torch.from_numpy(up).to(d), dt, torch.from_numpy(down).to(d),
                            E, H, I, k, norm, scale)
    return layer, (router, gate, up, down)


def _check(orc, layer, host, xs, what):
    from pyrite_amd import device
    router, gate, up, down = host
    announce("moe", what, f"E={layer.n_experts}", f"H={layer.hidden}", f"I={layer.inter}", f"k={layer.k}",
             f"batch={xs.shape[0]}")
    out, ids, wts = device.moe_ffn(layer, torch.from_numpy(np.ascontiguousarray(xs)).to("cuda:0"))
    torch.cuda.synchronize()
    out, ids, wts = out.cpu().numpy(), ids.cpu().numpy(), wts.cpu().numpy()
    for b in range(xs.shape[0]):
        ref, rids, rw, _ = orc.moe_ffn(router, layer.router_type, gate, layer.gate_type, up, layer.up_type,
                                       down, layer.down_type, layer.n_experts, layer.hidden, layer.inter,
                                       layer.k, xs[b].astype(np.float64), layer.norm_topk_prob, layer.scale)
        assert list(ids[b]) == list(rids), f"{what} b={b}: ids {list(ids[b])} != {list(rids)}"
        np.testing.assert_allclose(wts[b], rw, rtol=2e-7, atol=1e-30, err_msg=f"{what} b={b} weights")
        scale = float(np.max(np.abs(ref))) if ref.size else 0.0
        err = float(np.max(np.abs(out[b].astype(np.float64) - ref)))
        assert err <= 1e-4 * scale + 1e-30, f"{what} b={b}: max err {err} vs scale {scale}"
    return ids


@pytest.mark.parametrize("batch", [1, 5, 20, 40, 90])
def test_moe_small(orc, dev, batch):
    rng = np.random.default_rng(100 + batch)
    layer, host = _layer(orc, rng, 16, 256, 256, 4, seed=7 + batch)
    xs = np.stack([orc.normal(500 + b, 256) for b in range(batch)])
    _check(orc, layer, host, xs, "small")


@pytest.mark.parametrize("norm,scale", [(False, 1.0), (True, 2.5), (False, 0.5)])
def test_moe_weight_options(orc, dev, norm, scale):
    rng = np.random.default_rng(200)
    layer, host = _layer(orc, rng, 32, 512, 256, 6, seed=21, norm=norm, scale=scale)
    xs = np.stack([orc.normal(600 + b, 512) for b in range(3)])
    _check(orc, layer, host, xs, f"norm={norm} scale={scale}")


@pytest.mark.parametrize("batch", [4, 48])
def test_moe_other_types(orc, dev, batch):
    """Q5_K gate and up, Q3_K down (VALU experts at 4 tokens, matrix-core experts at 48);
    mixed gate/up types keep the VALU experts."""
    rng = np.random.default_rng(300)
    for types in ((0, 13, 13, 11), (0, 13, 23, 11), (0, 8, 8, 2)):
        layer, host = _layer(orc, rng, 16, 512, 256, 4, types=types, seed=31)
        xs = np.stack([orc.normal(700 + b, 512) for b in range(batch)])
        _check(orc, layer, host, xs, f"types {types}")


@pytest.mark.parametrize("E,H,I,k,types", [
    (32, 512, 768, 12, (0, 12, 12, 14)),    # twelve slots
    (24, 256, 512, 16, (0, 12, 12, 14)),    # sixteen slots
    (16, 256, 2048, 4, (0, 2, 2, 2)),       # two units per lane of a down row (Q4_0, 2048 columns)
    (16, 512, 256, 6, (0, 13, 13, 11)),     # Q5_K gate/up, Q3_K down
    (16, 512, 256, 3, (0, 8, 8, 8)),        # Q8_0 throughout, three slots
])
def test_moe_single_token_shapes(orc, dev, E, H, I, k, types):
    """One token (pairs in slot order, combine without the position table):
    slot counts above eight, rows of two units per lane, other block formats."""
    rng = np.random.default_rng(E * 1000 + k * 10 + I)
    layer, host = _layer(orc, rng, E, H, I, k, types=types, seed=E + k + I)
    xs = orc.normal(1100 + k, H)[None, :]
    _check(orc, layer, host, xs, f"single token E={E} k={k} types {types}")


def test_moe_many_items_per_workgroup(orc, dev):
    """300 tokens over 64 experts: the down launch has more items (about 1200:
    chunks x 4 row parts) than workgroups (at most 4 per CU), so workgroups
    walk contiguous item ranges of two or more, reusing a chunk's staged
    fragments across its parts.  Every 7th token and the last are checked."""
    rng = np.random.default_rng(5300)
    layer, host = _layer(orc, rng, 64, 512, 256, 8, seed=5301)
    xs = np.stack([orc.normal(5400 + b, 512) for b in range(300)])
    from pyrite_amd import device
    announce("moe", "many items", "E=64", "H=512", "I=256", "k=8", "batch=300")
    out, ids, wts = device.moe_ffn(layer, torch.from_numpy(np.ascontiguousarray(xs)).to("cuda:0"))
    torch.cuda.synchronize()
    out, ids, wts = out.cpu().numpy(), ids.cpu().numpy(), wts.cpu().numpy()
    router, gate, up, down = host
    for b in list(range(0, 300, 7)) + [299]:
        ref, rids, rw, _ = orc.moe_ffn(router, layer.router_type, gate, layer.gate_type, up, layer.up_type,
                                       down, layer.down_type, layer.n_experts, layer.hidden, layer.inter,
                                       layer.k, xs[b].astype(np.float64), layer.norm_topk_prob, layer.scale)
        assert list(ids[b]) == list(rids), f"b={b}: ids {list(ids[b])} != {list(rids)}"
        np.testing.assert_allclose(wts[b], rw, rtol=2e-7, atol=1e-30, err_msg=f"b={b} weights")
        scale = float(np.max(np.abs(ref)))
        err = float(np.max(np.abs(out[b].astype(np.float64) - ref)))
        assert err <= 1e-4 * scale + 1e-30, f"b={b}: max err {err} vs scale {scale}"


def test_moe_router_ties(orc, dev):
    """Duplicate router rows: equal logits, the lower expert index ranks first."""
    rng = np.random.default_rng(400)
    E, H = 32, 512
    layer, host = _layer(orc, rng, E, H, 256, 8, seed=41)
    router = host[0].view(np.float32).reshape(E, H).copy()
    x = orc.normal(800, H)
    logits = router.astype(np.float64) @ x.astype(np.float64)
    top = int(np.argmax(logits))
    for dst in (0, 5, 17, 31):
        if dst != top:
            router[dst] = router[top]
    # near tie: one weight changed by one ulp
    near = (top + 9) % E
    router[near] = router[top]
    router[near, 3] = np.nextafter(router[near, 3], np.float32(np.inf))
    rbytes = router.view(np.uint8).reshape(-1).copy()
    layer.router = torch.from_numpy(rbytes).to("cuda:0")
    ids = _check(orc, layer, (rbytes,) + host[1:], x[None, :], "ties")
    assert len(set(ids[0].tolist())) == 8


def test_moe_repeat_and_graph(orc, dev):
    """Back-to-back calls of two batch sizes and graph replays give identical
    outputs: the routing kernel's arrival counter and the shared workspace
    carry nothing from one call into the next."""
    from pyrite_amd import device
    rng = np.random.default_rng(900)
    layer, host = _layer(orc, rng, 16, 256, 256, 4, seed=91)
    xs = np.stack([orc.normal(900 + b, 256) for b in range(3)])
    xa = torch.from_numpy(xs).to("cuda:0")
    xb = xa[:1].clone()
    announce("moe", "repeat + graph", "E=16", "H=256", "I=256", "k=4", "batch=3,1")
    first_a = device.moe_ffn(layer, xa)[0].clone()
    first_b = device.moe_ffn(layer, xb)[0].clone()
    for _ in range(2):
        assert torch.equal(device.moe_ffn(layer, xa)[0], first_a)
        assert torch.equal(device.moe_ffn(layer, xb)[0], first_b)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    out = torch.empty_like(first_a)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        device.moe_ffn(layer, xa, out=out)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, first_a)
        assert torch.equal(device.moe_ffn(layer, xb)[0], first_b)
    torch.cuda.synchronize()
    _check(orc, layer, host, xs, "repeat")


def test_moe_qwen3_30b_shape(orc, dev):
    """Qwen3-30B-A3B MoE shape: 128 experts, hidden 2048, moe_intermediate 768, top-8."""
    rng = np.random.default_rng(20244)
    layer, host = _layer(orc, rng, 128, 2048, 768, 8, seed=20244000)
    for batch in (1, 8, 64):
        xs = np.stack([orc.normal(20244100 + b, 2048) for b in range(batch)])
        _check(orc, layer, host, xs, f"qwen3-30b b={batch}")


# ---------------------------------------------------------------- (-p, e) ranking
# The reference ranks experts by (-p, e), p = exp(l - peak) / total
# (pyrite/executor.py:765-767, pyrite/tensor_ops.py:513-521).  Distinct fp64
# logits can give equal probabilities (l - peak rounds them together, exp
# rounds them together, or the division does), and the lower index then ranks
# first even though its logit is smaller.  These routers are F64 with rows
# whose only nonzero weight is in column 0 and x[0] = 1, so those rows' logits
# are exactly their weights; every other row is dense, so its exact logit
# (which enters the total) needs the reference's own summation order.

def _tie_layer(orc, E, H, crafted, seed):
    from pyrite_amd import device
    rng = np.random.default_rng(seed)
    w = rng.normal(0.0, 0.002, size=(E, H))
    for e, v in crafted.items():
        w[e] = 0.0
        w[e, 0] = v
    router = np.ascontiguousarray(w, dtype=np.float64).view(np.uint8).reshape(-1).copy()
    I = 256
    gate = _fast_random(rng, 12, E * I, H)
    up = _fast_random(rng, 12, E * I, H)
    down = _fast_random(rng, 14, E * H, I)
    d = torch.device("cuda:0")
    layer = device.MoeLayer(28, torch.from_numpy(router).to(d), 12, torch.from_numpy(gate).to(d),
                            12, torch.from_numpy(up).to(d), 14, torch.from_numpy(down).to(d), E, H, I, 8)
    return layer, (router, gate, up, down)


def _tie_x(orc, H, seed):
    x = orc.normal(seed, H).astype(np.float32)
    x[0] = 1.0
    return x


def _ref_route(orc, router, E, H, x, k=8):
    logits = orc.matvec(28, router, x.astype(np.float64), E, H)
    ids, w, probs = orc.route(logits, k)
    by_logit = sorted(range(E), key=lambda e: (-logits[e], e))[:k]
    return logits, list(ids), probs, by_logit


def test_moe_rank_tie_at_peak(orc, dev):
    """Logits 0.3 (expert 40) and the next double below (expert 7): the
    probabilities are equal, so expert 7 ranks first."""
    E, H = 128, 256
    v = 0.3
    layer, host = _tie_layer(orc, E, H, {40: v, 7: float(np.nextafter(v, 0.0))}, seed=5101)
    x = _tie_x(orc, H, 5102)
    logits, ids, probs, by_logit = _ref_route(orc, host[0], E, H, x)
    assert ids[:2] == [7, 40] and by_logit[:2] == [40, 7] and probs[7] == probs[40], "case does not tie"
    _check(orc, layer, host, x[None, :], "tie at the peak")


def test_moe_rank_tie_at_boundary(orc, dev):
    """Two logits one double apart at the k-th place: the lower index (20)
    takes the last slot although expert 50's logit is larger."""
    E, H = 128, 256
    crafted = {3: 1.0, 10: 0.9, 11: 0.85, 12: 0.8, 13: 0.75, 14: 0.7, 15: 0.65}
    # 0.2 + j * 2^-55 and the double below it differ by a quarter ulp of
    # their difference from the peak, so l - peak often rounds them together;
    # the dense rows stay far below, so the crafted logits alone decide
    for j in range(1, 4000):
        c = 0.2 + j * 2.0 ** -55
        cr = {**crafted, 50: c, 20: float(np.nextafter(c, 0.0))}
        lg = np.array([cr.get(e, -1.0) for e in range(E)])
        ids, _, p = orc.route(lg, 8)
        if 20 in ids and 50 not in ids:
            break
    else:
        pytest.fail("no boundary tie found")
    layer, host = _tie_layer(orc, E, H, cr, seed=5201)
    x = _tie_x(orc, H, 5202)
    logits, ids, probs, by_logit = _ref_route(orc, host[0], E, H, x)
    assert 20 in ids and 50 not in ids and 50 in by_logit and 20 not in by_logit, "case does not tie"
    _check(orc, layer, host, x[None, :], "tie at the boundary")


def test_moe_rank_tie_in_division(orc, dev):
    """exp(l - peak) differs by one ulp between experts 9 and 60, yet
    dividing by the total rounds both probabilities to one value: expert 9
    (the smaller exp) ranks first.  Needs the exact total, i.e. every row's
    exact logit and the left-to-right sum."""
    import math
    E, H = 128, 256
    x = _tie_x(orc, H, 5302)
    found = None
    # exp values just below 1 (the top of their binade) and probabilities
    # near the bottom of theirs: a one-ulp step in exp is then often less
    # than one ulp of the quotient
    base = np.random.default_rng(5301).normal(0.0, 0.002, size=(E, H))
    for j in range(1, 200):
        va = 1.0 - j * 2.0 ** -20
        for d in range(1, 4):
            vb = va - d * 2.0 ** -53
            cr = {0: 1.0, 33: 0.95, 60: va, 9: vb}
            w = base.copy()
            for e, val in cr.items():
                w[e] = 0.0
                w[e, 0] = val
            router = np.ascontiguousarray(w).view(np.uint8).reshape(-1)
            logits, ids, probs, by_logit = _ref_route(orc, router, E, H, x)
            peak = max(logits)
            ea, eb = math.exp(logits[60] - peak), math.exp(logits[9] - peak)
            if ea != eb and probs[60] == probs[9] and ids.index(9) < ids.index(60):
                found = cr
                break
        if found:
            break
    assert found, "no division tie found"
    layer, host = _tie_layer(orc, E, H, found, seed=5301)
    _check(orc, layer, host, x[None, :], "tie in the division")


def test_moe_rank_ties_batch(orc, dev):
    """The peak tie as the first and last token of a batch, ordinary tokens
    between them: each token takes its own path through the ranking."""
    E, H = 128, 256
    v = 0.3
    layer, host = _tie_layer(orc, E, H, {40: v, 7: float(np.nextafter(v, 0.0))}, seed=5101)
    xs = np.stack([_tie_x(orc, H, 5102)] + [orc.normal(5400 + b, H) for b in range(5)] + [_tie_x(orc, H, 5102)])
    _check(orc, layer, host, xs.astype(np.float32), "ties in a batch")
