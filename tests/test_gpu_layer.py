"""GPU parity of the layer operations around the matvecs, and of a whole decode step.

- add_rms_norm: the residual sum is fp32 h + delta bit for bit; the norm is
  within one fp32 ulp of (float) of the oracle's fp64 rms_norm of that sum.
- matvec_swiglu: within the matvec bar 1e-4 * ||act||_2 * max|row| of the
  oracle's matvec of act = silu(gate) * up formed in fp64.
- attention_decode: token after token against oracle_attention (its own
  fp32 KV list, oldest-first eviction at the capacity), at Llama-3, Qwen3
  (QK-norm) and partial-rotary / narrow-value shapes: every output within
  2e-5 * max|value| (fp64 scores and softmax, fp32 sums of 256 values per
  chunk), the cached keys within one fp32 ulp of the oracle's.
- Decoder.step over a GGUF checkpoint written to disk (a dense Llama-like and
  a Qwen3-MoE-like model, two layers each, a KV capacity smaller than the
  sequence): logits against the oracle's fp64 composition of the same
  operations in the reference executor's order (pyrite/executor.py:795-875),
  within 2e-3 * max|logit| (fp32 activations between launches against fp64),
  and the greedy id equal to the oracle's wherever the oracle's top two
  logits are further apart than twice that bound.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle.oracle import TYPES, row_bytes
from tests import gguf_writer as gw
from tests.gpu_util import announce, assert_matvec_close

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from pyrite_amd import _lib
    _lib.load()
    return torch.device("cuda:0")


def _ulp32(x):
    x = np.abs(np.asarray(x, dtype=np.float32))
    return np.spacing(x).astype(np.float64)


@pytest.mark.parametrize("n,batch", [(4096, 1), (2048, 3), (1000, 2)])
def test_add_rms_norm(orc, dev, n, batch):
    from pyrite_amd import device
    rng = np.random.default_rng(n + batch)
    h = rng.standard_normal((batch, n)).astype(np.float32)
    d = (rng.standard_normal((batch, n)) * 0.3).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    announce("add_rms_norm", n, batch)
    ht = torch.from_numpy(h).to(dev)
    ho, nt = device.add_rms_norm(ht, torch.from_numpy(d).to(dev), torch.from_numpy(w).to(dev), 1e-5, h_out=ht)
    ho, nt = ho.cpu().numpy(), nt.cpu().numpy()
    s = h + d  # fp32 adds
    assert np.array_equal(ho.view(np.uint32), s.view(np.uint32))
    for b in range(batch):
        ref = orc.rms_norm(s[b].astype(np.float64), w.astype(np.float64), 1e-5)
        assert np.all(np.abs(nt[b] - ref) <= _ulp32(ref))


@pytest.mark.parametrize("t,rows,cols,batch", [(14, 4096, 14336, 1), (12, 2048, 5632, 2), (8, 300, 1024, 3),
                                                (2, 96, 512, 1), (13, 64, 256, 2)])
def test_matvec_swiglu(orc, dev, t, rows, cols, batch):
    from pyrite_amd import device
    payload = orc.quantize(t, orc.normal(3100 + rows, rows * cols, 0.0, 0.02).astype(np.float64))
    rng = np.random.default_rng(rows + cols)
    g = (rng.standard_normal((batch, cols)) * 3).astype(np.float32)
    u = rng.standard_normal((batch, cols)).astype(np.float32)
    g[0, :8] = [-61.0, -60.0, -59.9, 0.0, -0.0, 80.0, -1e-30, 1e-3]
    announce("matvec_swiglu", TYPES[t][0], rows, cols, batch)
    y = device.matvec_swiglu(t, torch.from_numpy(payload).to(dev), torch.from_numpy(g).to(dev),
                             torch.from_numpy(u).to(dev), rows, cols).cpu().numpy()
    rb = row_bytes(t, cols)
    rowmax = np.concatenate([np.abs(orc.dequantize_rows(t, payload[r0 * rb:min(rows, r0 + 512) * rb],
                                                        min(512, rows - r0), cols).reshape(-1, cols)).max(axis=1)
                             for r0 in range(0, rows, 512)])
    for b in range(batch):
        act = np.array([orc.silu(float(a)) for a in g[b].astype(np.float64)]) * u[b].astype(np.float64)
        ref = orc.matvec(t, payload, act, rows, cols)
        assert_matvec_close(y[b], ref, act, rowmax, f"swiglu {TYPES[t][0]} {rows}x{cols} b{b}")


def test_matvec_swiglu_refuses_what_it_cannot_stage(orc, dev):
    from pyrite_amd import _lib, device
    w = torch.zeros(64 * (40960 // 256) * 144, dtype=torch.uint8, device=dev)
    g = torch.zeros(1, 40960, device=dev)
    with pytest.raises(_lib.KernelError) as e:
        device.matvec_swiglu(12, w, g, g.clone(), 64, 40960)
    assert e.value.code == -2
    wf = torch.zeros(64 * 256 * 4, dtype=torch.uint8, device=dev)
    with pytest.raises(_lib.KernelError) as e:
        device.matvec_swiglu(0, wf, g[:, :256].contiguous(), g[:, :256].contiguous(), 64, 256)
    assert e.value.code == -1


ATTN_SHAPES = {
    # name: (n_heads, n_kv, head_dim, value_dim, rotary_dim, theta, qk_norm, capacity, tokens)
    "llama3": (32, 8, 128, 128, 0, 500000.0, False, 1024, 600),
    "qwen3": (16, 8, 128, 128, 0, 1000000.0, True, 512, 300),
    "partial_rotary": (6, 2, 64, 48, 32, 10000.0, False, 700, 520),
    "evicting": (8, 1, 64, 64, 0, 10000.0, True, 260, 400),
}


@pytest.mark.parametrize("name", list(ATTN_SHAPES))
def test_attention_decode(orc, dev, name):
    from pyrite_amd import device
    nh, nkv, hd, vd, rd, theta, qkn, cap, T = ATTN_SHAPES[name]
    rng = np.random.default_rng(sum(map(ord, name)))
    qn = (1 + 0.2 * rng.standard_normal(hd)).astype(np.float32) if qkn else None
    kn = (1 + 0.2 * rng.standard_normal(hd)).astype(np.float32) if qkn else None
    cache = device.AttentionCache(nh, nkv, hd, vd, cap, rope_theta=theta, rotary_dim=rd, eps=1e-6,
                                  q_norm=None if qn is None else torch.from_numpy(qn).to(dev),
                                  k_norm=None if kn is None else torch.from_numpy(kn).to(dev), device=dev)
    keys, vals = [], []  # the oracle's fp32 KV, oldest first
    checked = 0
    announce("attention", name, nh, nkv, hd, vd, rd, theta, qkn, cap, T)
    for pos in range(T):
        q = (rng.standard_normal(nh * hd) * 0.5).astype(np.float32)
        k = (rng.standard_normal(nkv * hd) * 0.5).astype(np.float32)
        v = rng.standard_normal(nkv * vd).astype(np.float32)
        out = device.attention_decode(cache, torch.from_numpy(q).to(dev), torch.from_numpy(k).to(dev),
                                      torch.from_numpy(v).to(dev), pos)
        # the reference appends, truncates to the capacity (oldest first), then attends
        # (pyrite/executor.py:729-735): cap - 1 earlier tokens plus this one
        del keys[:max(0, len(keys) - (cap - 1))]
        del vals[:max(0, len(vals) - (cap - 1))]
        n_prev = len(keys)
        kc = np.zeros((n_prev + 1, nkv * hd), np.float32)
        vc = np.zeros((n_prev + 1, nkv * vd), np.float32)
        if n_prev:
            kc[:n_prev], vc[:n_prev] = np.stack(keys), np.stack(vals)
        ref = orc.attention(q, k, v, nh, nkv, hd, vd, kc, vc, n_prev, pos, theta=theta, rotary_dim=rd,
                            eps=1e-6, q_norm=qn, k_norm=kn)
        keys.append(kc[n_prev].copy())
        vals.append(vc[n_prev].copy())
        if pos < 8 or pos % 37 == 0 or pos == T - 1 or cap - 2 <= pos <= cap + 2:
            got = out.cpu().numpy().astype(np.float64)
            bound = 2e-5 * float(np.abs(vc).max())
            err = float(np.abs(got - ref).max())
            assert err <= bound, f"{name} pos {pos}: max err {err} > {bound}"
            slot = pos % cap
            dk = cache.k_cache[slot].cpu().numpy()
            assert np.all(np.abs(dk.astype(np.float64) - kc[n_prev]) <= _ulp32(kc[n_prev])), f"{name} pos {pos} key"
            checked += 1
    assert checked > 8


def test_attention_refuses_bad_shapes(dev):
    from pyrite_amd import _lib, device
    cache = device.AttentionCache(6, 4, 64, 64, 16, device=dev)  # 6 heads over 4 kv heads
    z = torch.zeros(6 * 64, device=dev)
    with pytest.raises(_lib.KernelError) as e:
        device.attention_decode(cache, z, torch.zeros(4 * 64, device=dev), torch.zeros(4 * 64, device=dev), 0)
    assert e.value.code == -2


# ---------------------------------------------------------------- whole decode steps

def _model(orc, tmp_path, moe: bool):
    """A two-layer checkpoint: dense (Llama-like, GQA 4/2) or Qwen3-MoE-like (QK-norm, partial rotary)."""
    from pyrite_amd.decoder import DecoderConfig
    H, NH, NKV, HD, FF, V = 256, 4, 2, 64, 512, 384
    E, KX, MI = 8, 2, 256
    cfg = DecoderConfig(hidden_size=H, num_hidden_layers=2, num_attention_heads=NH, num_key_value_heads=NKV,
                        head_dim=HD, value_dim=HD, rope_theta=1e6 if moe else 5e5, rms_norm_eps=1e-6,
                        max_kv_tokens=4, rotary_dim=32 if moe else 0, num_experts_per_tok=KX if moe else 0)
    rng = np.random.default_rng(77 + moe)
    seed = [9000 + 100 * moe]

    def q(t, rows, cols):
        seed[0] += 1
        return orc.quantize(t, orc.normal(seed[0], rows * cols, 0.0, 0.02).astype(np.float64)).astype(np.uint8)

    def vec(n):
        return (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)

    host = {"token_embd.weight": ((H, V), 8, q(8, V, H)), "output.weight": ((H, V), 14, q(14, V, H)),
            "output_norm.weight": ((H,), 0, vec(H))}
    for i in range(2):
        p = f"blk.{i}."
        host[p + "attn_norm.weight"] = ((H,), 0, vec(H))
        host[p + "ffn_norm.weight"] = ((H,), 0, vec(H))
        host[p + "attn_q.weight"] = ((H, NH * HD), 12, q(12, NH * HD, H))
        host[p + "attn_k.weight"] = ((H, NKV * HD), 12, q(12, NKV * HD, H))
        host[p + "attn_v.weight"] = ((H, NKV * HD), 14 if i else 12, q(14 if i else 12, NKV * HD, H))
        host[p + "attn_output.weight"] = ((NH * HD, H), 12, q(12, H, NH * HD))
        if moe:
            host[p + "attn_q_norm.weight"] = ((HD,), 0, vec(HD))
            host[p + "attn_k_norm.weight"] = ((HD,), 0, vec(HD))
            host[p + "ffn_gate_inp.weight"] = ((H, E), 0, orc.normal(seed[0] + 50, E * H, 0.0, 0.02).astype(np.float32))
            host[p + "ffn_gate_exps.weight"] = ((H, MI, E), 12, q(12, E * MI, H))
            host[p + "ffn_up_exps.weight"] = ((H, MI, E), 12, q(12, E * MI, H))
            host[p + "ffn_down_exps.weight"] = ((MI, H, E), 14, q(14, E * H, MI))
        else:
            host[p + "ffn_gate.weight"] = ((H, FF), 12, q(12, FF, H))
            host[p + "ffn_up.weight"] = ((H, FF), 12, q(12, FF, H))
            host[p + "ffn_down.weight"] = ((FF, H), 14, q(14, H, FF))
    w = gw.Writer()
    for name, (dims, t, data) in host.items():
        w.tensor(name, dims, t, np.ascontiguousarray(data).view(np.uint8).tobytes())
    path = tmp_path / ("moe.gguf" if moe else "dense.gguf")
    path.write_bytes(w.bytes())
    return cfg, host, path


def _ref_steps(orc, cfg, host, tokens):
    """The oracle's fp64 composition, in the reference executor's order."""
    H, eps = cfg.hidden_size, cfg.rms_norm_eps
    nh, nkv, hd, vd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.value_dim

    def f64(name):
        return host[name][2].view(np.float32).astype(np.float64)

    def mv(name, x):
        (cols, rows, *_), t, data = host[name]
        return orc.matvec(t, data.view(np.uint8), np.asarray(x, np.float64), rows, cols)

    kv = [([], []) for _ in range(cfg.num_hidden_layers)]
    out = []
    et = host["token_embd.weight"][1]
    erb = row_bytes(et, H)
    for pos, tok in enumerate(tokens):
        h = orc.dequantize_rows(et, host["token_embd.weight"][2][tok * erb:(tok + 1) * erb], 1, H)
        for i in range(cfg.num_hidden_layers):
            p = f"blk.{i}."
            normed = orc.rms_norm(h, f64(p + "attn_norm.weight"), eps)
            qv, kvv, vv = mv(p + "attn_q.weight", normed), mv(p + "attn_k.weight", normed), mv(p + "attn_v.weight", normed)
            keys, vals = kv[i]
            # append, truncate to max_kv_tokens (oldest first), then attend (pyrite/executor.py:729-735)
            del keys[:max(0, len(keys) - (cfg.max_kv_tokens - 1))]
            del vals[:max(0, len(vals) - (cfg.max_kv_tokens - 1))]
            n_prev = len(keys)
            kc = np.zeros((n_prev + 1, nkv * hd), np.float32)
            vc = np.zeros((n_prev + 1, nkv * vd), np.float32)
            if n_prev:
                kc[:n_prev], vc[:n_prev] = np.stack(keys), np.stack(vals)
            qn = f64(p + "attn_q_norm.weight") if p + "attn_q_norm.weight" in host else None
            kn = f64(p + "attn_k_norm.weight") if p + "attn_k_norm.weight" in host else None
            a = orc.attention(qv, kvv, vv, nh, nkv, hd, vd, kc, vc, n_prev, pos, theta=cfg.rope_theta,
                              rotary_dim=cfg.rotary_dim, eps=eps, q_norm=qn, k_norm=kn)
            keys.append(kc[n_prev].copy())
            vals.append(vc[n_prev].copy())
            h = h + mv(p + "attn_output.weight", a)
            n2 = orc.rms_norm(h, f64(p + "ffn_norm.weight"), eps)
            if cfg.num_experts_per_tok:
                (hd_, E), rt, router = host[p + "ffn_gate_inp.weight"]
                (_, mi, _), gt, gate = host[p + "ffn_gate_exps.weight"]
                _, ut, up = host[p + "ffn_up_exps.weight"]
                _, dt, down = host[p + "ffn_down_exps.weight"]
                d, *_ = orc.moe_ffn(router.view(np.uint8), rt, gate, gt, up, ut, down, dt, E, H, mi,
                                    cfg.num_experts_per_tok, n2, cfg.norm_topk_prob, cfg.expert_weights_scale)
            else:
                g, u = mv(p + "ffn_gate.weight", n2), mv(p + "ffn_up.weight", n2)
                d = mv(p + "ffn_down.weight", np.array([orc.silu(x) for x in g]) * u)
            h = h + d
        normed = orc.rms_norm(h, f64("output_norm.weight"), eps)
        out.append(mv("output.weight", normed))
    return out


@pytest.mark.parametrize("moe", [False, True], ids=["dense", "moe"])
def test_decoder_steps_match_the_oracle(orc, dev, tmp_path, moe):
    from pyrite_amd.decoder import Decoder
    from pyrite_amd.gguf import GGUFReader
    from pyrite_amd.resident import ResidentTensors
    cfg, host, path = _model(orc, tmp_path, moe)
    tokens = [5, 17, 300, 17, 42, 5, 99]
    announce("decoder", "moe" if moe else "dense", "layers 2", "tokens", len(tokens), "kv capacity 4")
    dec = Decoder(ResidentTensors(GGUFReader(path), device=dev), cfg)
    got = []
    for pos, tok in enumerate(tokens):
        logits, ids = dec.step(tok, pos)
        got.append((logits.cpu().numpy().astype(np.float64), int(ids.cpu()[0])))
    ref = _ref_steps(orc, cfg, host, tokens)
    for pos, ((lg, gid), rl) in enumerate(zip(got, ref)):
        scale = float(np.abs(rl).max())
        err = float(np.abs(lg - rl).max())
        assert err <= 2e-3 * scale, f"pos {pos}: max err {err} vs max|logit| {scale}"
        top2 = np.sort(rl)[-2:]
        if top2[1] - top2[0] > 4e-3 * scale:
            assert gid == orc.argmax_first(rl), f"pos {pos}: id {gid} != {orc.argmax_first(rl)}"
