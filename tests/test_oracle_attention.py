"""Pins of the oracle's RoPE and single-token attention (oracle_rope,
oracle_attention: pyrite/executor.py:627-646, 685-755) by closed forms and
invariants, each chosen so that a plausible slip fails it: pairing (2i, 2i+1)
instead of (i, i + half), a wrong rotation sign, an angle not linear in the
position, a frequency off by a factor, a wrong query-head -> kv-head map,
a missing scale, the QK-norm not applied, keys not stored as fp32."""
from __future__ import annotations

import math

import numpy as np
import pytest


@pytest.fixture(scope="module")
def o(orc):
    return orc


def test_rope_position_zero_is_identity(o):
    x = np.random.default_rng(1).standard_normal(128)
    assert np.array_equal(o.rope(x, 0, 10000.0), x)


def test_rope_rotates_pairs_i_and_i_plus_half(o):
    """Each pair (i, i + 64) keeps its length; the tail beyond rotary_dim is untouched."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal(128)
    y = o.rope(x, 37, 10000.0)
    n0 = np.hypot(x[:64], x[64:])
    n1 = np.hypot(y[:64], y[64:])
    np.testing.assert_allclose(n1, n0, rtol=1e-14)
    # (2i, 2i+1) pairs are not preserved: the layout is not interleaved
    assert not np.allclose(np.hypot(y[0::2], y[1::2]), np.hypot(x[0::2], x[1::2]), rtol=1e-6)
    z = o.rope(x, 37, 10000.0, rotary_dim=64)
    assert np.array_equal(z[64:], x[64:])
    np.testing.assert_allclose(np.hypot(z[:32], z[32:64]), np.hypot(x[:32], x[32:64]), rtol=1e-14)


def test_rope_first_pair_turns_by_the_position_counterclockwise(o):
    """freq_0 = theta^0 = 1: e_0 at position p becomes cos p e_0 + sin p e_half."""
    for p in (1, 2, 5, 1000):
        e0 = np.zeros(16)
        e0[0] = 1.0
        y = o.rope(e0, p, 500000.0)
        assert y[0] == math.cos(p) and y[8] == math.sin(p)
        assert np.count_nonzero(y) == 2


def test_rope_frequencies(o):
    """Pair i turns by p * theta^(-2i / n_rot) (checked through the angle recovered from the output)."""
    theta, n = 10000.0, 32
    for i in (1, 5, 15):
        e = np.zeros(n)
        e[i] = 1.0
        y = o.rope(e, 3, theta)
        got = math.atan2(y[i + n // 2], y[i])
        want = 3 * theta ** (-2.0 * i / n)
        assert abs(got - want) < 1e-12


def test_rope_is_additive_in_position(o):
    x = np.random.default_rng(3).standard_normal(64)
    np.testing.assert_allclose(o.rope(o.rope(x, 11, 1e4), 29, 1e4), o.rope(x, 40, 1e4), rtol=0, atol=1e-12)


def test_rope_scores_depend_on_relative_position(o):
    rng = np.random.default_rng(4)
    q, k = rng.standard_normal(64), rng.standard_normal(64)
    a = float(o.rope(q, 50, 1e4) @ o.rope(k, 45, 1e4))
    b = float(o.rope(q, 1005, 1e4) @ o.rope(k, 1000, 1e4))
    assert abs(a - b) < 1e-10 * (1 + abs(a))


def _caches(n_tok, n_kv, hd, vd):
    return np.zeros((n_tok, n_kv * hd), np.float32), np.zeros((n_tok, n_kv * vd), np.float32)


def test_attention_single_token_returns_its_value(o):
    """One token: softmax of one score is 1, so each head returns its kv head's value (as fp32)."""
    rng = np.random.default_rng(5)
    nh, nkv, hd, vd = 8, 2, 16, 12
    q, k, v = rng.standard_normal(nh * hd), rng.standard_normal(nkv * hd), rng.standard_normal(nkv * vd)
    kc, vc = _caches(1, nkv, hd, vd)
    out = o.attention(q, k, v, nh, nkv, hd, vd, kc, vc, 0, 7)
    for h in range(nh):
        g = h // (nh // nkv)
        assert np.array_equal(out[h * vd:(h + 1) * vd], v[g * vd:(g + 1) * vd].astype(np.float32).astype(np.float64))


def test_attention_heads_read_their_group_kv_head(o):
    """Values constant per kv head (g + 1): head h returns h // group + 1."""
    nh, nkv, hd, vd, n_prev = 12, 3, 8, 4, 5
    rng = np.random.default_rng(6)
    kc, vc = _caches(n_prev + 1, nkv, hd, vd)
    kc[:n_prev] = rng.standard_normal((n_prev, nkv * hd))
    for g in range(nkv):
        vc[:, g * vd:(g + 1) * vd] = g + 1
    v = np.repeat(np.arange(1, nkv + 1, dtype=np.float64), vd)
    out = o.attention(rng.standard_normal(nh * hd), rng.standard_normal(nkv * hd), v, nh, nkv, hd, vd, kc, vc,
                      n_prev, 9)
    for h in range(nh):
        np.testing.assert_allclose(out[h * vd:(h + 1) * vd], h // (nh // nkv) + 1, rtol=1e-15)


def test_attention_equal_keys_average_the_values(o):
    nh, nkv, hd, vd, n_prev = 2, 1, 8, 6, 9
    rng = np.random.default_rng(7)
    k = rng.standard_normal(hd)
    kc, vc = _caches(n_prev + 1, nkv, hd, vd)
    kc[:] = o.rope(k, 4, 1e4).astype(np.float32)  # the stored key of the new token at position 4
    vc[:n_prev] = rng.standard_normal((n_prev, vd))
    v = rng.standard_normal(vd)
    out = o.attention(rng.standard_normal(nh * hd), k, v, nh, nkv, hd, vd, kc, vc, n_prev, 4)
    mean = vc.astype(np.float64).mean(axis=0)
    np.testing.assert_allclose(out[:vd], mean, rtol=1e-12)
    np.testing.assert_allclose(out[vd:], mean, rtol=1e-12)


def test_attention_scale_and_stored_key_precision(o):
    """Two tokens whose scores are s and 0: weights e^(s/sqrt(hd)) : 1 with
    s computed against the fp32-rounded stored key."""
    hd = 16
    q = np.zeros(hd)
    q[3] = 2.5
    kprev = np.zeros(hd, np.float32)
    kprev[3] = np.float32(0.1)  # stored as fp32: score = 2.5 * (double)(float)0.1
    kc = np.zeros((2, hd), np.float32)
    vc = np.zeros((2, 1), np.float32)
    kc[0] = kprev
    vc[0] = 1.0
    out = o.attention(q, np.zeros(hd), np.zeros(1), 1, 1, hd, 1, kc, vc, 1, 0)
    s = 2.5 * float(np.float32(0.1)) / math.sqrt(hd)
    assert abs(out[0] - math.exp(s) / (math.exp(s) + 1.0)) < 1e-15


def test_attention_qk_norm_makes_scores_scale_free(o):
    """With QK-norm, q and 3q attend identically; without it they do not."""
    rng = np.random.default_rng(8)
    nh, nkv, hd, vd, n_prev = 4, 2, 16, 8, 6
    q, k, v = rng.standard_normal(nh * hd), rng.standard_normal(nkv * hd), rng.standard_normal(nkv * vd)
    w = np.ones(hd)
    base = rng.standard_normal((n_prev, nkv * hd)).astype(np.float32)
    vals = rng.standard_normal((n_prev, nkv * vd)).astype(np.float32)

    def run(qq, qn):
        kc, vc = _caches(n_prev + 1, nkv, hd, vd)
        kc[:n_prev], vc[:n_prev] = base, vals
        # eps far below the mean square, so the norm is scale-free up to rounding
        return o.attention(qq, k, v, nh, nkv, hd, vd, kc, vc, n_prev, 3, q_norm=qn, k_norm=qn, eps=1e-30)
    np.testing.assert_allclose(run(q, w), run(3 * q, w), rtol=1e-12, atol=1e-14)
    assert not np.allclose(run(q, None), run(3 * q, None), rtol=1e-6)
