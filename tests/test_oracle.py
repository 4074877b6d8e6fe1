"""The CPU oracle, pinned before anything is compared against it.

Pins, per part of the oracle:
* decoders + matvec + dequantize_rows: golden vectors written by the reference's
  own native.c (built unmodified, tests/golden/make_golden.py) -- bit exact --
  plus the known answers of the reference's tests (test_tensor_ops.py:14-27,
  test_ggml_decoders.py:92-184) and invariants (zero blocks, linearity, row
  independence, expert slices);
* fp16 conversion: exhaustive against numpy's independent float16 code;
* K-quant encoders: byte-exact against the reference's tests/k_quant.py outputs;
* Q8_0/Q4_0 encoders: hand-derived known answers (scripts/build_vocab_fixture.py:45-89);
* routing/softmax/silu/argmax: defining properties and closed forms.
"""
from __future__ import annotations

import hashlib
import math
import struct

import numpy as np
import pytest

from oracle.oracle import TYPES, lcg_payload, reference, row_bytes


def _bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype="<f8").view("<u8")


def _sha(a: np.ndarray) -> bytes:
    return hashlib.sha256(np.ascontiguousarray(a, dtype="<f8").tobytes()).digest()


@pytest.fixture(scope="module")
def native_golden(golden_dir):
    return np.load(golden_dir / "native_kernels.npz")


@pytest.mark.parametrize("case", ["lcg", "rand", "special"])
@pytest.mark.parametrize("type_id", sorted(TYPES), ids=lambda t: TYPES[t][0])
def test_oracle_matches_reference_golden_vectors(orc, native_golden, type_id, case):
    key = f"t{type_id}_{case}"
    rows, cols = (int(v) for v in native_golden[key + "_shape"])
    payload = native_golden[key + "_payload"]
    x = native_golden[key + "_x"]
    got = orc.matvec(type_id, payload, x, rows, cols)
    exp = native_golden[key + "_matvec"]
    assert np.array_equal(_bits(got), _bits(exp)) or np.array_equal(np.isnan(got), np.isnan(exp)) and \
        np.array_equal(got[~np.isnan(got)], exp[~np.isnan(exp)])
    deq = orc.dequantize_rows(type_id, payload, rows, cols)
    assert _sha(deq) == native_golden[key + "_dequant_sha"].tobytes()
    if case == "lcg":
        assert np.array_equal(_bits(deq), _bits(native_golden[key + "_dequant"]))


def test_oracle_matches_reference_on_config_shaped_inputs(orc, golden_dir):
    z = np.load(golden_dir / "seeded_kernels.npz")
    keys = sorted({k.rsplit("_", 1)[0] for k in z.files if k.endswith("_payload")})
    assert len(keys) == 10
    for key in keys:
        t = int(key.split("_")[0][1:])
        rows, cols = (int(v) for v in key.split("_")[1].split("x"))
        got = orc.matvec(t, z[key + "_payload"], z[key + "_x"], rows, cols)
        assert np.array_equal(_bits(got), _bits(z[key + "_matvec"])), key
        deq = orc.dequantize_rows(t, z[key + "_payload"], rows, cols)
        assert _sha(deq) == z[key + "_dequant_sha"].tobytes(), key


def test_oracle_matches_live_reference_build_when_present(orc):
    ref = reference()
    if ref is None:
        pytest.skip("oracle/_ref was not built (no reference checkout)")
    assert ref.native_types() == orc.native_types()
    rng = np.random.default_rng(77)
    for t, (name, bs, bpb) in TYPES.items():
        rows, cols = 5, 1024
        if t in (0, 28):
            payload = rng.standard_normal(rows * cols).astype("<f4" if t == 0 else "<f8").view(np.uint8).copy()
        else:
            payload = rng.integers(0, 256, rows * row_bytes(t, cols), dtype=np.uint8)
        x = rng.standard_normal(cols)
        a, b = orc.dequantize_rows(t, payload, rows, cols), ref.dequantize_rows(t, payload, rows, cols)
        assert np.array_equal(np.isnan(a), np.isnan(b)), name
        assert np.array_equal(_bits(a)[~np.isnan(a)], _bits(b)[~np.isnan(b)]), name


def test_native_type_table():
    from oracle.oracle import oracle

    ids = oracle().native_types()
    assert ids == [0, 1, 2, 3, 6, 7, 8, 9, 10, 11, 12, 13, 14, 20, 23, 24, 25, 26, 27, 28, 30]


# ------------------------------------------------------------------ error codes
def test_error_codes_follow_the_reference(orc):
    """pyrite/kernels/native.c:496-525, 562-566: -1 type, -2 geometry, -3 buffer."""
    data = np.zeros(row_bytes(12, 256) * 2, dtype=np.uint8)
    x = np.zeros(256)
    out = np.zeros(2)
    assert orc.matvec_raw(99, data, x, out, 2, 256) == -1
    assert orc.matvec_raw(12, data, x, out, 0, 256) == -2
    assert orc.matvec_raw(12, data, x, out, 2, 0) == -2
    assert orc.matvec_raw(12, data, np.zeros(100), out, 2, 100) == -2
    assert orc.matvec_raw(12, data[:-1], x, out, 2, 256) == -3
    assert orc.matvec_raw(12, None, x, out, 2, 256) == -3
    assert orc.matvec_raw(12, data, None, out, 2, 256) == -3
    assert orc.matvec_raw(12, data, x, out, 2, 256) == 0


# ------------------------------------------------------------------ known answers
def test_known_answers_from_reference_tests(orc):
    # test_tensor_ops.py:14-27
    assert orc.decode_block(0, np.frombuffer(struct.pack("<f", 1.5), np.uint8))[0] == 1.5
    assert orc.decode_block(1, np.frombuffer(struct.pack("<e", 2.5), np.uint8))[0] == 2.5
    assert orc.decode_block(30, np.frombuffer(struct.pack("<H", 0x3F80), np.uint8))[0] == 1.0
    q8 = np.frombuffer(struct.pack("<e", 1.0) + bytes([1] * 32), np.uint8)
    assert list(orc.decode_block(8, q8)) == [1.0] * 32
    q4 = np.frombuffer(struct.pack("<e", 1.0) + bytes([0x88] * 16), np.uint8)
    assert list(orc.decode_block(2, q4)) == [0.0] * 32
    # test_ggml_decoders.py:180-184: low nibble is element i, high is i + 16
    q4 = np.frombuffer(struct.pack("<e", 1.0) + bytes([0x80] * 16), np.uint8)
    assert list(orc.decode_block(2, q4)) == [-8.0] * 16 + [0.0] * 16
    # :164-168 Q8_1 = d | s | qs
    q81 = np.frombuffer(struct.pack("<e", 0.5) + struct.pack("<e", 0.25) + bytes([2] * 32), np.uint8)
    assert list(orc.decode_block(9, q81)) == [1.0] * 32
    # :156-161 BF16 is the top half of an fp32
    for word in [0x3F80, 0xBF80, 0x4048, 0x0000, 0x7F7F]:
        exp = struct.unpack("<f", struct.pack("<I", word << 16))[0]
        assert orc.decode_block(30, np.frombuffer(struct.pack("<H", word), np.uint8))[0] == exp
    # :171-177 float decoders are exact
    for v in [0.0, -1.5, 3.25, 1e-5]:
        assert orc.decode_block(0, np.frombuffer(struct.pack("<f", v), np.uint8))[0] == struct.unpack("<f", struct.pack("<f", v))[0]
        assert orc.decode_block(28, np.frombuffer(struct.pack("<d", v), np.uint8))[0] == v
    # :112-124 Q2_K layout: scales[16] | qs[64] | d | dmin
    scales = bytes([0x21] + [0] * 15)
    qs = bytes([0xE4] * 64)
    blk = np.frombuffer(scales + qs + struct.pack("<ee", 0.5, 0.25), np.uint8)
    y = orc.decode_block(10, blk)
    assert y[0] == 0.5 * 1 * (0xE4 & 3) - 0.25 * 2
    assert y[16] == 0.0


def test_q3_k_decoder_against_reference_packing(orc, golden_dir):
    """Bytes packed by the reference's pack_q3_k_block (test_ggml_decoders.py:92-108)
    decode to d*(code-32)*(level-4): a closed form independent of the decoder."""
    z = np.load(golden_dir / "k_quant_vectors.npz")
    codes, levels = z["q3pack_codes"], z["q3pack_levels"]
    y = orc.decode_block(11, z["q3pack_bytes"])
    exp = [0.03125 * (int(codes[g]) - 32) * (int(levels[16 * g + i]) - 4) for g in range(16) for i in range(16)]
    assert list(y) == exp


def test_q4_k_and_q6_k_closed_forms(orc):
    """Hand-built blocks with every code distinct: value == d*sc*q - dmin*m (Q4_K),
    d*sc*(q-32) (Q6_K), with the GGML element order written out independently."""
    rng = np.random.default_rng(5)
    # Q4_K: scales j<4 plain 6-bit; j>=4 split (pyrite/kernels/native.c:52-60)
    sc = rng.integers(0, 64, 8)
    mn = rng.integers(0, 64, 8)
    s = np.zeros(12, np.int64)
    for j in range(8):
        if j < 4:
            s[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
            s[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        else:
            s[j + 4] = (sc[j] & 15) | ((mn[j] & 15) << 4)
    codes = rng.integers(0, 16, 256)
    qs = np.zeros(128, np.int64)
    for c in range(4):
        for l in range(32):
            qs[32 * c + l] = codes[64 * c + l] | (codes[64 * c + 32 + l] << 4)
    blk = np.frombuffer(struct.pack("<ee", 0.125, 0.0625), np.uint8).tolist() + s.tolist() + qs.tolist()
    y = orc.decode_block(12, np.array(blk, np.uint8))
    for e in range(256):
        j = e // 32
        assert y[e] == 0.125 * sc[j] * codes[e] - 0.0625 * mn[j]
    # Q6_K: element e = 128h + 32g + l; 4-bit part in ql, 2-bit part in qh
    q = rng.integers(0, 64, 256)
    scales = rng.integers(-128, 128, 16)
    ql = np.zeros(128, np.int64)
    qh = np.zeros(64, np.int64)
    for e in range(256):
        h, g, l = e // 128, (e // 32) % 4, e % 32
        byte = 64 * h + l + (32 if g in (1, 3) else 0)
        ql[byte] |= (q[e] & 15) << (4 if g >= 2 else 0)
        qh[32 * h + l] |= (q[e] >> 4) << (2 * g)
    blk = ql.tolist() + qh.tolist() + (scales & 0xFF).tolist() + list(struct.pack("<e", 0.25))
    y = orc.decode_block(14, np.array(blk, np.uint8))
    for e in range(256):
        h, g, l = e // 128, (e // 32) % 4, e % 32
        assert y[e] == 0.25 * scales[8 * h + 2 * g + l // 16] * (q[e] - 32)


# ------------------------------------------------------------------ invariants
@pytest.mark.parametrize("type_id", sorted(TYPES), ids=lambda t: TYPES[t][0])
def test_invariants(orc, type_id):
    name, bs, bpb = TYPES[type_id]
    rows, cols = 6, 512
    zero = np.zeros(rows * row_bytes(type_id, cols), np.uint8)
    assert not np.any(orc.dequantize_rows(type_id, zero, rows, cols))
    payload = lcg_payload(type_id, rows, cols, seed=99)
    rng = np.random.default_rng(type_id)
    x1, x2 = rng.standard_normal(cols), rng.standard_normal(cols)
    full = orc.matvec(type_id, payload, x1, rows, cols)
    # rows are independent: a sub-range call equals the slice of the full call
    rb = row_bytes(type_id, cols)
    part = orc.matvec(type_id, payload[2 * rb:5 * rb], x1, 3, cols)
    assert np.array_equal(_bits(part), _bits(full[2:5]))
    # linear in x (to rounding) and equal to an independent numpy contraction
    w = orc.dequantize_rows(type_id, payload, rows, cols).reshape(rows, cols)
    if np.all(np.isfinite(w)):
        scale = np.abs(w).sum(1) * (np.abs(x1) + np.abs(x2)).max() + 1e-300
        lin = orc.matvec(type_id, payload, x1 + x2, rows, cols) - full - orc.matvec(type_id, payload, x2, rows, cols)
        assert np.all(np.abs(lin) <= 1e-12 * scale)
        assert np.all(np.abs(full - w @ x1) <= 1e-12 * scale)


def test_expert_slice_equals_full_decode_slice(orc):
    """pyrite/qwen3_moe.py:364-398: expert e of a stacked tensor starts at
    e * (rows*cols/bs) * bpb and decodes to the same values as the full tensor."""
    for t in (12, 14, 8):
        n_exp, rows, cols = 4, 8, 512
        stack = lcg_payload(t, n_exp * rows, cols, seed=3)
        full = orc.dequantize_rows(t, stack, n_exp * rows, cols)
        per = rows * row_bytes(t, cols)
        for e in range(n_exp):
            part = orc.dequantize_rows(t, stack[e * per:(e + 1) * per], rows, cols)
            assert np.array_equal(_bits(part), _bits(full[e * rows * cols:(e + 1) * rows * cols]))


# ------------------------------------------------------------------ fp16
def test_half_to_double_exhaustive(orc):
    words = np.arange(65536, dtype=np.uint16)
    exp = words.view(np.float16).astype(np.float64)
    got = np.array([orc.half_to_double(int(w)) for w in words])
    nan = np.isnan(exp)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(_bits(got[~nan]), _bits(exp[~nan]))


def test_double_to_half_rounds_to_nearest_even(orc):
    rng = np.random.default_rng(11)
    vals = np.concatenate([
        rng.standard_normal(3000) * 10.0 ** rng.integers(-9, 5, 3000),
        # exact ties between neighbouring halves, normal and subnormal
        (np.arange(0, 2000, dtype=np.float64) + 0.5) * 2.0 ** -24,
        (np.arange(1024, 2047, dtype=np.float64) + 0.5) * 2.0 ** -10,
        np.array([65504.0, 65519.99, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 0.0, -0.0]),
    ])
    for v in vals:
        h, ovf = orc.double_to_half(float(v))
        ref = np.array([v], dtype=np.float64).astype(np.float16)
        assert not ovf
        assert h == int(ref.view(np.uint16)[0]), v
    assert orc.double_to_half(65520.0)[1] is True


# ------------------------------------------------------------------ quantizers
@pytest.mark.parametrize("case", ["sincos", "normal", "wide", "pos", "flatgroup"])
@pytest.mark.parametrize("type_id", [10, 11, 12, 13, 14])
def test_k_quant_encoders_match_reference_bytes(orc, golden_dir, case, type_id):
    z = np.load(golden_dir / "k_quant_vectors.npz")
    got = orc.quantize(type_id, z[f"{case}_values"])
    assert np.array_equal(got, z[f"{case}_t{type_id}"])


def test_q8_0_and_q4_0_encoder_known_answers(orc):
    # Q8_0: d = amax/127, codes round half away from zero (build_vocab_fixture.py:45-66)
    d = 127.0 / 127.0
    v = np.array([127.0, -127.0, 0.5, -0.5, 1.49, 2.5, -2.5, 0.0] + [3.0] * 24)
    b = orc.quantize(8, v)
    assert struct.unpack("<e", bytes(b[:2]))[0] == d
    codes = b[2:].view(np.int8)
    assert list(codes[:8]) == [127, -127, 1, -1, 1, 3, -3, 0]
    # Q4_0: d = best/-8 with best the first value of largest magnitude; code = trunc(v/d + 8.5)
    v = np.zeros(32)
    v[3], v[7] = -8.0, 8.0  # first max-magnitude is -8 -> d = 1.0
    v[0], v[16], v[1] = 1.0, -0.5, 7.4
    b = orc.quantize(2, v)
    assert struct.unpack("<e", bytes(b[:2]))[0] == 1.0
    qs = b[2:]
    assert qs[0] & 15 == 9 and qs[0] >> 4 == 8  # v[16] = -0.5 -> trunc(8.0) = 8
    assert qs[3] & 15 == 0 and qs[7] & 15 == 15 and qs[1] & 15 == 15


@pytest.mark.parametrize("type_id", [3, 6, 7, 9, 20, 23, 2, 8, 12, 13, 14, 10, 11])
def test_encoders_round_trip(orc, type_id):
    """Decode(encode(w)) stays within the type's quantization step of w."""
    name, bs, bpb = TYPES[type_id]
    w = orc.normal(4242 + type_id, 4096, 0.0, 0.02).astype(np.float64)
    payload = orc.quantize(type_id, w)
    assert payload.size == 4096 // bs * bpb
    y = orc.dequantize_rows(type_id, payload, 1, 4096)
    amax = np.abs(w).reshape(-1, 32).max(1).repeat(32)
    rel = {2: 0.16, 3: 0.08, 6: 0.08, 7: 0.04, 8: 0.01, 9: 0.01, 20: 0.16, 23: 0.2,
           12: 0.2, 13: 0.1, 14: 0.05, 10: 0.7, 11: 0.6}[type_id]
    assert np.all(np.abs(y - w) <= rel * amax + 1e-6)
    corr = np.corrcoef(y, w)[0, 1]
    assert corr > {10: 0.8, 11: 0.8}.get(type_id, 0.95)


# ------------------------------------------------------------------ routing math
def test_softmax_closed_forms(orc):
    p = orc.softmax(np.array([0.3, -1.2, 2.0, 0.0]))
    assert abs(p.sum() - 1.0) < 1e-15
    a, b = 0.7, -0.4
    two = orc.softmax(np.array([a, b]))
    assert abs(two[0] - 1.0 / (1.0 + math.exp(b - a))) < 1e-15
    assert np.all(orc.softmax(np.full(7, 3.3)) == 1.0 / 7)
    shifted = orc.softmax(np.array([0.3, -1.2, 2.0, 0.0]) + 100.0)
    assert np.allclose(shifted, p, rtol=1e-13)


def test_silu_closed_forms(orc):
    assert orc.silu(0.0) == 0.0
    assert orc.silu(-60.0) == 0.0 and orc.silu(-60.5) == 0.0
    assert orc.silu(-59.9) != 0.0
    for v in [0.1, 1.7, 8.0, 33.0]:
        assert abs((orc.silu(v) - orc.silu(-v)) - v) <= 1e-14 * max(1.0, v)
    assert abs(orc.silu(1.0) - 1.0 / (1.0 + math.exp(-1.0))) < 1e-16


def test_argmax_first_index_on_ties(orc):
    assert orc.argmax_first(np.array([1.0, 3.0, 3.0, 2.0])) == 1
    assert orc.argmax_first(np.array([-1.0])) == 0
    assert orc.argmax_first(np.array([0.0, -0.0, 0.0])) == 0


def test_rms_norm_closed_form(orc):
    x = np.array([3.0, 4.0])
    y = orc.rms_norm(x, eps=0.0)
    assert np.allclose(y, x / math.sqrt(12.5), rtol=1e-15)


@pytest.mark.parametrize("seed", range(40))
def test_routing_order_properties(orc, seed):
    """Brute force over small expert counts with forced ties: the k chosen ids
    are exactly the largest probabilities, ties broken by the lower expert id
    (pyrite/executor.py:765-767), in that order; renormalised weights sum to 1."""
    rng = np.random.default_rng(seed)
    n = int(rng.integers(2, 9))
    k = int(rng.integers(1, n + 1))
    logits = rng.integers(-3, 4, n).astype(np.float64) * 0.5  # many exact ties
    ids, w, probs = orc.route(logits, k, norm_topk_prob=True)
    order = sorted(range(n), key=lambda e: (-probs[e], e))
    chosen = list(ids)
    assert len(set(chosen)) == k
    # every unchosen expert is beaten by (or tied with and later than) each chosen one
    for e in set(range(n)) - set(chosen):
        for c in chosen:
            assert probs[c] > probs[e] or (probs[c] == probs[e] and c < e)
    # chosen order is descending probability, ties by id
    for a, b in zip(chosen, chosen[1:]):
        assert probs[a] > probs[b] or (probs[a] == probs[b] and a < b)
    assert chosen == order[:k]
    assert abs(w.sum() - 1.0) < 1e-15
    ids2, w2, _ = orc.route(logits, k, norm_topk_prob=False, scale=2.5)
    assert list(ids2) == chosen
    assert np.allclose(w2, probs[chosen] * 2.5, rtol=1e-15)


def test_moe_ffn_composition(orc):
    """The oracle MoE FFN equals an independent numpy composition of the
    dequantized experts (different summation order, so 1e-12 relative)."""
    E, H, I, k = 8, 256, 512, 3
    router = orc.normal(1, E * H, 0.0, 0.02).view(np.uint8).copy()
    gate = orc.quantize(12, orc.normal(2, E * I * H, 0.0, 0.02).astype(np.float64))
    up = orc.quantize(12, orc.normal(3, E * I * H, 0.0, 0.02).astype(np.float64))
    down = orc.quantize(14, orc.normal(4, E * H * I, 0.0, 0.02).astype(np.float64))
    x = orc.normal(5, H).astype(np.float64)
    out, ids, w, logits = orc.moe_ffn(router, 0, gate, 12, up, 12, down, 14, E, H, I, k, x)
    R = router.view("<f4").astype(np.float64).reshape(E, H)
    assert np.allclose(logits, R @ x, rtol=1e-12, atol=1e-14)
    G = orc.dequantize_rows(12, gate, E * I, H).reshape(E, I, H)
    U = orc.dequantize_rows(12, up, E * I, H).reshape(E, I, H)
    D = orc.dequantize_rows(14, down, E * H, I).reshape(E, H, I)
    ref = np.zeros(H)
    for e, we in zip(ids, w):
        g, u = G[e] @ x, U[e] @ x
        act = g / (1.0 + np.exp(-g)) * u
        ref += we * (D[e] @ act)
    assert np.allclose(out, ref, rtol=1e-10, atol=1e-12)


def test_generator_statistics(orc):
    z = orc.normal(123, 200000, 0.0, 1.0).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    assert np.array_equal(orc.normal(123, 10), orc.normal(123, 10))
    assert not np.array_equal(orc.normal(123, 10), orc.normal(124, 10))
