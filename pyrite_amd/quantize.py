"""Vectorised GGML block encoders (numpy) for preparing device-resident weights.

The K-quant encoders follow the reference's fixture quantizers
(tests/k_quant.py:61-285: naive min/max scale selection with the exact ggml
packing, Python round() = round-half-even, fp16 via IEEE round-to-nearest-even
with a +-65504 clamp); Q8_0 and Q4_0 follow scripts/build_vocab_fixture.py:45-89
(round half away from zero; truncation of v/d + 8.5).  The reference has no
encoder for Q4_1, Q5_0, Q5_1, Q8_1, IQ4_NL and IQ4_XS; those below are naive
byte-valid encoders of this package.  All arithmetic is float64 in the same
order as those algorithms, so the bytes are identical to a scalar evaluation.
"""
from __future__ import annotations

import numpy as np

from .ggml_types import spec

IQ4_VALUES = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], dtype=np.float64)


def _f16(v: np.ndarray) -> np.ndarray:
    """float64 -> binary16 (round to nearest even) after a +-65504 clamp, as float64."""
    return np.clip(v, -65504.0, 65504.0).astype(np.float16).astype(np.float64)


def _f16_bytes(v: np.ndarray) -> np.ndarray:
    return np.clip(v, -65504.0, 65504.0).astype("<f2").view(np.uint8).reshape(*v.shape, 2)


def _f16_bytes_strict(v: np.ndarray) -> np.ndarray:
    h = np.asarray(v, dtype=np.float64).astype("<f2")
    if not np.all(np.isfinite(h)):
        raise OverflowError("value does not fit binary16")
    return h.view(np.uint8).reshape(*np.shape(v), 2)


def _safe_div(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    with np.errstate(divide="ignore", invalid="ignore"):
        return np.where(b != 0, a / np.where(b != 0, b, 1.0), 0.0)


def _pack_k4(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """8 (scale, min) 6-bit pairs -> 12 bytes, per block (tests/k_quant.py:35-49)."""
    sc = np.clip(sc, 0, 63).astype(np.int64)
    mn = np.clip(mn, 0, 63).astype(np.int64)
    s = np.zeros(sc.shape[:-1] + (12,), dtype=np.int64)
    for j in range(8):
        if j < 4:
            s[..., j] |= sc[..., j]
            s[..., j + 4] |= mn[..., j]
        else:
            s[..., j + 4] = (sc[..., j] & 15) | ((mn[..., j] & 15) << 4)
            s[..., j - 4] |= (sc[..., j] >> 4) << 6
            s[..., j] |= (mn[..., j] >> 4) << 6
    return s


def _unpack_k4(s: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    sc = np.zeros(s.shape[:-1] + (8,), dtype=np.int64)
    mn = np.zeros_like(sc)
    for j in range(8):
        if j < 4:
            sc[..., j] = s[..., j] & 63
            mn[..., j] = s[..., j + 4] & 63
        else:
            sc[..., j] = (s[..., j + 4] & 15) | ((s[..., j - 4] >> 6) << 4)
            mn[..., j] = (s[..., j + 4] >> 4) | ((s[..., j] >> 6) << 4)
    return sc, mn


def _q45_k(b: np.ndarray, five: bool) -> np.ndarray:
    top = 31.0 if five else 15.0
    g = b.reshape(-1, 8, 32)
    lo, hi = g.min(axis=2), g.max(axis=2)
    scales_f = np.where(hi > lo, (hi - lo) / top, 0.0)
    mins_f = np.where(hi > lo, -lo, 0.0)
    max_scale, max_min = scales_f.max(axis=1), mins_f.max(axis=1)
    inv_scale = _safe_div(np.full_like(max_scale, 63.0), max_scale) * (max_scale > 0)
    inv_min = _safe_div(np.full_like(max_min, 63.0), max_min) * (max_min > 0)
    sc = np.rint(inv_scale[:, None] * scales_f)
    mn = np.rint(inv_min[:, None] * mins_f)
    packed = _pack_k4(sc, mn)
    d = np.where(max_scale > 0, _f16(max_scale / 63.0), 0.0)
    dmin = np.where(max_min > 0, _f16(max_min / 63.0), 0.0)
    usc, umn = _unpack_k4(packed)
    step = d[:, None] * usc
    offset = dmin[:, None] * umn
    lv = np.rint(_safe_div(g + offset[:, :, None], np.broadcast_to(step[:, :, None], g.shape)))
    lv = np.where(step[:, :, None] != 0, np.clip(lv, 0, top), 0).astype(np.int64).reshape(-1, 256)
    n = b.shape[0]
    head = np.concatenate([
        _f16_bytes(np.where(max_scale > 0, max_scale / 63.0, 0.0)),
        _f16_bytes(np.where(max_min > 0, max_min / 63.0, 0.0)),
        packed.astype(np.uint8),
    ], axis=1)
    chunks = lv.reshape(n, 4, 2, 32)  # [c][low/high][l]
    if not five:
        qs = (chunks[:, :, 0, :] | (chunks[:, :, 1, :] << 4)).reshape(n, 128)
        return np.concatenate([head, qs.astype(np.uint8)], axis=1)
    low, high = chunks[:, :, 0, :], chunks[:, :, 1, :]
    qh = np.zeros((n, 32), dtype=np.int64)
    for c in range(4):
        qh |= ((low[:, c, :] > 15).astype(np.int64) << (2 * c)) | ((high[:, c, :] > 15).astype(np.int64) << (2 * c + 1))
    ql = ((low & 15) | ((high & 15) << 4)).reshape(n, 128)
    return np.concatenate([head, qh.astype(np.uint8), ql.astype(np.uint8)], axis=1)


def _q6_k(b: np.ndarray) -> np.ndarray:
    n = b.shape[0]
    peak = np.abs(b).max(axis=1)
    d = _f16(peak / (64.0 * 31.0))
    step = d * 64.0
    if np.any((peak > 0) & (step == 0)):
        raise OverflowError("Q6_K step underflows to zero")
    lv = np.clip(np.rint(_safe_div(b, np.broadcast_to(step[:, None], b.shape))) + 32, 0, 63).astype(np.int64)
    q = lv.reshape(n, 2, 4, 32)  # [h][g][l]
    ql = np.zeros((n, 2, 64), dtype=np.int64)
    ql[:, :, :32] = (q[:, :, 0] & 15) | ((q[:, :, 2] & 15) << 4)
    ql[:, :, 32:] = (q[:, :, 1] & 15) | ((q[:, :, 3] & 15) << 4)
    qh = (q[:, :, 0] >> 4) | ((q[:, :, 1] >> 4) << 2) | ((q[:, :, 2] >> 4) << 4) | ((q[:, :, 3] >> 4) << 6)
    out = np.concatenate([ql.reshape(n, 128).astype(np.uint8), qh.reshape(n, 64).astype(np.uint8),
                          np.full((n, 16), 64, dtype=np.uint8), _f16_bytes(peak / (64.0 * 31.0))], axis=1)
    out[peak <= 0] = 0
    return out


def _q2_k(b: np.ndarray) -> np.ndarray:
    n = b.shape[0]
    g = b.reshape(n, 16, 16)
    lo, hi = g.min(axis=2), g.max(axis=2)
    rng = hi - lo
    max_range = rng.max(axis=1)
    max_neg = np.where(lo < 0.0, -lo, -np.inf).max(axis=1)
    max_neg = np.where(np.isfinite(max_neg), max_neg, 0.0)
    d = np.where(max_range > 0, _f16(max_range / 45.0), 0.0)
    dmin = np.where(max_neg > 0, _f16(max_neg / 15.0), 0.0)
    sc = np.where(rng > 0, 15, 0)
    mn = np.where((dmin[:, None] > 0) & (lo < 0.0), np.rint(_safe_div(-lo, np.broadcast_to(dmin[:, None], lo.shape))), 0)
    mn = np.clip(mn, 0, 15).astype(np.int64)
    step = d[:, None] * sc
    offset = dmin[:, None] * mn
    code = np.rint(_safe_div(g + offset[:, :, None], np.broadcast_to(step[:, :, None], g.shape)))
    code = np.where(step[:, :, None] != 0, np.clip(code, 0, 3), 0).astype(np.int64)
    quants = np.zeros((n, 64), dtype=np.int64)
    for grp in range(16):
        half, shift, base = grp // 8, 2 * ((grp % 8) // 2), (grp // 8) * 32 + (grp % 2) * 16
        quants[:, base:base + 16] |= code[:, grp, :] << shift
        _ = half
    scales = ((mn << 4) | sc).astype(np.uint8)
    return np.concatenate([scales, quants.astype(np.uint8),
                           _f16_bytes(np.where(max_range > 0, max_range / 45.0, 0.0)),
                           _f16_bytes(np.where(max_neg > 0, max_neg / 15.0, 0.0))], axis=1)


def _q3_k(b: np.ndarray) -> np.ndarray:
    n = b.shape[0]
    g = b.reshape(n, 16, 16)
    lo, hi = g.min(axis=2), g.max(axis=2)
    gs = np.where(hi > lo, (hi - lo) / 7.0, 0.0)
    peak = gs.max(axis=1)
    d_all = np.where(peak > 0, _f16(peak / 31.0), 0.0)
    codes = np.where(d_all[:, None] > 0,
                     np.clip(32 + np.rint(_safe_div(gs, np.broadcast_to(d_all[:, None], gs.shape))), 0, 63), 32)
    codes = codes.astype(np.int64)
    span = hi - lo
    lv = np.rint(_safe_div(g - lo[:, :, None], np.broadcast_to(span[:, :, None], g.shape)) * 7.0)
    lv = np.where(span[:, :, None] > 0, np.clip(lv, 0, 7), 4).astype(np.int64).reshape(n, 256)
    sc = np.zeros((n, 12), dtype=np.int64)
    for j in range(16):
        low = codes[:, j] & 15
        if j < 8:
            sc[:, j] = low
        else:
            sc[:, j - 8] |= low << 4
        sc[:, 8 + j % 4] |= (codes[:, j] >> 4) << (2 * (j // 4))
    q = np.where(lv > 3, lv - 4, lv)
    hmask = np.zeros((n, 32), dtype=np.int64)
    for j in range(8):
        hmask |= (lv[:, 32 * j:32 * j + 32] > 3).astype(np.int64) << j
    qr = q.reshape(n, 2, 4, 32)
    qs = (qr[:, :, 0] | (qr[:, :, 1] << 2) | (qr[:, :, 2] << 4) | (qr[:, :, 3] << 6)).reshape(n, 64)
    return np.concatenate([hmask.astype(np.uint8), qs.astype(np.uint8), sc.astype(np.uint8),
                           _f16_bytes_strict(np.where(peak > 0, peak / 31.0, 0.0))], axis=1)


def _q8_0(b: np.ndarray) -> np.ndarray:
    amax = np.abs(b).max(axis=1)
    d = amax / 127.0
    inv = _safe_div(np.ones_like(d), d)
    v = b * inv[:, None]
    q = np.where(v >= 0, np.trunc(v + 0.5), -np.trunc(-v + 0.5))
    q = np.clip(q, -127, 127).astype(np.int64) & 0xFF
    return np.concatenate([_f16_bytes_strict(d), q.astype(np.uint8)], axis=1)


def _first_absmax(b: np.ndarray) -> np.ndarray:
    """The first value of largest magnitude per block (strict > keeps the first)."""
    idx = np.argmax(np.abs(b), axis=1)
    return np.take_along_axis(b, idx[:, None], axis=1)[:, 0]


def _q4_0(b: np.ndarray) -> np.ndarray:
    best = _first_absmax(b)
    d = best / -8.0
    inv = _safe_div(np.ones_like(d), d)
    q = np.clip(np.trunc(b * inv[:, None] + 8.5), 0, 15).astype(np.int64)
    qs = q[:, :16] | (q[:, 16:] << 4)
    return np.concatenate([_f16_bytes_strict(d), qs.astype(np.uint8)], axis=1)


def _q41_q51(b: np.ndarray, five: bool) -> np.ndarray:
    top = 31.0 if five else 15.0
    lo, hi = b.min(axis=1), b.max(axis=1)
    d = (hi - lo) / top
    dq, mq = _f16(d), _f16(lo)
    q = np.where(dq[:, None] > 0, np.clip(np.rint(_safe_div(b - mq[:, None], np.broadcast_to(dq[:, None], b.shape))), 0, top), 0)
    q = q.astype(np.int64)
    qs = (q[:, :16] & 15) | ((q[:, 16:] & 15) << 4)
    parts = [_f16_bytes(d), _f16_bytes(lo)]
    if five:
        qh = ((q >> 4) & 1) << np.arange(32)
        parts.append(qh.sum(axis=1).astype("<u4").view(np.uint8).reshape(-1, 4))
    parts.append(qs.astype(np.uint8))
    return np.concatenate(parts, axis=1)


def _q5_0(b: np.ndarray) -> np.ndarray:
    best = _first_absmax(b)
    d = _f16(best / -16.0)
    q = np.where(d[:, None] != 0, np.clip(np.rint(_safe_div(b, np.broadcast_to(d[:, None], b.shape))) + 16, 0, 31), 16)
    q = q.astype(np.int64)
    qh = (((q >> 4) & 1) << np.arange(32)).sum(axis=1).astype("<u4").view(np.uint8).reshape(-1, 4)
    qs = (q[:, :16] & 15) | ((q[:, 16:] & 15) << 4)
    return np.concatenate([_f16_bytes(best / -16.0), qh, qs.astype(np.uint8)], axis=1)


def _q8_1(b: np.ndarray) -> np.ndarray:
    amax = np.abs(b).max(axis=1)
    d = _f16(amax / 127.0)
    q = np.where(d[:, None] != 0, np.clip(np.rint(_safe_div(b, np.broadcast_to(d[:, None], b.shape))), -127, 127), 0)
    q = q.astype(np.int64)
    s = d * q.sum(axis=1)
    return np.concatenate([_f16_bytes(d), _f16_bytes(s), (q & 0xFF).astype(np.uint8)], axis=1)


def _iq4_nearest(t: np.ndarray) -> np.ndarray:
    """Index of the codebook entry nearest to t; ties keep the lower index.

    The nearest entry is one of the two that bracket t, so only those two
    distances are compared (with the same rounded |t - K| values a scan over
    all sixteen entries would compare)."""
    lo = np.clip(np.searchsorted(IQ4_VALUES, t, side="left") - 1, 0, 14)
    e0 = np.abs(t - IQ4_VALUES[lo])
    e1 = np.abs(t - IQ4_VALUES[lo + 1])
    return np.where(e1 < e0, lo + 1, lo)


def _iq4_nl(b: np.ndarray) -> np.ndarray:
    best = _first_absmax(b)
    d = _f16(best / IQ4_VALUES[0])
    idx = np.where(d[:, None] != 0, _iq4_nearest(_safe_div(b, np.broadcast_to(d[:, None], b.shape))), 8)
    qs = idx[:, :16] | (idx[:, 16:] << 4)
    return np.concatenate([_f16_bytes(best / IQ4_VALUES[0]), qs.astype(np.uint8)], axis=1)


def _iq4_xs(b: np.ndarray) -> np.ndarray:
    n = b.shape[0]
    g = b.reshape(n, 8, 32)
    idx = np.argmax(np.abs(g), axis=2)
    best = np.take_along_axis(g, idx[:, :, None], axis=2)[:, :, 0]
    sub = best / IQ4_VALUES[0]
    sidx = np.argmax(np.abs(sub), axis=1)
    maxs = np.take_along_axis(sub, sidx[:, None], axis=1)[:, 0]
    maxs = np.where(np.abs(maxs) > 0, maxs, 0.0)  # an all-zero block keeps +0.0
    d = _f16(-maxs / 32.0)
    ls = np.where(d[:, None] != 0, np.clip(np.rint(_safe_div(sub, np.broadcast_to(d[:, None], sub.shape))), -32, 31), 0)
    ls = ls.astype(np.int64)
    code = ls + 32
    sl = np.zeros((n, 4), dtype=np.int64)
    for ib in range(8):
        sl[:, ib // 2] |= (code[:, ib] & 15) << (4 * (ib & 1))
    sh = (((code >> 4) & 3) << (2 * np.arange(8))).sum(axis=1)
    dl = d[:, None] * ls
    q = np.where(dl[:, :, None] != 0, _iq4_nearest(_safe_div(g, np.broadcast_to(dl[:, :, None], g.shape))), 8)
    qs = (q[:, :, :16] | (q[:, :, 16:] << 4)).reshape(n, 128)
    return np.concatenate([_f16_bytes(-maxs / 32.0), sh.astype("<u2").view(np.uint8).reshape(n, 2),
                           sl.astype(np.uint8), qs.astype(np.uint8)], axis=1)


def quantize(type_id: int, values: np.ndarray) -> np.ndarray:
    """Encode float values (any shape, flattened row-major) into GGML blocks of ``type_id``."""
    t = spec(type_id)
    v = np.ascontiguousarray(values, dtype=np.float64).ravel()
    if v.size % t.block_size:
        raise ValueError(f"{t.name} needs a multiple of {t.block_size} values")
    if type_id == 0:
        return v.astype("<f4").view(np.uint8).copy()
    if type_id == 1:
        return _f16_bytes_strict(v).ravel().copy()
    if type_id == 30:
        f = v.astype("<f4").view("<u4").astype(np.uint64)
        r = ((f + 0x7FFF + ((f >> 16) & 1)) >> 16).astype("<u2")
        return r.view(np.uint8).copy()
    if type_id == 28:
        return v.astype("<f8").view(np.uint8).copy()
    if type_id in (24, 25, 26, 27):
        dt = {24: "<i1", 25: "<i2", 26: "<i4", 27: "<i8"}[type_id]
        info = np.iinfo(dt)
        return np.clip(np.rint(v), info.min, info.max).astype(dt).view(np.uint8).copy()
    b = v.reshape(-1, t.block_size)
    enc = {
        2: _q4_0, 3: lambda x: _q41_q51(x, False), 6: _q5_0, 7: lambda x: _q41_q51(x, True), 8: _q8_0,
        9: _q8_1, 10: _q2_k, 11: _q3_k, 12: lambda x: _q45_k(x, False), 13: lambda x: _q45_k(x, True),
        14: _q6_k, 20: _iq4_nl, 23: _iq4_xs,
    }[type_id]
    out = enc(b)
    assert out.shape == (b.shape[0], t.bytes_per_block), (type_id, out.shape)
    return np.ascontiguousarray(out, dtype=np.uint8).ravel()
