/*
 * CPU oracle for the fused GGML dequantize x matvec hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the reference the HIP kernels are compared against,
 * never the thing measured or shipped.  Build flags (oracle/Makefile) keep
 * IEEE double semantics: no fast-math and no FMA contraction, so every
 * rounding happens where the C source says, exactly as in the reference build
 * (`cc -O3 -std=c99`, pyrite/kernels/native.py:113, which is ISO mode and
 * therefore contraction-free).
 *
 * Decoders follow the GGML block layouts that the reference decodes in
 * pyrite/kernels/native.c; each one cites the lines it restates.  Products of
 * a half scale and small integers are exact in double, so the only roundings
 * are the ones the reference also performs (one add/sub for the types with a
 * minimum or offset).
 */
#include "pyrite_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ geometry */

typedef struct {
    int id;
    unsigned block;     /* elements per block */
    unsigned bytes;     /* bytes per block */
} type_info;

/* Same ids and order as the reference table (pyrite/kernels/native.c:451-473);
 * pyrite_native_types reports ids in table order, so the order is part of the
 * observable contract. */
static const type_info TYPES[] = {
    {0, 1, 4},     {1, 1, 2},     {2, 32, 18},   {3, 32, 20},   {6, 32, 22},
    {7, 32, 24},   {8, 32, 34},   {9, 32, 36},   {10, 256, 84}, {11, 256, 110},
    {12, 256, 144}, {13, 256, 176}, {14, 256, 210}, {20, 32, 18}, {23, 256, 136},
    {24, 1, 1},    {25, 1, 2},    {26, 1, 4},    {27, 1, 8},    {28, 1, 8},
    {30, 1, 2},
};
#define N_TYPES (sizeof(TYPES) / sizeof(TYPES[0]))

static const type_info *find_type(int id) {
    for (size_t i = 0; i < N_TYPES; ++i)
        if (TYPES[i].id == id) return &TYPES[i];
    return NULL;
}

int oracle_native_types(int *ids, size_t capacity) {
    /* pyrite/kernels/native.c:484-494 */
    if (ids == NULL) return (int)N_TYPES;
    size_t n = capacity < N_TYPES ? capacity : N_TYPES;
    for (size_t i = 0; i < n; ++i) ids[i] = TYPES[i].id;
    return (int)n;
}

int oracle_type_geometry(int type_id, size_t *block_size, size_t *bytes_per_block) {
    const type_info *t = find_type(type_id);
    if (!t) return 0;
    *block_size = t->block;
    *bytes_per_block = t->bytes;
    return 1;
}

/* ------------------------------------------------------------------ scalars */

static uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t le32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* binary16 -> binary32 widening, then to double (pyrite/kernels/native.c:23-50).
 * Normal, infinite and NaN halves widen by re-biasing the exponent; subnormal
 * halves are mant * 2^-24, which is exact in binary32. */
static float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 31u;
    uint32_t m = h & 1023u;
    uint32_t bits;
    if (e == 0) {
        float mag = ldexpf((float)m, -24);
        return sign ? -mag : mag;
    }
    if (e == 31) bits = sign | 0x7f800000u | (m << 13);
    else bits = sign | ((e + 112u) << 23) | (m << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

double oracle_half_to_double(uint16_t h) { return (double)half_to_float(h); }

/* Round a double to binary16, ties to even, as CPython's struct '<e' does
 * (tests/k_quant.py:18-26 uses it for every stored scale). */
uint16_t oracle_double_to_half(double v, int *overflow) {
    if (overflow) *overflow = 0;
    uint16_t sign = signbit(v) ? 0x8000u : 0;
    double a = fabs(v);
    if (isnan(v)) return (uint16_t)(sign | 0x7e00u);
    if (isinf(v)) {
        if (overflow) *overflow = 1;
        return (uint16_t)(sign | 0x7c00u);
    }
    if (a == 0.0) return sign;
    int e;
    (void)frexp(a, &e);     /* a = f * 2^e, f in [0.5, 1) */
    int exp2 = e - 1;        /* a = (2f) * 2^exp2, 2f in [1, 2) */
    unsigned units;
    unsigned biased;
    double scaled;
    if (exp2 < -14) {
        /* subnormal: value in units of 2^-24 */
        scaled = ldexp(a, 24);
        biased = 0;
    } else {
        /* normal: 10 fraction bits below the leading one */
        scaled = ldexp(a, 10 - exp2);
        biased = (unsigned)(exp2 + 15);
    }
    units = (unsigned)scaled;            /* truncate */
    double rem = scaled - (double)units; /* exact: scaled < 2^11 */
    if (rem > 0.5 || (rem == 0.5 && (units & 1u))) ++units;
    if (biased == 0) {
        /* 1024 units of 2^-24 is the smallest normal, encoded as exponent 1 */
        return (uint16_t)(sign | units);
    }
    if (units >= 2048u) { /* mantissa carry */
        units >>= 1;
        ++biased;
    }
    if (biased >= 31u) {
        if (overflow) *overflow = 1;
        return (uint16_t)(sign | 0x7c00u);
    }
    return (uint16_t)(sign | (biased << 10) | (units & 1023u));
}

/* 6-bit (scale, min) pair j of a Q4_K/Q5_K super-block
 * (pyrite/kernels/native.c:52-60). */
static void k4_scale_min(const uint8_t *s, int j, int *sc, int *mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* Unpack the sixteen 6-bit Q3_K scale codes (stored as scale + 32) from 12
 * bytes: the low nibbles come from bytes 0..7 (low nibble for j<8, high for
 * j>=8) and the top two bits from bytes 8..11 (pyrite/kernels/native.c:134-143). */
static void q3k_scales(const uint8_t *s, int out[16]) {
    for (int j = 0; j < 16; ++j) {
        int low = (j < 8) ? (s[j] & 15) : (s[j - 8] >> 4);
        int high = (s[8 + (j & 3)] >> (2 * (j >> 2))) & 3;
        out[j] = low | (high << 4);
    }
}

/* kvalues_iq4nl, the IQ4 non-linear codebook (pyrite/kernels/native.c:347-349) */
static const int IQ4[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                            1,    13,   25,  38,  53,  69,  89,  113};

/* ------------------------------------------------------------------ decoders */

int oracle_decode_block(int type_id, const uint8_t *b, double *y) {
    switch (type_id) {
    case 0: { /* F32 (native.c:238-244) */
        float f;
        memcpy(&f, b, 4);
        y[0] = (double)f;
        return 0;
    }
    case 1: y[0] = oracle_half_to_double(le16(b)); return 0;          /* F16 (:250-252) */
    case 30: {                                                         /* BF16 (:254-259) */
        uint32_t bits = (uint32_t)le16(b) << 16;
        float f;
        memcpy(&f, &bits, 4);
        y[0] = (double)f;
        return 0;
    }
    case 28: memcpy(y, b, 8); return 0;                                /* F64 (:246-248) */
    case 24: y[0] = (double)(int8_t)b[0]; return 0;                    /* I8 (:261) */
    case 25: y[0] = (double)(int16_t)le16(b); return 0;                /* I16 (:263-265) */
    case 26: y[0] = (double)(int32_t)le32(b); return 0;                /* I32 (:267-271) */
    case 27: {                                                         /* I64 (:273-279) */
        uint64_t u = (uint64_t)le32(b) | ((uint64_t)le32(b + 4) << 32);
        y[0] = (double)(int64_t)u;
        return 0;
    }
    case 2: { /* Q4_0: d | qs[16]; element i low nibble, i+16 high (native.c:281-288) */
        double d = oracle_half_to_double(le16(b));
        for (int i = 0; i < 16; ++i) {
            y[i] = d * (double)((b[2 + i] & 15) - 8);
            y[i + 16] = d * (double)((b[2 + i] >> 4) - 8);
        }
        return 0;
    }
    case 3: { /* Q4_1: d | m | qs[16]; d*q + m (native.c:290-298) */
        double d = oracle_half_to_double(le16(b)), m = oracle_half_to_double(le16(b + 2));
        for (int i = 0; i < 16; ++i) {
            y[i] = d * (double)(b[4 + i] & 15) + m;
            y[i + 16] = d * (double)(b[4 + i] >> 4) + m;
        }
        return 0;
    }
    case 6: { /* Q5_0: d | qh u32 | qs[16]; fifth bit i and i+16 of qh (native.c:300-314) */
        double d = oracle_half_to_double(le16(b));
        uint32_t qh = le32(b + 2);
        for (int i = 0; i < 16; ++i) {
            int lo = (b[6 + i] & 15) | (int)(((qh >> i) & 1u) << 4);
            int hi = (b[6 + i] >> 4) | (int)(((qh >> (i + 16)) & 1u) << 4);
            y[i] = d * ((double)lo - 16.0);
            y[i + 16] = d * ((double)hi - 16.0);
        }
        return 0;
    }
    case 7: { /* Q5_1: d | m | qh | qs[16]; d*q5 + m (native.c:316-328) */
        double d = oracle_half_to_double(le16(b)), m = oracle_half_to_double(le16(b + 2));
        uint32_t qh = le32(b + 4);
        for (int i = 0; i < 16; ++i) {
            int lo = (b[8 + i] & 15) | (int)(((qh >> i) & 1u) << 4);
            int hi = (b[8 + i] >> 4) | (int)(((qh >> (i + 16)) & 1u) << 4);
            y[i] = d * (double)lo + m;
            y[i + 16] = d * (double)hi + m;
        }
        return 0;
    }
    case 8:   /* Q8_0: d | i8 qs[32] (native.c:330-336) */
    case 9: { /* Q8_1: d | s | i8 qs[32], s unused (native.c:338-344) */
        double d = oracle_half_to_double(le16(b));
        const uint8_t *qs = b + (type_id == 8 ? 2 : 4);
        for (int i = 0; i < 32; ++i) y[i] = d * (double)(int8_t)qs[i];
        return 0;
    }
    case 20: { /* IQ4_NL: d | qs[16]; d * K[nibble] (native.c:351-358) */
        double d = oracle_half_to_double(le16(b));
        for (int i = 0; i < 16; ++i) {
            y[i] = d * (double)IQ4[b[2 + i] & 15];
            y[i + 16] = d * (double)IQ4[b[2 + i] >> 4];
        }
        return 0;
    }
    case 23: { /* IQ4_XS: d | scales_h u16 | scales_l[4] | qs[128] (native.c:364-379) */
        double d = oracle_half_to_double(le16(b));
        unsigned sh = le16(b + 2);
        for (int ib = 0; ib < 8; ++ib) {
            int ls = ((b[4 + ib / 2] >> (4 * (ib & 1))) & 15) | (int)(((sh >> (2 * ib)) & 3u) << 4);
            double dl = d * ((double)ls - 32.0);
            const uint8_t *qs = b + 8 + 16 * ib;
            for (int j = 0; j < 16; ++j) {
                y[32 * ib + j] = dl * (double)IQ4[qs[j] & 15];
                y[32 * ib + j + 16] = dl * (double)IQ4[qs[j] >> 4];
            }
        }
        return 0;
    }
    case 10: { /* Q2_K: scales[16] | qs[64] | d | dmin (native.c:381-408) */
        double d = oracle_half_to_double(le16(b + 80)), dmin = oracle_half_to_double(le16(b + 82));
        /* element e: half h = e/128, shift group g = (e%128)/32, 16-run r = (e%32)/16;
         * code byte qs[32h + 16r + l], bits 2g..2g+1; scale byte 8h + 2g + r */
        for (int e = 0; e < 256; ++e) {
            int h = e >> 7, g = (e >> 5) & 3, r = (e >> 4) & 1, l = e & 15;
            uint8_t sc = b[8 * h + 2 * g + r];
            int q = (b[16 + 32 * h + 16 * r + l] >> (2 * g)) & 3;
            double dl = d * (double)(sc & 15);
            double ml = dmin * (double)(sc >> 4);
            y[e] = dl * (double)q - ml;
        }
        return 0;
    }
    case 11: { /* Q3_K: hmask[32] | qs[64] | scales[12] | d (native.c:129-171) */
        double d = oracle_half_to_double(le16(b + 108));
        int sc[16];
        q3k_scales(b + 96, sc);
        for (int e = 0; e < 256; ++e) {
            int h = e >> 7, g = (e >> 5) & 3, r = (e >> 4) & 1, l = e & 15;
            int low = (b[32 + 32 * h + 16 * r + l] >> (2 * g)) & 3;
            /* hmask bit (4h + g) of byte 16r + l; a clear bit subtracts 4 */
            int hbit = (b[16 * r + l] >> (4 * h + g)) & 1;
            int v = low - (hbit ? 0 : 4);
            double dl = d * ((double)sc[8 * h + 2 * g + r] - 32.0);
            y[e] = dl * (double)v;
        }
        return 0;
    }
    case 12:   /* Q4_K: d | dmin | scales[12] | qs[128] (native.c:173-197) */
    case 13: { /* Q5_K: d | dmin | scales[12] | qh[32] | qs[128] (native.c:410-437) */
        double d = oracle_half_to_double(le16(b)), dmin = oracle_half_to_double(le16(b + 2));
        const uint8_t *qs = b + (type_id == 12 ? 16 : 48);
        const uint8_t *qh = b + 16;
        for (int c = 0; c < 4; ++c) { /* 64-element chunk: low nibbles then high */
            for (int half = 0; half < 2; ++half) {
                int j = 2 * c + half, sc, mn;
                k4_scale_min(b + 4, j, &sc, &mn);
                double d1 = d * (double)sc, m1 = dmin * (double)mn;
                for (int l = 0; l < 32; ++l) {
                    int q = half ? (qs[32 * c + l] >> 4) : (qs[32 * c + l] & 15);
                    if (type_id == 13 && ((qh[l] >> j) & 1)) q += 16;
                    y[64 * c + 32 * half + l] = d1 * (double)q - m1;
                }
            }
        }
        return 0;
    }
    case 14: { /* Q6_K: ql[128] | qh[64] | i8 scales[16] | d (native.c:199-225) */
        double d = oracle_half_to_double(le16(b + 208));
        for (int e = 0; e < 256; ++e) {
            int h = e >> 7, g = (e >> 5) & 3, l = e & 31;
            /* g selects (ql offset, nibble): 0:(l,lo) 1:(l+32,lo) 2:(l,hi) 3:(l+32,hi) */
            uint8_t lq = b[64 * h + l + 32 * (g & 1)];
            int low = (g & 2) ? (lq >> 4) : (lq & 15);
            int high = (b[128 + 32 * h + l] >> (2 * g)) & 3;
            int q = (low | (high << 4)) - 32;
            int8_t s = (int8_t)b[192 + 8 * h + 2 * g + l / 16];
            y[e] = d * (double)s * (double)q;
        }
        return 0;
    }
    default:
        return -1;
    }
}

/* ------------------------------------------------------------------ C-ABI twins */

static int geometry(int type_id, size_t rows, size_t cols, size_t *row_bytes,
                    size_t *expected, const type_info **out) {
    /* pyrite/kernels/native.c:496-516 */
    const type_info *t = find_type(type_id);
    if (!t) return -1;
    if (rows == 0 || cols == 0 || cols % t->block != 0 || cols / t->block > SIZE_MAX / t->bytes)
        return -2;
    *row_bytes = (cols / t->block) * t->bytes;
    if (*row_bytes > SIZE_MAX / rows) return -2;
    *expected = *row_bytes * rows;
    *out = t;
    return 0;
}

int oracle_matvec(int type_id, const uint8_t *data, size_t data_len, const double *x,
                  double *out, size_t rows, size_t cols) {
    /* pyrite/kernels/native.c:518-555: per row, decode block by block and add
     * w*x into one double accumulator in column order. */
    size_t row_bytes = 0, expected = 0;
    const type_info *t = NULL;
    int g = geometry(type_id, rows, cols, &row_bytes, &expected, &t);
    if (g != 0) return g;
    if (!data || !x || !out || data_len != expected) return -3;
    double scratch[256];
    for (size_t r = 0; r < rows; ++r) {
        const uint8_t *row = data + r * row_bytes;
        double sum = 0.0;
        for (size_t c = 0; c < cols; c += t->block) {
            oracle_decode_block(type_id, row + (c / t->block) * t->bytes, scratch);
            for (size_t l = 0; l < t->block; ++l) sum += scratch[l] * x[c + l];
        }
        out[r] = sum;
    }
    return 0;
}

int oracle_dequantize_rows(int type_id, const uint8_t *data, size_t data_len, double *out,
                           size_t rows, size_t cols) {
    /* pyrite/kernels/native.c:557-576 */
    size_t row_bytes = 0, expected = 0;
    const type_info *t = NULL;
    int g = geometry(type_id, rows, cols, &row_bytes, &expected, &t);
    if (g != 0) return g;
    if (!data || !out || data_len != expected || cols > SIZE_MAX / rows) return -3;
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; c += t->block)
            oracle_decode_block(type_id, data + r * row_bytes + (c / t->block) * t->bytes,
                                out + r * cols + c);
    return 0;
}

/* ------------------------------------------------------------------ quantizers */

/* Python's round(): nearest, ties to even (the default FE_TONEAREST mode). */
static double py_round(double v) { return nearbyint(v); }
static long clampl(long v, long lo, long hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* _f16 of tests/k_quant.py:18-21: clamp to +-65504, then round to half */
static double f16_clamped(double v) {
    double c = v > 65504.0 ? 65504.0 : (v < -65504.0 ? -65504.0 : v);
    return oracle_half_to_double(oracle_double_to_half(c, NULL));
}
static void put16(uint8_t *p, uint16_t h) { p[0] = (uint8_t)h; p[1] = (uint8_t)(h >> 8); }
static void put_f16_clamped(uint8_t *p, double v) {
    double c = v > 65504.0 ? 65504.0 : (v < -65504.0 ? -65504.0 : v);
    put16(p, oracle_double_to_half(c, NULL));
}
/* struct.pack('<e', v) without clamping: fails where Python raises */
static int put_f16_strict(uint8_t *p, double v) {
    int ovf = 0;
    uint16_t h = oracle_double_to_half(v, &ovf);
    if (ovf) return -4;
    put16(p, h);
    return 0;
}

static double vmin(const double *v, int n) { double m = v[0]; for (int i = 1; i < n; ++i) if (v[i] < m) m = v[i]; return m; }
static double vmax(const double *v, int n) { double m = v[0]; for (int i = 1; i < n; ++i) if (v[i] > m) m = v[i]; return m; }

/* _pack_k4_scales, tests/k_quant.py:35-49 */
static void pack_k4(const long sc_in[8], const long mn_in[8], uint8_t s[12]) {
    memset(s, 0, 12);
    for (int j = 0; j < 8; ++j) {
        long sc = clampl(sc_in[j], 0, 63), mn = clampl(mn_in[j], 0, 63);
        if (j < 4) {
            s[j] = (uint8_t)sc;
            s[j + 4] = (uint8_t)mn;
        } else {
            s[j + 4] = (uint8_t)((sc & 15) | ((mn & 15) << 4));
            s[j - 4] |= (uint8_t)((sc >> 4) << 6);
            s[j] |= (uint8_t)((mn >> 4) << 6);
        }
    }
}

/* encode_q4_k / encode_q5_k, tests/k_quant.py:61-157 (levels = 15 or 31) */
static void enc_q45_k(const double *v, uint8_t *o, int five) {
    const double top = five ? 31.0 : 15.0;
    double sf[8], mf[8];
    for (int j = 0; j < 8; ++j) {
        double lo = vmin(v + 32 * j, 32), hi = vmax(v + 32 * j, 32);
        if (hi > lo) { sf[j] = (hi - lo) / top; mf[j] = -lo; }
        else { sf[j] = 0.0; mf[j] = 0.0; }
    }
    double max_scale = vmax(sf, 8), max_min = vmax(mf, 8);
    double inv_scale = max_scale > 0 ? 63.0 / max_scale : 0.0;
    double inv_min = max_min > 0 ? 63.0 / max_min : 0.0;
    long sc[8], mn[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = (long)py_round(inv_scale * sf[j]);
        mn[j] = (long)py_round(inv_min * mf[j]);
    }
    uint8_t packed[12];
    pack_k4(sc, mn, packed);
    double d = max_scale > 0 ? f16_clamped(max_scale / 63.0) : 0.0;
    double dmin = max_min > 0 ? f16_clamped(max_min / 63.0) : 0.0;
    int levels[256] = {0};
    for (int j = 0; j < 8; ++j) {
        int s, m;
        k4_scale_min(packed, j, &s, &m);
        double step = d * s;
        if (step == 0.0) continue;
        double offset = dmin * m;
        for (int i = 0; i < 32; ++i)
            levels[32 * j + i] = (int)clampl((long)py_round((v[32 * j + i] + offset) / step), 0, (long)top);
    }
    put_f16_clamped(o, max_scale > 0 ? max_scale / 63.0 : 0.0);
    put_f16_clamped(o + 2, max_min > 0 ? max_min / 63.0 : 0.0);
    memcpy(o + 4, packed, 12);
    if (!five) {
        for (int c = 0; c < 4; ++c)
            for (int i = 0; i < 32; ++i)
                o[16 + 32 * c + i] = (uint8_t)(levels[64 * c + i] | (levels[64 * c + i + 32] << 4));
        return;
    }
    uint8_t *qh = o + 16, *ql = o + 48;
    memset(qh, 0, 32);
    int m1 = 1, m2 = 2;
    for (int c = 0; c < 4; ++c) {
        for (int j = 0; j < 32; ++j) {
            int lo = levels[64 * c + j], hi = levels[64 * c + j + 32];
            if (lo > 15) { lo -= 16; qh[j] |= (uint8_t)m1; }
            if (hi > 15) { hi -= 16; qh[j] |= (uint8_t)m2; }
            ql[32 * c + j] = (uint8_t)(lo | (hi << 4));
        }
        m1 <<= 2;
        m2 <<= 2;
    }
}

/* encode_q6_k, tests/k_quant.py:160-190 */
static int enc_q6_k(const double *v, uint8_t *o) {
    double peak = 0.0;
    for (int i = 0; i < 256; ++i) if (fabs(v[i]) > peak) peak = fabs(v[i]);
    memset(o, 0, 210);
    if (peak <= 0.0) return 0;
    double d = f16_clamped(peak / (64.0 * 31.0));
    double step = d * 64.0;
    if (step == 0.0) return -4; /* Python: round(inf) raises */
    int lv[256];
    for (int i = 0; i < 256; ++i) lv[i] = (int)clampl((long)py_round(v[i] / step) + 32, 0, 63);
    for (int h = 0; h < 2; ++h) {
        for (int i = 0; i < 32; ++i) {
            int q1 = lv[128 * h + i], q2 = lv[128 * h + i + 32];
            int q3 = lv[128 * h + i + 64], q4 = lv[128 * h + i + 96];
            o[64 * h + i] = (uint8_t)((q1 & 15) | ((q3 & 15) << 4));
            o[64 * h + i + 32] = (uint8_t)((q2 & 15) | ((q4 & 15) << 4));
            o[128 + 32 * h + i] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
        }
    }
    for (int i = 0; i < 16; ++i) o[192 + i] = 64;
    put_f16_clamped(o + 208, peak / (64.0 * 31.0));
    return 0;
}

/* encode_q2_k, tests/k_quant.py:193-222 */
static void enc_q2_k(const double *v, uint8_t *o) {
    double range[16], max_range, max_neg = 0.0;
    int have_neg = 0;
    for (int g = 0; g < 16; ++g) {
        double lo = vmin(v + 16 * g, 16);
        range[g] = vmax(v + 16 * g, 16) - lo;
        if (lo < 0.0) {
            if (!have_neg || -lo > max_neg) max_neg = -lo;
            have_neg = 1;
        }
    }
    max_range = vmax(range, 16);
    double d = max_range > 0 ? f16_clamped(max_range / 45.0) : 0.0;
    double dmin = max_neg > 0 ? f16_clamped(max_neg / 15.0) : 0.0;
    memset(o, 0, 84);
    for (int g = 0; g < 16; ++g) {
        double lo = vmin(v + 16 * g, 16);
        int sc = range[g] > 0 ? 15 : 0;
        long mn = (dmin > 0 && lo < 0.0) ? (long)py_round(-lo / dmin) : 0;
        mn = clampl(mn, 0, 15);
        o[g] = (uint8_t)((mn << 4) | sc);
        double step = d * sc, offset = dmin * (double)mn;
        int half = g / 8, shift = 2 * ((g % 8) / 2), base = half * 32 + (g % 2) * 16;
        for (int i = 0; i < 16; ++i) {
            int code = step != 0.0 ? (int)clampl((long)py_round((v[16 * g + i] + offset) / step), 0, 3) : 0;
            o[16 + base + i] |= (uint8_t)(code << shift);
        }
    }
    put_f16_clamped(o + 80, max_range > 0 ? max_range / 45.0 : 0.0);
    put_f16_clamped(o + 82, max_neg > 0 ? max_neg / 15.0 : 0.0);
}

/* pack_q3_k_block / encode_q3_k, tests/k_quant.py:225-285 */
static int enc_q3_k(const double *v, uint8_t *o) {
    double gs[16];
    for (int g = 0; g < 16; ++g) {
        double lo = vmin(v + 16 * g, 16), hi = vmax(v + 16 * g, 16);
        gs[g] = hi > lo ? (hi - lo) / 7.0 : 0.0;
    }
    double peak = vmax(gs, 16);
    double d_all = peak > 0 ? f16_clamped(peak / 31.0) : 0.0;
    int codes[16], levels[256];
    for (int g = 0; g < 16; ++g) {
        codes[g] = d_all > 0 ? (int)clampl(32 + (long)py_round(gs[g] / d_all), 0, 63) : 32;
        double lo = vmin(v + 16 * g, 16), hi = vmax(v + 16 * g, 16);
        for (int i = 0; i < 16; ++i)
            levels[16 * g + i] = hi > lo ? (int)clampl((long)py_round((v[16 * g + i] - lo) / (hi - lo) * 7.0), 0, 7) : 4;
    }
    memset(o, 0, 110);
    uint8_t *hmask = o, *qs = o + 32, *sc = o + 96;
    for (int j = 0; j < 16; ++j) {
        int low = codes[j] & 15;
        if (j < 8) sc[j] = (uint8_t)low;
        else sc[j - 8] |= (uint8_t)(low << 4);
        sc[8 + j % 4] |= (uint8_t)((codes[j] >> 4) << (2 * (j / 4)));
    }
    int q[256];
    for (int j = 0; j < 256; ++j) {
        q[j] = levels[j] > 3 ? levels[j] - 4 : levels[j];
        if (levels[j] > 3) hmask[j % 32] |= (uint8_t)(1u << (j / 32));
    }
    for (int h = 0; h < 2; ++h)
        for (int i = 0; i < 32; ++i)
            qs[32 * h + i] = (uint8_t)(q[128 * h + i] | (q[128 * h + i + 32] << 2) |
                                       (q[128 * h + i + 64] << 4) | (q[128 * h + i + 96] << 6));
    return put_f16_strict(o + 108, peak > 0 ? peak / 31.0 : 0.0);
}

/* _round_half_away of scripts/build_vocab_fixture.py:45-51 */
static long round_half_away(double v) { return v >= 0 ? (long)(v + 0.5) : -(long)(-v + 0.5); }

/* encode_q8_0, scripts/build_vocab_fixture.py:54-66 */
static int enc_q8_0(const double *v, uint8_t *o) {
    double amax = 0.0;
    for (int i = 0; i < 32; ++i) if (fabs(v[i]) > amax) amax = fabs(v[i]);
    double d = amax / 127.0, inv = d != 0.0 ? 1.0 / d : 0.0;
    if (put_f16_strict(o, d)) return -4;
    for (int i = 0; i < 32; ++i) o[2 + i] = (uint8_t)(clampl(round_half_away(v[i] * inv), -127, 127) & 0xFF);
    return 0;
}

/* encode_q4_0, scripts/build_vocab_fixture.py:69-89 */
static int enc_q4_0(const double *v, uint8_t *o) {
    double amax = 0.0, best = 0.0;
    for (int i = 0; i < 32; ++i) if (amax < fabs(v[i])) { amax = fabs(v[i]); best = v[i]; }
    double d = best / -8.0, inv = d != 0.0 ? 1.0 / d : 0.0;
    if (put_f16_strict(o, d)) return -4;
    for (int j = 0; j < 16; ++j) {
        long lo = clampl((long)(v[j] * inv + 8.5), 0, 15);
        long hi = clampl((long)(v[j + 16] * inv + 8.5), 0, 15);
        o[2 + j] = (uint8_t)(lo | (hi << 4));
    }
    return 0;
}

/* The reference ships no quantizer for the types below; these are naive,
 * byte-valid encoders of our own (min/max scale choice, nearest code), used
 * only to produce fixture bytes.  Validity is checked by decode round trip. */
static void enc_q4_1_q5_1(const double *v, uint8_t *o, int five) {
    double lo = vmin(v, 32), hi = vmax(v, 32), top = five ? 31.0 : 15.0;
    double d = (hi - lo) / top;
    put_f16_clamped(o, d);
    put_f16_clamped(o + 2, lo);
    double dq = f16_clamped(d), mq = f16_clamped(lo);
    int q[32];
    for (int i = 0; i < 32; ++i)
        q[i] = dq > 0 ? (int)clampl((long)py_round((v[i] - mq) / dq), 0, (long)top) : 0;
    uint8_t *qs = o + (five ? 8 : 4);
    uint32_t qh = 0;
    for (int i = 0; i < 16; ++i) {
        qs[i] = (uint8_t)((q[i] & 15) | ((q[i + 16] & 15) << 4));
        qh |= (uint32_t)((q[i] >> 4) & 1) << i;
        qh |= (uint32_t)((q[i + 16] >> 4) & 1) << (i + 16);
    }
    if (five) memcpy(o + 4, &qh, 4);
}

static void enc_q5_0(const double *v, uint8_t *o) {
    double amax = 0.0, best = 0.0;
    for (int i = 0; i < 32; ++i) if (amax < fabs(v[i])) { amax = fabs(v[i]); best = v[i]; }
    double d = f16_clamped(best / -16.0);
    put_f16_clamped(o, best / -16.0);
    int q[32];
    for (int i = 0; i < 32; ++i) q[i] = d != 0.0 ? (int)clampl((long)py_round(v[i] / d) + 16, 0, 31) : 16;
    uint32_t qh = 0;
    for (int i = 0; i < 16; ++i) {
        o[6 + i] = (uint8_t)((q[i] & 15) | ((q[i + 16] & 15) << 4));
        qh |= (uint32_t)((q[i] >> 4) & 1) << i;
        qh |= (uint32_t)((q[i + 16] >> 4) & 1) << (i + 16);
    }
    memcpy(o + 2, &qh, 4);
}

static void enc_q8_1(const double *v, uint8_t *o) {
    double amax = 0.0;
    for (int i = 0; i < 32; ++i) if (fabs(v[i]) > amax) amax = fabs(v[i]);
    double d = f16_clamped(amax / 127.0);
    long sum = 0;
    for (int i = 0; i < 32; ++i) {
        long q = d != 0.0 ? clampl((long)py_round(v[i] / d), -127, 127) : 0;
        o[4 + i] = (uint8_t)(q & 0xFF);
        sum += q;
    }
    put_f16_clamped(o, d);
    put_f16_clamped(o + 2, d * (double)sum);
}

static int iq4_nearest(double t) {
    int best = 0;
    double err = fabs(t - IQ4[0]);
    for (int k = 1; k < 16; ++k) {
        double e = fabs(t - IQ4[k]);
        if (e < err) { err = e; best = k; }
    }
    return best;
}

static void enc_iq4_nl(const double *v, uint8_t *o) {
    double amax = 0.0, best = 0.0;
    for (int i = 0; i < 32; ++i) if (amax < fabs(v[i])) { amax = fabs(v[i]); best = v[i]; }
    double d = f16_clamped(best / (double)IQ4[0]);
    put_f16_clamped(o, best / (double)IQ4[0]);
    for (int i = 0; i < 16; ++i) {
        int a = d != 0.0 ? iq4_nearest(v[i] / d) : 8, b = d != 0.0 ? iq4_nearest(v[i + 16] / d) : 8;
        o[2 + i] = (uint8_t)(a | (b << 4));
    }
}

static void enc_iq4_xs(const double *v, uint8_t *o) {
    double sub[8], maxs = 0.0, amaxs = 0.0;
    for (int ib = 0; ib < 8; ++ib) {
        double amax = 0.0, best = 0.0;
        for (int i = 0; i < 32; ++i) if (amax < fabs(v[32 * ib + i])) { amax = fabs(v[32 * ib + i]); best = v[32 * ib + i]; }
        sub[ib] = best / (double)IQ4[0];
        if (fabs(sub[ib]) > amaxs) { amaxs = fabs(sub[ib]); maxs = sub[ib]; }
    }
    double d = f16_clamped(-maxs / 32.0);
    put_f16_clamped(o, -maxs / 32.0);
    uint16_t sh = 0;
    memset(o + 4, 0, 4);
    for (int ib = 0; ib < 8; ++ib) {
        long ls = d != 0.0 ? clampl((long)py_round(sub[ib] / d), -32, 31) : 0;
        int code = (int)(ls + 32);
        o[4 + ib / 2] |= (uint8_t)((code & 15) << (4 * (ib & 1)));
        sh |= (uint16_t)(((code >> 4) & 3) << (2 * ib));
        double dl = d * (double)ls;
        for (int j = 0; j < 16; ++j) {
            int a = dl != 0.0 ? iq4_nearest(v[32 * ib + j] / dl) : 8;
            int b = dl != 0.0 ? iq4_nearest(v[32 * ib + j + 16] / dl) : 8;
            o[8 + 16 * ib + j] = (uint8_t)(a | (b << 4));
        }
    }
    put16(o + 2, sh);
}

long oracle_quantize(int type_id, const double *v, size_t n, uint8_t *out) {
    const type_info *t = find_type(type_id);
    if (!t) return -1;
    if (n % t->block) return -2;
    size_t nb = n / t->block;
    for (size_t i = 0; i < nb; ++i) {
        const double *x = v + i * t->block;
        uint8_t *o = out + i * t->bytes;
        int rc = 0;
        switch (type_id) {
        case 0: { float f = (float)x[0]; memcpy(o, &f, 4); break; }
        case 1: rc = put_f16_strict(o, x[0]); break;
        case 30: { /* binary32 then round-to-nearest-even on the low 16 bits */
            float f = (float)x[0];
            uint32_t u;
            memcpy(&u, &f, 4);
            if ((u & 0x7fffffffu) > 0x7f800000u) u = (u | 0x00400000u);
            else u += 0x7fffu + ((u >> 16) & 1u);
            put16(o, (uint16_t)(u >> 16));
            break;
        }
        case 28: memcpy(o, x, 8); break;
        case 24: o[0] = (uint8_t)(int8_t)clampl((long)py_round(x[0]), -128, 127); break;
        case 25: { uint16_t h = (uint16_t)(int16_t)clampl((long)py_round(x[0]), -32768, 32767); put16(o, h); break; }
        case 26: { int32_t q = (int32_t)clampl((long)py_round(x[0]), INT32_MIN, INT32_MAX); memcpy(o, &q, 4); break; }
        case 27: { int64_t q = (int64_t)llrint(x[0]); memcpy(o, &q, 8); break; }
        case 2: rc = enc_q4_0(x, o); break;
        case 3: enc_q4_1_q5_1(x, o, 0); break;
        case 6: enc_q5_0(x, o); break;
        case 7: enc_q4_1_q5_1(x, o, 1); break;
        case 8: rc = enc_q8_0(x, o); break;
        case 9: enc_q8_1(x, o); break;
        case 10: enc_q2_k(x, o); break;
        case 11: rc = enc_q3_k(x, o); break;
        case 12: enc_q45_k(x, o, 0); break;
        case 13: enc_q45_k(x, o, 1); break;
        case 14: rc = enc_q6_k(x, o); break;
        case 20: enc_iq4_nl(x, o); break;
        case 23: enc_iq4_xs(x, o); break;
        default: return -1;
        }
        if (rc) return rc;
    }
    return (long)(nb * t->bytes);
}

/* ------------------------------------------------------------------ generator */

static uint64_t splitmix64(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void oracle_fill_normal(uint64_t seed, double mean, double stddev, float *out, size_t n) {
    /* two uniforms in (0,1] and [0,1) -> two normals (Box-Muller) */
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        double u1 = 1.0 - (double)(splitmix64(&s) >> 11) * 0x1.0p-53;
        double u2 = (double)(splitmix64(&s) >> 11) * 0x1.0p-53;
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(mean + stddev * (r * cos(two_pi * u2)));
        if (i + 1 < n) out[i + 1] = (float)(mean + stddev * (r * sin(two_pi * u2)));
    }
}

/* ------------------------------------------------------------------ routing */

void oracle_softmax(const double *v, size_t n, double *out) {
    /* pyrite/tensor_ops.py:513-521: subtract the max, exp, sum left to right */
    if (n == 0) return;
    double peak = v[0];
    for (size_t i = 1; i < n; ++i) if (v[i] > peak) peak = v[i];
    double total = 0.0;
    for (size_t i = 0; i < n; ++i) { out[i] = exp(v[i] - peak); total += out[i]; }
    if (total <= 0.0) {
        for (size_t i = 0; i < n; ++i) out[i] = 1.0 / (double)n;
        return;
    }
    for (size_t i = 0; i < n; ++i) out[i] = out[i] / total;
}

double oracle_silu(double v) {
    /* pyrite/tensor_ops.py:509-510 */
    return v > -60.0 ? v / (1.0 + exp(-v)) : 0.0;
}

void oracle_rms_norm(const double *x, const double *w, size_t n, double eps, double *out) {
    /* pyrite/tensor_ops.py:502-506 */
    double ss = 0.0;
    for (size_t i = 0; i < n; ++i) ss += x[i] * x[i];
    double inv = 1.0 / sqrt(ss / (double)(n ? n : 1) + eps);
    for (size_t i = 0; i < n; ++i) out[i] = x[i] * inv * w[i];
}

long oracle_argmax_first(const double *v, size_t n) {
    /* pyrite/sampler.py:12-15: max() keeps the first index of the maximum */
    if (n == 0) return -1;
    size_t best = 0;
    for (size_t i = 1; i < n; ++i) if (v[i] > v[best]) best = i;
    return (long)best;
}

void oracle_rope(double *v, size_t n, long position, double theta, size_t rotary_dim) {
    /* pyrite/executor.py:627-646: pairs (i, i + half) of the first n_rot values */
    size_t n_rot = rotary_dim == 0 ? n : (rotary_dim < n ? rotary_dim : n);
    size_t half = n_rot / 2;
    for (size_t i = 0; i < half; ++i) {
        double freq = pow(theta, -2.0 * (double)i / (double)n_rot);
        double angle = (double)position * freq;
        double c = cos(angle), s = sin(angle);
        double x0 = v[i], x1 = v[i + half];
        v[i] = x0 * c - x1 * s;
        v[i + half] = x0 * s + x1 * c;
    }
}

int oracle_attention(const double *q, const double *k, const double *v, size_t n_heads, size_t n_kv,
                     size_t head_dim, size_t value_dim, size_t rotary_dim, double theta, double eps,
                     const double *q_norm, const double *k_norm, long position, float *k_cache,
                     float *v_cache, size_t n_prev, double *out) {
    /* pyrite/executor.py:685-755 (prep_head :712-715, cache append :729-733,
     * scores, softmax and weighted values :739-754) */
    if (n_heads == 0 || n_kv == 0 || n_heads % n_kv || head_dim == 0 || head_dim > 4096 || value_dim == 0)
        return -2;
    size_t group = n_heads / n_kv, n_tok = n_prev + 1;
    double *qh = malloc(sizeof(double) * (head_dim * 2 + n_tok * 2));
    if (!qh) return -3;
    double *tmp = qh + head_dim, *scores = tmp + head_dim, *probs = scores + n_tok;
    /* keys and values of this token: normed and rotated keys, stored as fp32 */
    for (size_t g = 0; g < n_kv; ++g) {
        const double *src = k + g * head_dim;
        if (k_norm) oracle_rms_norm(src, k_norm, head_dim, eps, tmp);
        else memcpy(tmp, src, sizeof(double) * head_dim);
        oracle_rope(tmp, head_dim, position, theta, rotary_dim);
        for (size_t i = 0; i < head_dim; ++i) k_cache[n_prev * n_kv * head_dim + g * head_dim + i] = (float)tmp[i];
        for (size_t i = 0; i < value_dim; ++i)
            v_cache[n_prev * n_kv * value_dim + g * value_dim + i] = (float)v[g * value_dim + i];
    }
    double scale = 1.0 / sqrt((double)head_dim);
    for (size_t h = 0; h < n_heads; ++h) {
        const double *src = q + h * head_dim;
        if (q_norm) oracle_rms_norm(src, q_norm, head_dim, eps, qh);
        else memcpy(qh, src, sizeof(double) * head_dim);
        oracle_rope(qh, head_dim, position, theta, rotary_dim);
        size_t g = h / group;
        for (size_t t = 0; t < n_tok; ++t) {
            const float *key = k_cache + t * n_kv * head_dim + g * head_dim;
            double sc = 0.0;
            for (size_t i = 0; i < head_dim; ++i) sc += qh[i] * (double)key[i];
            scores[t] = sc * scale;
        }
        oracle_softmax(scores, n_tok, probs);
        double *o = out + h * value_dim;
        for (size_t i = 0; i < value_dim; ++i) o[i] = 0.0;
        for (size_t t = 0; t < n_tok; ++t) {
            if (probs[t] == 0.0) continue;
            const float *val = v_cache + t * n_kv * value_dim + g * value_dim;
            for (size_t i = 0; i < value_dim; ++i) o[i] += probs[t] * (double)val[i];
        }
    }
    free(qh);
    return 0;
}

int oracle_route(const double *logits, size_t n, size_t k, int norm_topk_prob,
                 double scale, int *ids, double *weights, double *probs_out) {
    /* pyrite/executor.py:765-774: softmax, order by (-p, e), keep k,
     * renormalise when asked and the total is positive, then scale. */
    if (n == 0 || k == 0 || k > n || n > 4096) return -2;
    double probs[4096];
    unsigned char taken[4096];
    oracle_softmax(logits, n, probs);
    memset(taken, 0, n);
    for (size_t s = 0; s < k; ++s) {
        long best = -1;
        for (size_t e = 0; e < n; ++e) {
            if (taken[e]) continue;
            if (best < 0 || probs[e] > probs[best]) best = (long)e; /* ties keep lower e */
        }
        taken[best] = 1;
        ids[s] = (int)best;
        weights[s] = probs[best];
    }
    if (norm_topk_prob) {
        double total = 0.0;
        for (size_t s = 0; s < k; ++s) total += weights[s];
        if (total > 0) for (size_t s = 0; s < k; ++s) weights[s] = weights[s] / total;
    }
    if (scale != 1.0) for (size_t s = 0; s < k; ++s) weights[s] = weights[s] * scale;
    if (probs_out) memcpy(probs_out, probs, n * sizeof(double));
    return 0;
}

static size_t slice_bytes(int type_id, size_t rows, size_t cols) {
    const type_info *t = find_type(type_id);
    if (!t || cols % t->block) return 0;
    return rows * (cols / t->block) * t->bytes;
}

int oracle_moe_ffn(const uint8_t *router, size_t router_len, int router_type,
                   const uint8_t *gate, size_t gate_len, int gate_type,
                   const uint8_t *up, size_t up_len, int up_type,
                   const uint8_t *down, size_t down_len, int down_type,
                   size_t n_experts, size_t hidden, size_t inter, size_t k,
                   int norm_topk_prob, double scale,
                   const double *x, double *out, int *ids, double *weights,
                   double *router_logits) {
    size_t gs = slice_bytes(gate_type, inter, hidden), us = slice_bytes(up_type, inter, hidden);
    size_t ds = slice_bytes(down_type, hidden, inter);
    if (!gs || !us || !ds || gate_len != gs * n_experts || up_len != us * n_experts ||
        down_len != ds * n_experts || n_experts > 4096 || inter > 65536 || hidden > 65536)
        return -2;
    double logits[4096];
    int rc = oracle_matvec(router_type, router, router_len, x, logits, n_experts, hidden);
    if (rc) return rc;
    if (router_logits) memcpy(router_logits, logits, n_experts * sizeof(double));
    rc = oracle_route(logits, n_experts, k, norm_topk_prob, scale, ids, weights, NULL);
    if (rc) return rc;
    double *g = malloc(sizeof(double) * (2 * inter + inter + hidden));
    if (!g) return -3;
    double *u = g + inter, *act = u + inter, *y = act + inter;
    for (size_t i = 0; i < hidden; ++i) out[i] = 0.0;
    for (size_t s = 0; s < k; ++s) {
        if (weights[s] == 0.0) continue;
        size_t e = (size_t)ids[s];
        if ((rc = oracle_matvec(gate_type, gate + e * gs, gs, x, g, inter, hidden)) ||
            (rc = oracle_matvec(up_type, up + e * us, us, x, u, inter, hidden)))
            break;
        for (size_t i = 0; i < inter; ++i) act[i] = oracle_silu(g[i]) * u[i];
        if ((rc = oracle_matvec(down_type, down + e * ds, ds, act, y, hidden, inter))) break;
        for (size_t i = 0; i < hidden; ++i) out[i] += weights[s] * y[i];
    }
    free(g);
    return rc;
}
