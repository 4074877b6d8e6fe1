// MFMA dequant-matvec for the GGML block formats (batch 1..8), gfx950.
//
// y[t][r] = sum_c dequant(W)[r][c] * x[t][c]   (pyrite/kernels/native.c:518-555,
// fp32 accumulation, t < 8 activation vectors).
//
// Operands of v_mfma_f32_16x16x32_f16 (lane l: m or n = l % 16, group g = l / 16,
// K-slots 8g..8g+7 of a 32-column step; D lane l holds column n, rows 4g..4g+3):
//   A (16 x 32) = activations: row m = 2t + p holds the fp16 "hi" (p = 0) or
//                 "lo" (p = 1) part of x[t], with hi + lo = x to ~2^-22;
//   B (32 x 16) = weights: column n is weight row r0 + n; the K-slot values
//                 are exact fp16 integers built from the block codes, with
//                 the 6-bit sub-block scale folded in where the product stays
//                 exactly representable (|value| <= 2048);
//   D (16 x 16) = per lane: row r0 + n, token-parts 4g..4g+3 (two tokens).
// The block scale(s) (fp16 d, dmin) multiply D once per block ("epilogue").
// Codes become fp16 without arithmetic: v_perm_b32 interleaves a code byte c
// with 0x64, giving the half 1024 + c; one v_pk_fma_f16 then yields
// s * (c - offset) exactly (single rounding of an exactly representable
// result).  Where s * c could exceed 11 significant bits (Q6_K's int8 scales,
// IQ4_XS's 6-bit scale times the codebook) the scale is split s = 16*s1 + s0
// and the block accumulates two D's: 16 * D1 + D0.
//
// Schedule: a workgroup (4 waves) owns a 32-row tile (two 16-row MFMA column
// tiles sharing the A fragment); its waves split the row's blocks round-robin
// and the 4 partial results are summed in LDS in a fixed order, so results are
// deterministic.  Workgroups loop over tiles.  The A fragments of the whole
// row (or of a K chunk when they exceed the LDS budget) are built once per
// workgroup in LDS, compacted to the token-parts in use (MB = 2 * tokens).
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "common.h"
#include "dispatch.h"

namespace pyrite {

typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- fp16 helpers
__device__ __forceinline__ uint32_t bias_lo(uint32_t codes) {  // (1024 + c0, 1024 + c1)
    return __builtin_amdgcn_perm(0x64646464u, codes, 0x04010400u);
}
__device__ __forceinline__ uint32_t bias_hi(uint32_t codes) {  // (1024 + c2, 1024 + c3)
    return __builtin_amdgcn_perm(0x64646464u, codes, 0x04030402u);
}
__device__ __forceinline__ uint32_t pk_fma(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(h2v, a),
                                                                  __builtin_bit_cast(h2v, b),
                                                                  __builtin_bit_cast(h2v, c)));
}
__device__ __forceinline__ uint32_t pk_add(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v, a) + __builtin_bit_cast(h2v, b));
}
// (v, v) as a packed half pair; v must be exactly representable
__device__ __forceinline__ uint32_t splat_h(float v) {
    const uint32_t h = __builtin_bit_cast(unsigned short, (_Float16)v);
    return h | (h << 16);
}

// 8 byte codes (two dwords) -> 4 dwords of halves s * (c - off).  Exact when
// s * (c - off) and (1024 + off) * s are both exactly representable in fp16.
__device__ __forceinline__ void scaled8(uint32_t c0, uint32_t c1, float s, float off, uint32_t (&b)[4]) {
    const uint32_t S = splat_h(s), O = splat_h(-(1024.f + off) * s);
    b[0] = pk_fma(bias_lo(c0), S, O);
    b[1] = pk_fma(bias_hi(c0), S, O);
    b[2] = pk_fma(bias_lo(c1), S, O);
    b[3] = pk_fma(bias_hi(c1), S, O);
}
// 8 byte codes -> 4 dwords of halves (c - off) (exact)
__device__ __forceinline__ void offset8(uint32_t c0, uint32_t c1, float off, uint32_t (&b)[4]) {
    const uint32_t O = splat_h(-(1024.f + off));
    b[0] = pk_add(bias_lo(c0), O);
    b[1] = pk_add(bias_hi(c0), O);
    b[2] = pk_add(bias_lo(c1), O);
    b[3] = pk_add(bias_hi(c1), O);
}
// 8 byte codes -> 4 dwords of halves s * (c - off), for offsets whose product
// (1024 + off) * s is not exactly representable: subtract, then multiply
// (both exact)
__device__ __forceinline__ void offset_scaled8(uint32_t c0, uint32_t c1, float off, float s, uint32_t (&b)[4]) {
    offset8(c0, c1, off, b);
    const h2v S = __builtin_bit_cast(h2v, splat_h(s));
#pragma unroll
    for (int i = 0; i < 4; ++i) b[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v, b[i]) * S);
}
__device__ __forceinline__ void splat8(float v, uint32_t (&b)[4]) {
    const uint32_t s = splat_h(v);
    b[0] = b[1] = b[2] = b[3] = s;
}

// 8 bytes at p (any alignment when !AL) as two dwords
template <bool AL>
__device__ __forceinline__ void ld8(const uint8_t* p, uint32_t& a, uint32_t& b) {
    uint32_t w[2];
    ld_span<8, AL>(p, w);
    a = w[0];
    b = w[1];
}

// ---------------------------------------------------------------- formats
// Each format supplies:
//   BS, BPB, STEPS (= BS / 32), NACC (1 or 2 accumulators per block)
//   Raw: the lane's bytes of one block (lane group g owns K-slots 8g..8g+7)
//   load<AL>(blk, g, raw)
//   frag(raw, step, g, b[NACC][4]): B fragments of one 32-column step
//   epi(raw, D[NACC], acc): acc += block scale(s) applied to D
template <int T> struct Mx;

// Q4_K: d | dmin | scales[12] | qs[128] (pyrite/kernels/native.c:173-197).
// step j (sub-block j): columns 32j + l; j = 2c + h -> nibble h of qs[32c + l].
template <> struct Mx<T_Q4_K> {
    static constexpr int BS = 256, BPB = 144, STEPS = 8, NACC = 2;
    struct Raw { uint32_t hd[4]; uint32_t q[4][2]; };
    template <bool AL>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
        ld_span<16, AL>(b, r.hd);
#pragma unroll
        for (int c = 0; c < 4; ++c) ld8<AL>(b + 16 + 32 * c + 8 * g, r.q[c][0], r.q[c][1]);
    }
    __device__ __forceinline__ static void scale_min(const Raw& r, int j, float& sc, float& mn) {
        k4_scale_min(r.hd, j, sc, mn);
    }
    __device__ __forceinline__ static void k4_scale_min(const uint32_t (&hd)[4], int j, float& sc, float& mn) {
        const uint32_t s0 = hd[1], s1 = hd[2], s2 = hd[3];
        uint32_t a, m;
        if (j < 4) {
            a = (s0 >> (8 * j)) & 63;
            m = (s1 >> (8 * j)) & 63;
        } else {
            const int k = 8 * (j - 4);
            a = ((s2 >> k) & 15) | (((s0 >> k) >> 6 & 3) << 4);
            m = ((s2 >> k) >> 4 & 15) | (((s1 >> k) >> 6 & 3) << 4);
        }
        sc = (float)a;
        mn = (float)m;
    }
    __device__ __forceinline__ static void frag(const Raw& r, int j, int, uint32_t (&b)[2][4]) {
        const int c = j >> 1;
        uint32_t x0 = r.q[c][0], x1 = r.q[c][1];
        if (j & 1) { x0 >>= 4; x1 >>= 4; }
        float sc, mn;
        scale_min(r, j, sc, mn);
        scaled8(x0 & 0x0F0F0F0Fu, x1 & 0x0F0F0F0Fu, sc, 0.f, b[0]);
        splat8(mn, b[1]);
    }
    __device__ __forceinline__ static void epi(const Raw& r, const f4v (&D)[2], f4v& acc) {
        const float d = half_bits_to_float(r.hd[0]), dmin = half_bits_to_float(r.hd[0] >> 16);
        acc += d * D[0] - dmin * D[1];
    }
};

// Q5_K: as Q4_K with a fifth bit, qh[l] bit j (native.c:410-437).
template <> struct Mx<T_Q5_K> {
    static constexpr int BS = 256, BPB = 176, STEPS = 8, NACC = 2;
    struct Raw { uint32_t hd[4]; uint32_t h[2]; uint32_t q[4][2]; };
    template <bool AL>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
        ld_span<16, AL>(b, r.hd);
        ld8<AL>(b + 16 + 8 * g, r.h[0], r.h[1]);
#pragma unroll
        for (int c = 0; c < 4; ++c) ld8<AL>(b + 48 + 32 * c + 8 * g, r.q[c][0], r.q[c][1]);
    }
    __device__ __forceinline__ static void frag(const Raw& r, int j, int, uint32_t (&b)[2][4]) {
        const int c = j >> 1;
        uint32_t x0 = r.q[c][0], x1 = r.q[c][1];
        if (j & 1) { x0 >>= 4; x1 >>= 4; }
        x0 = (x0 & 0x0F0F0F0Fu) | (((r.h[0] >> j) & 0x01010101u) << 4);
        x1 = (x1 & 0x0F0F0F0Fu) | (((r.h[1] >> j) & 0x01010101u) << 4);
        float sc, mn;
        Mx<T_Q4_K>::k4_scale_min(r.hd, j, sc, mn);
        scaled8(x0, x1, sc, 0.f, b[0]);
        splat8(mn, b[1]);
    }
    __device__ __forceinline__ static void epi(const Raw& r, const f4v (&D)[2], f4v& acc) {
        const float d = half_bits_to_float(r.hd[0]), dmin = half_bits_to_float(r.hd[0] >> 16);
        acc += d * D[0] - dmin * D[1];
    }
};

// Q6_K: ql[128] | qh[64] | int8 scales[16] | d (native.c:199-225).
// step s: h = s / 4, g' = s % 4, columns 128h + 32g' + l; low nibble g' >> 1 of
// ql[64h + 32(g' & 1) + l], two high bits 2g' of qh[32h + l], scale
// 8h + 2g' + l / 16.  The int8 scale is split 16*s1 + s0.
template <> struct Mx<T_Q6_K> {
    static constexpr int BS = 256, BPB = 210, STEPS = 8, NACC = 2;
    struct Raw { uint32_t ql[4][2]; uint32_t qh[2][2]; uint32_t sc[4]; uint32_t d; };
    template <bool AL>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
#pragma unroll
        for (int k = 0; k < 4; ++k) ld8<AL>(b + 64 * (k >> 1) + 32 * (k & 1) + 8 * g, r.ql[k][0], r.ql[k][1]);
#pragma unroll
        for (int h = 0; h < 2; ++h) ld8<AL>(b + 128 + 32 * h + 8 * g, r.qh[h][0], r.qh[h][1]);
        ld_span<16, AL>(b + 192, r.sc);
        uint32_t dd[1];
        ld_span<2, AL>(b + 208, dd);
        r.d = dd[0];
    }
    __device__ __forceinline__ static void frag(const Raw& r, int s, int g, uint32_t (&b)[2][4]) {
        const int h = s >> 2, gp = s & 3;
        const int k = 2 * h + (gp & 1);
        uint32_t x0 = r.ql[k][0], x1 = r.ql[k][1];
        if (gp & 2) { x0 >>= 4; x1 >>= 4; }
        x0 = (x0 & 0x0F0F0F0Fu) | (((r.qh[h][0] >> (2 * gp)) & 0x03030303u) << 4);
        x1 = (x1 & 0x0F0F0F0Fu) | (((r.qh[h][1] >> (2 * gp)) & 0x03030303u) << 4);
        const int idx = 8 * h + 2 * gp + (g >> 1);
        const int sv = (int)(int8_t)((r.sc[idx >> 2] >> (8 * (idx & 3))) & 0xFF);
        const int s1 = sv >> 4, s0 = sv & 15;
        scaled8(x0, x1, (float)s1, 32.f, b[0]);
        scaled8(x0, x1, (float)s0, 32.f, b[1]);
    }
    __device__ __forceinline__ static void epi(const Raw& r, const f4v (&D)[2], f4v& acc) {
        acc += half_bits_to_float(r.d) * (16.f * D[0] + D[1]);
    }
};

// Q3_K: hmask[32] | qs[64] | scales[12] | d (native.c:129-171).
// step s: h = s / 4, g' = s % 4, columns 128h + 32g' + l: code bits 2g' of
// qs[32h + l], high bit 4h + g' of hmask[l] (clear -> minus 4), 6-bit scale
// j = 8h + 2g' + l / 16 stored as scale + 32.
template <> struct Mx<T_Q3_K> {
    static constexpr int BS = 256, BPB = 110, STEPS = 8, NACC = 1;
    struct Raw { uint32_t qs[2][2]; uint32_t hm[2]; uint32_t sc[3]; uint32_t d; };
    template <bool AL>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
#pragma unroll
        for (int h = 0; h < 2; ++h) ld8<AL>(b + 32 + 32 * h + 8 * g, r.qs[h][0], r.qs[h][1]);
        ld8<AL>(b + 8 * g, r.hm[0], r.hm[1]);
        ld_span<12, AL>(b + 96, r.sc);
        uint32_t dd[1];
        ld_span<2, AL>(b + 108, dd);
        r.d = dd[0];
    }
    __device__ __forceinline__ static void frag(const Raw& r, int s, int g, uint32_t (&b)[1][4]) {
        const int h = s >> 2, gp = s & 3;
        const uint32_t x0 = ((r.qs[h][0] >> (2 * gp)) & 0x03030303u) |
                            (((r.hm[0] >> (4 * h + gp)) & 0x01010101u) << 2);
        const uint32_t x1 = ((r.qs[h][1] >> (2 * gp)) & 0x03030303u) |
                            (((r.hm[1] >> (4 * h + gp)) & 0x01010101u) << 2);
        const int j = 8 * h + 2 * gp + (g >> 1);
        const int lb = (int)((r.sc[(j & 7) >> 2] >> (8 * (j & 3))) & 0xFF);
        const int low4 = (j < 8) ? (lb & 15) : (lb >> 4);
        const int hi2 = (int)((r.sc[2] >> (8 * (j & 3))) >> (2 * (j >> 2)) & 3);
        // (c - 4) * (scale - 32): -1028 * scale is not exact in fp16, so the
        // offset is removed before the (exact) product
        offset_scaled8(x0, x1, 4.f, (float)((low4 | (hi2 << 4)) - 32), b[0]);
    }
    __device__ __forceinline__ static void epi(const Raw& r, const f4v (&D)[1], f4v& acc) {
        acc += half_bits_to_float(r.d) * D[0];
    }
};

// Q2_K: scales[16] | qs[64] | d | dmin (native.c:381-408).  Same column
// layout as Q3_K; scale byte 8h + 2g' + l / 16 = (min << 4) | scale.
template <> struct Mx<T_Q2_K> {
    static constexpr int BS = 256, BPB = 84, STEPS = 8, NACC = 2;
    struct Raw { uint32_t qs[2][2]; uint32_t sc[4]; uint32_t dd; };
    template <bool AL>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
#pragma unroll
        for (int h = 0; h < 2; ++h) ld8<AL>(b + 16 + 32 * h + 8 * g, r.qs[h][0], r.qs[h][1]);
        ld_span<16, AL>(b, r.sc);
        uint32_t dd[1];
        ld_span<4, AL>(b + 80, dd);
        r.dd = dd[0];
    }
    __device__ __forceinline__ static void frag(const Raw& r, int s, int g, uint32_t (&b)[2][4]) {
        const int h = s >> 2, gp = s & 3;
        const uint32_t x0 = (r.qs[h][0] >> (2 * gp)) & 0x03030303u;
        const uint32_t x1 = (r.qs[h][1] >> (2 * gp)) & 0x03030303u;
        const int j = 8 * h + 2 * gp + (g >> 1);
        const uint32_t sb = (r.sc[j >> 2] >> (8 * (j & 3))) & 0xFF;
        scaled8(x0, x1, (float)(sb & 15), 0.f, b[0]);
        splat8((float)(sb >> 4), b[1]);
    }
    __device__ __forceinline__ static void epi(const Raw& r, const f4v (&D)[2], f4v& acc) {
        acc += half_bits_to_float(r.dd) * D[0] - half_bits_to_float(r.dd >> 16) * D[1];
    }
};

// IQ4_XS: d | scales_h | scales_l[4] | qs[128] (native.c:364-379).
// step ib: columns 32ib + l; l < 16 low nibble of qs[16ib + l], else high
// nibble of qs[16ib + l - 16]; value d * (ls - 32) * K[n], (ls - 32) split 16*s1 + s0.
template <> struct Mx<T_IQ4_XS> {
    static constexpr int BS = 256, BPB = 136, STEPS = 8, NACC = 2;
    struct Raw { uint32_t hd[2]; uint32_t q[8][2]; };
    template <bool AL>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
        ld_span<8, AL>(b, r.hd);
#pragma unroll
        for (int ib = 0; ib < 8; ++ib) ld8<AL>(b + 8 + 16 * ib + 8 * (g & 1), r.q[ib][0], r.q[ib][1]);
    }
    __device__ __forceinline__ static void frag(const Raw& r, int ib, int g, uint32_t (&b)[2][4]) {
        uint32_t x0 = r.q[ib][0], x1 = r.q[ib][1];
        if (g & 2) { x0 >>= 4; x1 >>= 4; }
        x0 = iq4_lut4(x0 & 0x0F0F0F0Fu);
        x1 = iq4_lut4(x1 & 0x0F0F0F0Fu);
        const uint32_t sl = (r.hd[1] >> (8 * (ib >> 1))) & 0xFF;
        const int ls = (int)(((sl >> (4 * (ib & 1))) & 15) | (((r.hd[0] >> (16 + 2 * ib)) & 3) << 4)) - 32;
        const int s1 = ls >> 4, s0 = ls & 15;
        scaled8(x0, x1, (float)s1, 128.f, b[0]);
        scaled8(x0, x1, (float)s0, 128.f, b[1]);
    }
    __device__ __forceinline__ static void epi(const Raw& r, const f4v (&D)[2], f4v& acc) {
        acc += half_bits_to_float(r.hd[0]) * (16.f * D[0] + D[1]);
    }
};

// 32-element blocks: one step per block; lane group g owns columns 8g..8g+7,
// the low nibbles of qs[8g..] for g < 2 and the high nibbles of qs[8(g-2)..].
template <int OFF, int NB, bool AL>
__device__ __forceinline__ void ld_nib8(const uint8_t* b, int g, uint32_t& x0, uint32_t& x1) {
    ld8<AL>(b + OFF + 8 * (g & 1), x0, x1);
    if (g & 2) { x0 >>= 4; x1 >>= 4; }
    x0 &= 0x0F0F0F0Fu;
    x1 &= 0x0F0F0F0Fu;
}

// Q4_0: d | qs[16]; d * (q - 8) (native.c:281-288)
template <> struct Mx<T_Q4_0> {
    static constexpr int BS = 32, BPB = 18, STEPS = 1, NACC = 1;
    struct Raw { uint32_t x0, x1, d; };
    template <bool AL>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
        ld_nib8<2, 18, AL>(b, g, r.x0, r.x1);
        uint32_t dd[1];
        ld_span<2, AL>(b, dd);
        r.d = dd[0];
    }
    __device__ __forceinline__ static void frag(const Raw& r, int, int, uint32_t (&b)[1][4]) {
        offset8(r.x0, r.x1, 8.f, b[0]);
    }
    __device__ __forceinline__ static void epi(const Raw& r, const f4v (&D)[1], f4v& acc) {
        acc += half_bits_to_float(r.d) * D[0];
    }
};

// IQ4_NL: d | qs[16]; d * K[n] (native.c:351-358)
template <> struct Mx<T_IQ4_NL> {
    static constexpr int BS = 32, BPB = 18, STEPS = 1, NACC = 1;
    struct Raw { uint32_t x0, x1, d; };
    template <bool AL>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
        ld_nib8<2, 18, AL>(b, g, r.x0, r.x1);
        uint32_t dd[1];
        ld_span<2, AL>(b, dd);
        r.d = dd[0];
    }
    __device__ __forceinline__ static void frag(const Raw& r, int, int, uint32_t (&b)[1][4]) {
        offset8(iq4_lut4(r.x0), iq4_lut4(r.x1), 128.f, b[0]);
    }
    __device__ __forceinline__ static void epi(const Raw& r, const f4v (&D)[1], f4v& acc) {
        acc += half_bits_to_float(r.d) * D[0];
    }
};

// Q4_1: d | m | qs[16]; d * q + m (native.c:290-298).  D[1] = sum of x.
template <> struct Mx<T_Q4_1> {
    static constexpr int BS = 32, BPB = 20, STEPS = 1, NACC = 2;
    struct Raw { uint32_t x0, x1, dm; };
    template <bool AL>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
        ld_nib8<4, 20, AL>(b, g, r.x0, r.x1);
        uint32_t dd[1];
        ld_span<4, AL>(b, dd);
        r.dm = dd[0];
    }
    __device__ __forceinline__ static void frag(const Raw& r, int, int, uint32_t (&b)[2][4]) {
        offset8(r.x0, r.x1, 0.f, b[0]);
        splat8(1.f, b[1]);
    }
    __device__ __forceinline__ static void epi(const Raw& r, const f4v (&D)[2], f4v& acc) {
        acc += half_bits_to_float(r.dm) * D[0] + half_bits_to_float(r.dm >> 16) * D[1];
    }
};

// fifth bits of columns 8g'..8g'+7 (g' = g & 1, +16 for the high nibbles) from qh
__device__ __forceinline__ void q5_high(uint32_t qh, int g, uint32_t& x0, uint32_t& x1) {
    const int base = 8 * (g & 1) + 16 * (g >> 1);
    x0 |= spread4(qh >> base) << 4;
    x1 |= spread4(qh >> (base + 4)) << 4;
}

// Q5_0: d | qh | qs[16]; d * (q5 - 16) (native.c:300-314)
template <> struct Mx<T_Q5_0> {
    static constexpr int BS = 32, BPB = 22, STEPS = 1, NACC = 1;
    struct Raw { uint32_t x0, x1, d; };
    template <bool AL>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
        ld_nib8<6, 22, AL>(b, g, r.x0, r.x1);
        uint32_t w[2];
        ld_span<6, AL>(b, w);
        r.d = w[0];
        q5_high(__builtin_amdgcn_alignbyte(w[1], w[0], 2u), g, r.x0, r.x1);
    }
    __device__ __forceinline__ static void frag(const Raw& r, int, int, uint32_t (&b)[1][4]) {
        offset8(r.x0, r.x1, 16.f, b[0]);
    }
    __device__ __forceinline__ static void epi(const Raw& r, const f4v (&D)[1], f4v& acc) {
        acc += half_bits_to_float(r.d) * D[0];
    }
};

// Q5_1: d | m | qh | qs[16]; d * q5 + m (native.c:316-328)
template <> struct Mx<T_Q5_1> {
    static constexpr int BS = 32, BPB = 24, STEPS = 1, NACC = 2;
    struct Raw { uint32_t x0, x1, dm; };
    template <bool AL>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
        ld_nib8<8, 24, AL>(b, g, r.x0, r.x1);
        uint32_t w[2];
        ld_span<8, AL>(b, w);
        r.dm = w[0];
        q5_high(w[1], g, r.x0, r.x1);
    }
    __device__ __forceinline__ static void frag(const Raw& r, int, int, uint32_t (&b)[2][4]) {
        offset8(r.x0, r.x1, 0.f, b[0]);
        splat8(1.f, b[1]);
    }
    __device__ __forceinline__ static void epi(const Raw& r, const f4v (&D)[2], f4v& acc) {
        acc += half_bits_to_float(r.dm) * D[0] + half_bits_to_float(r.dm >> 16) * D[1];
    }
};

// Q8_0 / Q8_1: d (| s) | int8 qs[32]; d * q (native.c:330-344).  Codes are
// biased to unsigned (xor 0x80) before the fp16 conversion.
template <int OFF, int NB>
struct MxQ8 {
    static constexpr int BS = 32, BPB = NB, STEPS = 1, NACC = 1;
    struct Raw { uint32_t x0, x1, d; };
    template <bool AL>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
        ld8<AL>(b + OFF + 8 * g, r.x0, r.x1);
        uint32_t dd[1];
        ld_span<2, AL>(b, dd);
        r.d = dd[0];
    }
    __device__ __forceinline__ static void frag(const Raw& r, int, int, uint32_t (&b)[1][4]) {
        offset8(r.x0 ^ 0x80808080u, r.x1 ^ 0x80808080u, 128.f, b[0]);
    }
    __device__ __forceinline__ static void epi(const Raw& r, const f4v (&D)[1], f4v& acc) {
        acc += half_bits_to_float(r.d) * D[0];
    }
};
template <> struct Mx<T_Q8_0> : MxQ8<2, 34> {};
template <> struct Mx<T_Q8_1> : MxQ8<4, 36> {};

// ---------------------------------------------------------------- kernel

struct MxDesc {
    const uint8_t* W;
    unsigned long long row_bytes;
    const float* X;
    unsigned long long ldx;
    float* Y;
    unsigned long long ldy;
    float* part;          // split-K partial sums [ksplit][tiles][32 rows][8 tokens]
    unsigned* counters;   // per-tile arrival counters; zero between launches
    int rows;
    int cols;
    int batch;            // activation vectors (<= 8)
    int ksplit;           // K parts (workgroup tasks per 32-row tile)
    int kpart_steps;      // 32-column steps per K part (a multiple of the block's steps)
    int tiles;            // ceil(rows / 32)
    int task_begin;       // first task of this matrix; tasks = ksplit * tiles
    int pad;
};

constexpr int kMxMaxGroup = 16;
struct MxGroup {
    int n;
    int total_tasks;
    MxDesc d[kMxMaxGroup];
};

constexpr int kRedBytes = 4 * 2 * 64 * 4 * 4;  // [wave][row tile][lane][4] floats
constexpr int kPF = 2;                          // blocks per wave loaded ahead of their use

// Barrier for LDS hand-offs only: waits for this wave's LDS traffic, not for
// its outstanding global loads (which may be blocks prefetched for later).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// exponent e >= 0 with mx * 2^-e < 2^15
__device__ __forceinline__ int exp_for(float mx) {
    if (!(mx >= 32768.f) || !(mx < 3.0e38f)) return 0;
    int e;
    (void)frexpf(mx, &e);
    return e - 15;
}

// A fragments of steps [s0, s1) into LDS, laid out [step][group][MB] x 16 bytes
// (8 halves: hi or lo parts of x[t][32 s + 8 group + i] * 2^-e_t).  Also
// records max |x| per token (as ordered uint bits of a non-negative float).
template <int MB>
__device__ __forceinline__ void stage_x(const MxDesc& d, int s0, int s1, int tid, const int* tok_exp,
                                        unsigned* tok_max, uint4* frag) {
    const int count = (s1 - s0) * 4 * MB;
    for (int idx = tid; idx < count; idx += 256) {
        const int s = s0 + idx / (4 * MB), rem = idx % (4 * MB);
        const int gg = rem / MB, mm = rem % MB, t = mm >> 1;
        uint32_t v[4] = {0u, 0u, 0u, 0u};
        if (t < d.batch) {
            const float* xp = d.X + t * d.ldx + 32 * s + 8 * gg;
            const float4 a = ld_x4(xp), b = ld_x4(xp + 4);
            float xs[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            float mx = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(xs[i]));
            if ((mm & 1) == 0 && mx > 0.f) atomicMax(&tok_max[t], __float_as_uint(mx));
            const int e = tok_exp[t];
            if (e) {
#pragma unroll
                for (int i = 0; i < 8; ++i) xs[i] = __builtin_amdgcn_ldexpf(xs[i], -e);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const _Float16 h0 = (_Float16)xs[2 * i], h1 = (_Float16)xs[2 * i + 1];
                _Float16 o0 = h0, o1 = h1;
                if (mm & 1) {
                    o0 = (_Float16)(xs[2 * i] - (float)h0);
                    o1 = (_Float16)(xs[2 * i + 1] - (float)h1);
                }
                v[i] = (uint32_t)__builtin_bit_cast(unsigned short, o0) |
                       ((uint32_t)__builtin_bit_cast(unsigned short, o1) << 16);
            }
        }
        frag[idx] = make_uint4(v[0], v[1], v[2], v[3]);
    }
}

// One block of two 16-row column tiles: B fragments, MFMAs, block epilogue.
template <int T, int MB>
__device__ __forceinline__ void mx_block(const typename Mx<T>::Raw& ra, const typename Mx<T>::Raw& rb,
                                         const uint4* fblk, int g, int n, f4v (&acc)[2]) {
    using F = Mx<T>;
    f4v Da[F::NACC], Db[F::NACC];
#pragma unroll
    for (int p = 0; p < F::NACC; ++p) {
        Da[p] = f4v{0.f, 0.f, 0.f, 0.f};
        Db[p] = f4v{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int st = 0; st < F::STEPS; ++st) {
        uint4 av = make_uint4(0u, 0u, 0u, 0u);
        if (n < MB) av = fblk[(st * 4 + g) * MB + n];
        const uint32_t aw[4] = {av.x, av.y, av.z, av.w};
        const h8v a = __builtin_bit_cast(h8v, aw);
        uint32_t ba[F::NACC][4], bb[F::NACC][4];
        F::frag(ra, st, g, ba);
        F::frag(rb, st, g, bb);
#pragma unroll
        for (int p = 0; p < F::NACC; ++p) {
            Da[p] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(h8v, ba[p]), Da[p], 0, 0, 0);
            Db[p] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(h8v, bb[p]), Db[p], 0, 0, 0);
        }
    }
    F::epi(ra, Da, acc[0]);
    F::epi(rb, Db, acc[1]);
}

template <int T, int MB, bool AL>
__global__ __launch_bounds__(256) void mx_kernel(const MxGroup grp) {
    using F = Mx<T>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    float* red = reinterpret_cast<float*>(smem);
    uint4* frag = reinterpret_cast<uint4*>(smem + kRedBytes);
    __shared__ int tok_exp[8];
    __shared__ unsigned tok_max[8];
    __shared__ int last_flag;

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, n = lane & 15;
    int staged_mi = -1, staged_kp = -1;

    for (int task = blockIdx.x; task < grp.total_tasks; task += gridDim.x) {
        int mi = 0;
        while (mi + 1 < grp.n && task >= grp.d[mi + 1].task_begin) ++mi;
        const MxDesc& d = grp.d[mi];
        const int local = task - d.task_begin;
        const int kp = local / d.tiles, tile = local - kp * d.tiles;
        const int rows = d.rows;
        const int nblk = d.cols / F::BS;
        const int kps = d.kpart_steps;
        const int s0 = kp * kps;
        const int s1 = (s0 + kps < (d.cols >> 5)) ? s0 + kps : (d.cols >> 5);
        const int kb0 = s0 / F::STEPS;
        const int kb1 = (s1 / F::STEPS < nblk) ? s1 / F::STEPS : nblk;

        const long long r0 = (long long)tile * 32 + n, r1 = r0 + 16;
        const uint8_t* rp0 = d.W + (r0 < rows ? r0 : rows - 1) * d.row_bytes;
        const uint8_t* rp1 = d.W + (r1 < rows ? r1 : rows - 1) * d.row_bytes;

        // first blocks of this wave, loaded before the (possible) staging
        typename F::Raw ra[kPF], rb[kPF];
        int blk = kb0 + w;
#pragma unroll
        for (int p = 0; p < kPF; ++p) {
            const int bq = blk + 4 * p;
            if (bq < kb1) {
                F::template load<AL>(rp0 + (size_t)bq * F::BPB, g, ra[p]);
                F::template load<AL>(rp1 + (size_t)bq * F::BPB, g, rb[p]);
            }
        }

        if (mi != staged_mi || kp != staged_kp) {
            // Per-token power-of-two scale 2^-e keeping |x * 2^-e| < 2^15 so the
            // fp16 hi part cannot overflow; results are multiplied back by 2^e
            // (exact).  The maxima are gathered while staging and the part is
            // staged again in the rare case a scale is needed.
            lds_barrier();
            if (tid < 8) {
                tok_exp[tid] = 0;
                tok_max[tid] = 0u;
            }
            lds_barrier();
            stage_x<MB>(d, s0, s1, tid, tok_exp, tok_max, frag);
            lds_barrier();
            bool rescale = false;
            for (int t = 0; t < 8; ++t) rescale |= __uint_as_float(tok_max[t]) >= 32768.f;
            if (rescale) {  // uniform across the workgroup
                if (tid < 8) tok_exp[tid] = exp_for(__uint_as_float(tok_max[tid]));
                lds_barrier();
                stage_x<MB>(d, s0, s1, tid, tok_exp, tok_max, frag);
                lds_barrier();
            }
            staged_mi = mi;
            staged_kp = kp;
        }

        f4v acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        while (blk < kb1) {
#pragma unroll
            for (int p = 0; p < kPF; ++p) {
                const int bq = blk + 4 * p;
                if (bq < kb1) mx_block<T, MB>(ra[p], rb[p], frag + (bq * F::STEPS - s0) * 4 * MB, g, n, acc);
            }
            blk += 4 * kPF;
#pragma unroll
            for (int p = 0; p < kPF; ++p) {
                const int bq = blk + 4 * p;
                if (bq < kb1) {
                    F::template load<AL>(rp0 + (size_t)bq * F::BPB, g, ra[p]);
                    F::template load<AL>(rp1 + (size_t)bq * F::BPB, g, rb[p]);
                }
            }
        }

        // Sum the 4 waves' partials in a fixed order.  Lane (n, g) of wave w
        // holds rows r0 / r1 and token-parts 4g..4g+3 = tokens 2g and 2g+1 (hi, lo).
        float* rw = red + (w * 2 * 64 + lane) * 4;
        *reinterpret_cast<f4v*>(rw) = acc[0];
        *reinterpret_cast<f4v*>(rw + 64 * 4) = acc[1];
        lds_barrier();
        const int rt = tid >> 7, t = (tid >> 4) & 7, nn = tid & 15;
        float sum;
        {
            const int src = ((t >> 1) << 4) | nn, j = (t & 1) * 2;
            sum = 0.f;
#pragma unroll
            for (int ww = 0; ww < 4; ++ww) {
                const float* q = red + ((ww * 2 + rt) * 64 + src) * 4;
                sum += q[j] + q[j + 1];
            }
            sum = __builtin_amdgcn_ldexpf(sum, tok_exp[t]);
        }
        const int trow = rt * 16 + nn;
        const long long row = (long long)tile * 32 + trow;
        if (d.ksplit == 1) {
            if (t < d.batch && row < rows) d.Y[t * d.ldy + row] = sum;
        } else {
            // split K: publish this part; the last part to arrive sums all parts
            // in part order (deterministic) and writes y, then re-arms the
            // counter (device-coherent hand-off, see st_dev / arrive_dev).
            float* pt = d.part + ((size_t)kp * d.tiles + tile) * 256;
            st_dev(pt + trow * 8 + t, sum);
            drain_dev();
            __syncthreads();
            if (tid == 0) last_flag = arrive_dev(&d.counters[tile]) == (unsigned)(d.ksplit - 1);
            __syncthreads();
            if (last_flag) {
                float tot = 0.f;
                for (int k = 0; k < d.ksplit; ++k) tot += ld_dev(d.part + ((size_t)k * d.tiles + tile) * 256 + trow * 8 + t);
                if (t < d.batch && row < rows) d.Y[t * d.ldy + row] = tot;
                if (tid == 0) st_dev(&d.counters[tile], 0u);
            }
        }
        lds_barrier();
    }
}

// ---------------------------------------------------------------- launcher

constexpr long long kMxTargetWgs = 1024;
// bytes of A fragments per workgroup: with the reduction area and the small
// static arrays the workgroup stays within 64 KiB of LDS
constexpr int kMxLdsBudget = 65536 - kRedBytes - 512;

struct MxPlanOut {
    long long tasks;
    size_t part_floats;
    size_t counters;
    int max_kps;
};

template <int T, int MB>
static MxPlanOut mx_plan(MxGroup& grp) {
    using F = Mx<T>;
    MxPlanOut out{0, 0, 0, 0};
    int kc = kMxLdsBudget / (MB * 64);
    kc -= kc % F::STEPS;
    for (int i = 0; i < grp.n; ++i) {
        MxDesc& d = grp.d[i];
        const int nsteps = d.cols / 32, nblk = d.cols / F::BS;
        d.tiles = (d.rows + 31) / 32;
        // K parts: only as many as the LDS budget for the activations needs
        // (a matrix's parts depend on its own shape, never on its group)
        int ks = (nsteps + kc - 1) / kc;
        int bpp = (nblk + ks - 1) / ks;  // blocks per part
        ks = (nblk + bpp - 1) / bpp;
        d.ksplit = ks;
        d.kpart_steps = bpp * F::STEPS;
        d.task_begin = (int)out.tasks;
        out.tasks += (long long)ks * d.tiles;
        if (ks > 1) {
            out.part_floats += (size_t)ks * d.tiles * 256;
            out.counters += d.tiles;
        }
        if (d.kpart_steps > out.max_kps) out.max_kps = d.kpart_steps;
    }
    return out;
}

// Split-K workspace, one per device, grown on demand.  Counters are zeroed
// when allocated and every launch leaves them at zero.  Launches that split K
// on one device must be ordered on one stream (they share this buffer).
struct MxWorkspace {
    float* part = nullptr;
    size_t part_cap = 0;
    unsigned* counters = nullptr;
    size_t counter_cap = 0;
};
static MxWorkspace g_ws[64];

static hipError_t mx_workspace(size_t part_floats, size_t counters, float** part, unsigned** ctr,
                               hipStream_t stream) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= 64) return e != hipSuccess ? e : hipErrorInvalidDevice;
    MxWorkspace& w = g_ws[dev];
    if (part_floats > w.part_cap || counters > w.counter_cap) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
            return hipErrorStreamCaptureUnsupported;  // grow the workspace before capturing
        (void)hipStreamSynchronize(stream);
        if (part_floats > w.part_cap) {
            if (w.part) (void)hipFree(w.part);
            w.part = nullptr;
            w.part_cap = 0;
            const size_t want = part_floats + part_floats / 2;
            if ((e = hipMalloc(&w.part, want * sizeof(float))) != hipSuccess) return e;
            w.part_cap = want;
        }
        if (counters > w.counter_cap) {
            if (w.counters) (void)hipFree(w.counters);
            w.counters = nullptr;
            w.counter_cap = 0;
            const size_t want = counters + counters / 2 + 256;
            if ((e = hipMalloc(&w.counters, want * sizeof(unsigned))) != hipSuccess) return e;
            if ((e = hipMemset(w.counters, 0, want * sizeof(unsigned))) != hipSuccess) return e;
            w.counter_cap = want;
        }
    }
    *part = w.part;
    *ctr = w.counters;
    return hipSuccess;
}

template <int T, int MB, bool AL>
static hipError_t mx_launch_group(MxGroup& grp, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    const MxPlanOut plan = mx_plan<T, MB>(grp);
    grp.total_tasks = (int)plan.tasks;
    if (plan.part_floats) {
        float* part = nullptr;
        unsigned* ctr = nullptr;
        hipError_t e = mx_workspace(plan.part_floats, plan.counters, &part, &ctr, stream);
        if (e != hipSuccess) return e;
        size_t po = 0, co = 0;
        for (int i = 0; i < grp.n; ++i) {
            MxDesc& d = grp.d[i];
            if (d.ksplit > 1) {
                d.part = part + po;
                d.counters = ctr + co;
                po += (size_t)d.ksplit * d.tiles * 256;
                co += d.tiles;
            } else {
                d.part = nullptr;
                d.counters = nullptr;
            }
        }
    }
    const long long wgs = plan.tasks < kMxTargetWgs ? plan.tasks : kMxTargetWgs;
    const size_t lds = kRedBytes + (size_t)plan.max_kps * 4 * MB * 16;
    if (start || stop)
        hipExtLaunchKernelGGL((mx_kernel<T, MB, AL>), dim3((unsigned)wgs), dim3(256), (uint32_t)lds, stream, start,
                              stop, 0, grp);
    else
        hipLaunchKernelGGL((mx_kernel<T, MB, AL>), dim3((unsigned)wgs), dim3(256), lds, stream, grp);
    return hipGetLastError();
}

template <int T, bool AL>
static hipError_t mx_launch_type(int batch, MxGroup& grp, hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
    if constexpr (Geo<T>::bs > 1) {
        if (batch <= 1) return mx_launch_group<T, 2, AL>(grp, s, e0, e1);
        if (batch <= 2) return mx_launch_group<T, 4, AL>(grp, s, e0, e1);
        if (batch <= 4) return mx_launch_group<T, 8, AL>(grp, s, e0, e1);
        return mx_launch_group<T, 16, AL>(grp, s, e0, e1);
    }
    return hipErrorInvalidValue;
}

bool mx_type_supported(int type) {
    switch (type) {
    case T_Q4_0: case T_Q4_1: case T_Q5_0: case T_Q5_1: case T_Q8_0: case T_Q8_1: case T_Q2_K:
    case T_Q3_K: case T_Q4_K: case T_Q5_K: case T_Q6_K: case T_IQ4_NL: case T_IQ4_XS:
        return true;
    default:
        return false;
    }
}

// Launch the MFMA path for up to 8 activation vectors starting at vector
// `done` of each matrix; arguments already validated.
int mx_group_launch(int type, const MatvecArgs* mats, size_t n, size_t batch, size_t done, bool al,
                    hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    const TypeGeo geo = type_geo(type);
    for (size_t base = 0; base < n; base += kMxMaxGroup) {
        MxGroup grp;
        grp.n = (int)((n - base) < (size_t)kMxMaxGroup ? (n - base) : (size_t)kMxMaxGroup);
        for (int i = 0; i < grp.n; ++i) {
            const MatvecArgs& m = mats[base + i];
            MxDesc& d = grp.d[i];
            d.W = static_cast<const uint8_t*>(m.w);
            d.row_bytes = m.cols / geo.bs * geo.bpb;
            d.X = m.x + done * m.ldx;
            d.ldx = m.ldx;
            d.Y = m.y + done * m.ldy;
            d.ldy = m.ldy;
            d.rows = (int)m.rows;
            d.cols = (int)m.cols;
            d.batch = (int)batch;
            d.part = nullptr;
            d.counters = nullptr;
        }
        hipEvent_t e0 = base == 0 ? start : nullptr;
        hipEvent_t e1 = (base + kMxMaxGroup >= n) ? stop : nullptr;
        hipError_t e = hipSuccess;
#define PYRITE_MX_CASE(T)                                                                  \
    case T:                                                                              \
        e = al ? mx_launch_type<T, (Geo<T>::bpb % 4 == 0)>((int)batch, grp, stream, e0, e1) \
               : mx_launch_type<T, false>((int)batch, grp, stream, e0, e1);               \
        break;
        switch (type) {
            PYRITE_MX_CASE(T_Q4_0)
            PYRITE_MX_CASE(T_Q4_1)
            PYRITE_MX_CASE(T_Q5_0)
            PYRITE_MX_CASE(T_Q5_1)
            PYRITE_MX_CASE(T_Q8_0)
            PYRITE_MX_CASE(T_Q8_1)
            PYRITE_MX_CASE(T_Q2_K)
            PYRITE_MX_CASE(T_Q3_K)
            PYRITE_MX_CASE(T_Q4_K)
            PYRITE_MX_CASE(T_Q5_K)
            PYRITE_MX_CASE(T_Q6_K)
            PYRITE_MX_CASE(T_IQ4_NL)
            PYRITE_MX_CASE(T_IQ4_XS)
        default:
            return -1;
        }
#undef PYRITE_MX_CASE
        if (e != hipSuccess) return -4;
    }
    return 0;
}

}  // namespace pyrite
