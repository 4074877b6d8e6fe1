// Exact fp16 MFMA fragments of the GGML block formats, shared by the MFMA
// matvec (mx.hip, batch up to 8 per launch) and the MFMA dequant-GEMM
// (mg.hip, prefill-sized batches).
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

#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "common.h"

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

// ---------------------------------------------------------------- activations
// Largest finite |x| of 8 values (0 when none is finite and non-zero).
__device__ __forceinline__ float finite_max8(const float (&x)[8]) {
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float a = fabsf(x[i]);
        m = fmaxf(m, a <= 3.402823466e38f ? a : 0.f);
    }
    return m;
}

// Power-of-two exponent e that brings a token's largest finite |x| into
// [2^14, 2^15): the fp16 hi part of x * 2^-e cannot overflow, and its lo part
// stays a normal half down to 2^-29 of that maximum, so hi + lo carries x to
// ~2^-22 relative whatever the activations' scale.  0 for a token with no
// finite non-zero value.
__device__ __forceinline__ int norm_exp(float mx) {
    if (!(mx > 0.f)) return 0;
    return __builtin_amdgcn_frexp_expf(mx) - 15;
}

// fp16 hi and lo parts of 8 values scaled by 2^-e.  An infinite value keeps
// hi = +-inf and gets a finite lo (inf - inf would add a NaN the fp64 sum of
// the same products does not have); a NaN stays NaN in hi.
__device__ __forceinline__ void split8(const float (&x)[8], int e, uint4& hi, uint4& lo) {
    uint32_t h[4], l[4];
    const h2v big = {(_Float16)65504.f, (_Float16)65504.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = __builtin_amdgcn_ldexpf(x[2 * i], -e), b = __builtin_amdgcn_ldexpf(x[2 * i + 1], -e);
        const h2v hv = {(_Float16)a, (_Float16)b};
        h2v lv = {(_Float16)(a - (float)hv[0]), (_Float16)(b - (float)hv[1])};
        lv = __builtin_elementwise_min(__builtin_elementwise_max(lv, -big), big);
        h[i] = __builtin_bit_cast(uint32_t, hv);
        l[i] = __builtin_bit_cast(uint32_t, lv);
    }
    hi = make_uint4(h[0], h[1], h[2], h[3]);
    lo = make_uint4(l[0], l[1], l[2], l[3]);
}

// 8 bytes at p (any alignment when !AL) as two dwords
template <bool AL>
__device__ __forceinline__ void ld8(const uint8_t* p, uint32_t& a, uint32_t& b) {
    uint32_t w[2];
    ld_span<8, AL>(p, w);
    a = w[0];
    b = w[1];
}

// NB bytes at b + off in a copy of the weights in LDS (L; the MFMA matvec
// stages them there): the dwords from there rounded down to 4 bytes, one byte
// shift for the span (computed from b, so the spans of one block share it).
// The dword after the span is read too; the LDS area ends with padding so
// that it always exists.
template <int NB>
__device__ __forceinline__ void lds_span(const uint8_t* b, int off, uint32_t (&w)[(NB + 3) / 4]) {
    constexpr int N = (NB + 3) / 4;
    const uint32_t bs = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(b)) & 3u;
    const uint32_t s = (bs + static_cast<uint32_t>(off)) & 3u;
    const uint32_t* q = reinterpret_cast<const uint32_t*>(b + off - s);
    uint32_t t[N + 1];
#pragma unroll
    for (int k = 0; k <= N; ++k) t[k] = q[k];
#pragma unroll
    for (int k = 0; k < N; ++k) w[k] = __builtin_amdgcn_alignbyte(t[k + 1], t[k], s);
}
// NB bytes at b + off in global memory, any alignment: as lds_span (one
// shift from b), but only dwords that overlap the span are read, so no read
// leaves the page of the span's bytes: the dword after the first N is read
// only when the span reaches into it, else the last of the N again.
template <int NB>
__device__ __forceinline__ void gl_span(const uint8_t* b, int off, uint32_t (&w)[(NB + 3) / 4]) {
    constexpr int N = (NB + 3) / 4;
    const uint32_t bs = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(b)) & 3u;
    const uint32_t s = (bs + static_cast<uint32_t>(off)) & 3u;
    const uint32_t* q = reinterpret_cast<const uint32_t*>(b + off - s);
    uint32_t t[N + 1];
#pragma unroll
    for (int k = 0; k < N; ++k) t[k] = q[k];
    t[N] = q[s + NB > 4 * N ? N : N - 1];
#pragma unroll
    for (int k = 0; k < N; ++k) w[k] = __builtin_amdgcn_alignbyte(t[k + 1], t[k], s);
}
// the span reader of a format's load: global memory or LDS (L); unaligned
// global spans as dword-aligned loads realigned by v_alignbyte_b32, or (UA)
// as loads at the span's own byte address
template <int NB, bool AL, bool L, bool UA = false>
__device__ __forceinline__ void mx_span(const uint8_t* b, int off, uint32_t (&w)[(NB + 3) / 4]) {
    if constexpr (AL) ld_span<NB, AL>(b + off, w);
    else if constexpr (L) lds_span<NB>(b, off, w);
    else if constexpr (UA) ld_span<NB, false, true>(b + off, w);
    else gl_span<NB>(b, off, w);
}
template <bool AL, bool L, bool UA = false>
__device__ __forceinline__ void mx_ld8(const uint8_t* b, int off, uint32_t& x, uint32_t& y) {
    uint32_t w[2];
    mx_span<8, AL, L, UA>(b, off, w);
    x = w[0];
    y = w[1];
}
// bytes of LDS padding after staged weights read with L
constexpr int kMxLdsPad = 16;

// ---------------------------------------------------------------- K-slot maps
// Which 8 columns the K-slots of lane group g hold in step S (counted from the
// start of the row, 32 columns per step).  The A fragments (activations) are
// staged with the same map as the B fragments (weights) use, so the products
// pair up whatever the order: a dot product does not depend on the order of
// its terms' positions in K.
//   mode 0: columns 32 S + 8 g (step S = 32 consecutive columns);
//   mode 1: 256-column blocks, lane group g owns columns 64 g .. 64 g + 63 of
//           each block: 256 (S / 8) + 64 g + 8 (S % 8).  A lane then meets
//           two 32-column sub-blocks per block instead of eight, so their
//           scales are converted once per block.
__device__ __forceinline__ int mx_kcol(int mode, int S, int g) {
    return mode == 1 ? 256 * (S >> 3) + 64 * g + 8 * (S & 7) : 32 * S + 8 * g;
}

// ---------------------------------------------------------------- formats
// Each format supplies:
//   BS, BPB, STEPS (= BS / 32), NACC (1 or 2 accumulators per block)
//   Raw: the lane's bytes of one block (lane group g owns K-slots 8g..8g+7)
//   load<AL>(blk, g, raw)
//   frag(raw, step, g, b[NACC][4]): B fragments of one 32-column step
//   epi(raw, D[NACC], acc): acc += block scale(s) applied to D
// and optionally
//   KMODE: its K-slot map (mx_kcol; 0 when absent)
//   Pre, prep(raw, g, pre): per-block lane constants, after which the
//   fragments are frag(raw, pre, step, g, b)
template <int T> struct Mx;

template <class F, class = void> struct MxKMode { static constexpr int value = 0; };
template <class F> struct MxKMode<F, std::void_t<decltype(F::KMODE)>> { static constexpr int value = F::KMODE; };
template <class F, class = void> struct MxHasPre : std::false_type {};
template <class F> struct MxHasPre<F, std::void_t<typename F::Pre>> : std::true_type {};
struct MxNoPre {};
template <class F, bool = MxHasPre<F>::value> struct MxPreOf { using type = MxNoPre; };
template <class F> struct MxPreOf<F, true> { using type = typename F::Pre; };

// column of K-slot group g in step S of format F
template <class F>
__device__ __forceinline__ int mx_col(int S, int g) {
    return mx_kcol(MxKMode<F>::value, S, g);
}
template <class F>
__device__ __forceinline__ void mx_prep(const typename F::Raw& r, int g, typename MxPreOf<F>::type& p) {
    if constexpr (MxHasPre<F>::value) F::prep(r, g, p);
}
template <class F>
__device__ __forceinline__ void mx_frag(const typename F::Raw& r, const typename MxPreOf<F>::type& p, int st, int g,
                                        uint32_t (&b)[F::NACC][4]) {
    if constexpr (MxHasPre<F>::value) F::frag(r, p, st, g, b);
    else F::frag(r, st, g, b);
}

// Q4_K: d | dmin | scales[12] | qs[128] (pyrite/kernels/native.c:173-197).
// Sub-block j (columns 32j..32j+31, scale and min j): nibble j & 1 of
// qs[32 (j >> 1) + l].  K-slot map 1: lane group g holds qs[32g..32g+31],
// i.e. sub-blocks 2g (low nibbles, steps 0-3) and 2g + 1 (high nibbles,
// steps 4-7); step s takes bytes 8 (s & 3)..+7 of them.
template <> struct Mx<T_Q4_K> {
    static constexpr int BS = 256, BPB = 144, STEPS = 8, NACC = 2, KMODE = 1;
    struct Raw { uint32_t hd[4]; uint32_t q[8]; };
    // packed (s, s), (-1024 s, -1024 s) and (m, m) halves of sub-blocks 2g, 2g + 1
    struct Pre { uint32_t S[2], O[2], M[2]; };
    template <bool AL, bool L = false, bool UA = false>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
        mx_span<16, AL, L, UA>(b, 0, r.hd);
        mx_span<32, AL, L, UA>(b, 16 + 32 * g, r.q);
    }
    // scale and min of sub-block j, any j in 0..7 (get_scale_min_k4, native.c:52-61)
    __device__ __forceinline__ static void k4_scale_min_rt(const uint32_t (&hd)[4], int j, uint32_t& a, uint32_t& m) {
        const int sh = 8 * (j & 3);
        const uint32_t s0 = hd[1] >> sh, s1 = hd[2] >> sh, s2 = hd[3] >> sh;
        a = j < 4 ? (s0 & 63) : ((s2 & 15) | ((s0 >> 6 & 3) << 4));
        m = j < 4 ? (s1 & 63) : ((s2 >> 4 & 15) | ((s1 >> 6 & 3) << 4));
    }
    __device__ __forceinline__ static void prep(const Raw& r, int g, Pre& p) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            uint32_t a, m;
            k4_scale_min_rt(r.hd, 2 * g + h, a, m);
            p.S[h] = splat_h((float)a);
            p.O[h] = splat_h(-1024.f * (float)a);
            p.M[h] = splat_h((float)m);
        }
    }
    __device__ __forceinline__ static void frag(const Raw& r, const Pre& p, int s, int, uint32_t (&b)[2][4]) {
        const int h = s >> 2, k = s & 3;
        uint32_t x0 = r.q[2 * k], x1 = r.q[2 * k + 1];
        if (h) { x0 >>= 4; x1 >>= 4; }
        x0 &= 0x0F0F0F0Fu;
        x1 &= 0x0F0F0F0Fu;
        b[0][0] = pk_fma(bias_lo(x0), p.S[h], p.O[h]);
        b[0][1] = pk_fma(bias_hi(x0), p.S[h], p.O[h]);
        b[0][2] = pk_fma(bias_lo(x1), p.S[h], p.O[h]);
        b[0][3] = pk_fma(bias_hi(x1), p.S[h], p.O[h]);
        b[1][0] = b[1][1] = b[1][2] = b[1][3] = p.M[h];
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
    __device__ __forceinline__ static void epi(const Raw& r, const f4v (&D)[2], f4v& acc) {
        const float d = half_bits_to_float(r.hd[0]), dmin = half_bits_to_float(r.hd[0] >> 16);
        acc += d * D[0] - dmin * D[1];
    }
    // Dequant-GEMM form (mg.hip): the min term dmin * sum_j m_j S_j, with S_j
    // the activations' sum over sub-block j, is one MFMA per block against
    // staged sub-block sums, so the per-step fragments carry the codes only.
    static constexpr bool MINSUM = true;
    __device__ __forceinline__ static void frag_main(const Raw& r, const Pre& p, int s, uint32_t (&b)[4]) {
        const int h = s >> 2, k = s & 3;
        uint32_t x0 = r.q[2 * k], x1 = r.q[2 * k + 1];
        if (h) { x0 >>= 4; x1 >>= 4; }
        x0 &= 0x0F0F0F0Fu;
        x1 &= 0x0F0F0F0Fu;
        b[0] = pk_fma(bias_lo(x0), p.S[h], p.O[h]);
        b[1] = pk_fma(bias_hi(x0), p.S[h], p.O[h]);
        b[2] = pk_fma(bias_lo(x1), p.S[h], p.O[h]);
        b[3] = pk_fma(bias_hi(x1), p.S[h], p.O[h]);
    }
    // B of the min MFMA: K-slots j and 8 + j (lane groups 0 and 1, against
    // the hi and lo parts of the staged sub-block sums) hold 32 m_j (exact:
    // at most 2016), the other K-slots 0.  The staged sums carry 2^-5.
    __device__ __forceinline__ static void min_frag(const Raw& r, int g, uint32_t (&b)[4]) {
        const uint32_t m03 = r.hd[2] & 0x3F3F3F3Fu;
        const uint32_t m47 = ((r.hd[3] >> 4) & 0x0F0F0F0Fu) | ((r.hd[2] >> 2) & 0x30303030u);
        const float sc = g < 2 ? 32.f : 0.f;
        const uint32_t S = splat_h(sc), O = splat_h(-1024.f * sc);
        b[0] = pk_fma(bias_lo(m03), S, O);
        b[1] = pk_fma(bias_hi(m03), S, O);
        b[2] = pk_fma(bias_lo(m47), S, O);
        b[3] = pk_fma(bias_hi(m47), S, O);
    }
    __device__ __forceinline__ static float dscale(const Raw& r) { return half_bits_to_float(r.hd[0]); }
    __device__ __forceinline__ static float mscale(const Raw& r) { return half_bits_to_float(r.hd[0] >> 16); }
};

// Q5_K: as Q4_K with a fifth bit, qh[l] bit j (native.c:410-437).
template <> struct Mx<T_Q5_K> {
    static constexpr int BS = 256, BPB = 176, STEPS = 8, NACC = 2;
    struct Raw { uint32_t hd[4]; uint32_t h[2]; uint32_t q[4][2]; };
    template <bool AL, bool L = false, bool UA = false>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
        mx_span<16, AL, L, UA>(b, 0, r.hd);
        mx_ld8<AL, L, UA>(b, 16 + 8 * g, r.h[0], r.h[1]);
#pragma unroll
        for (int c = 0; c < 4; ++c) mx_ld8<AL, L, UA>(b, 48 + 32 * c + 8 * g, r.q[c][0], r.q[c][1]);
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
    template <bool AL, bool L = false, bool UA = false>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
#pragma unroll
        for (int k = 0; k < 4; ++k) mx_ld8<AL, L, UA>(b, 64 * (k >> 1) + 32 * (k & 1) + 8 * g, r.ql[k][0], r.ql[k][1]);
#pragma unroll
        for (int h = 0; h < 2; ++h) mx_ld8<AL, L, UA>(b, 128 + 32 * h + 8 * g, r.qh[h][0], r.qh[h][1]);
        mx_span<16, AL, L, UA>(b, 192, r.sc);
        uint32_t dd[1];
        mx_span<2, AL, L, UA>(b, 208, dd);
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
    template <bool AL, bool L = false, bool UA = false>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
#pragma unroll
        for (int h = 0; h < 2; ++h) mx_ld8<AL, L, UA>(b, 32 + 32 * h + 8 * g, r.qs[h][0], r.qs[h][1]);
        mx_ld8<AL, L, UA>(b, 8 * g, r.hm[0], r.hm[1]);
        mx_span<12, AL, L, UA>(b, 96, r.sc);
        uint32_t dd[1];
        mx_span<2, AL, L, UA>(b, 108, dd);
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
    template <bool AL, bool L = false, bool UA = false>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
#pragma unroll
        for (int h = 0; h < 2; ++h) mx_ld8<AL, L, UA>(b, 16 + 32 * h + 8 * g, r.qs[h][0], r.qs[h][1]);
        mx_span<16, AL, L, UA>(b, 0, r.sc);
        uint32_t dd[1];
        mx_span<4, AL, L, UA>(b, 80, dd);
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
    template <bool AL, bool L = false, bool UA = false>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
        mx_span<8, AL, L, UA>(b, 0, r.hd);
#pragma unroll
        for (int ib = 0; ib < 8; ++ib) mx_ld8<AL, L, UA>(b, 8 + 16 * ib + 8 * (g & 1), r.q[ib][0], r.q[ib][1]);
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
template <int OFF, int NB, bool AL, bool L, bool UA = false>
__device__ __forceinline__ void ld_nib8(const uint8_t* b, int g, uint32_t& x0, uint32_t& x1) {
    mx_ld8<AL, L, UA>(b, OFF + 8 * (g & 1), x0, x1);
    if (g & 2) { x0 >>= 4; x1 >>= 4; }
    x0 &= 0x0F0F0F0Fu;
    x1 &= 0x0F0F0F0Fu;
}

// Q4_0: d | qs[16]; d * (q - 8) (native.c:281-288)
template <> struct Mx<T_Q4_0> {
    static constexpr int BS = 32, BPB = 18, STEPS = 1, NACC = 1;
    struct Raw { uint32_t x0, x1, d; };
    template <bool AL, bool L = false, bool UA = false>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
        ld_nib8<2, 18, AL, L, UA>(b, g, r.x0, r.x1);
        uint32_t dd[1];
        mx_span<2, AL, L, UA>(b, 0, dd);
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
    template <bool AL, bool L = false, bool UA = false>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
        ld_nib8<2, 18, AL, L, UA>(b, g, r.x0, r.x1);
        uint32_t dd[1];
        mx_span<2, AL, L, UA>(b, 0, dd);
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
    template <bool AL, bool L = false, bool UA = false>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
        ld_nib8<4, 20, AL, L, UA>(b, g, r.x0, r.x1);
        uint32_t dd[1];
        mx_span<4, AL, L, UA>(b, 0, dd);
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
    template <bool AL, bool L = false, bool UA = false>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
        ld_nib8<6, 22, AL, L, UA>(b, g, r.x0, r.x1);
        uint32_t w[2];
        mx_span<6, AL, L, UA>(b, 0, w);
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
    template <bool AL, bool L = false, bool UA = false>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
        ld_nib8<8, 24, AL, L, UA>(b, g, r.x0, r.x1);
        uint32_t w[2];
        mx_span<8, AL, L, UA>(b, 0, w);
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
    template <bool AL, bool L = false, bool UA = false>
    __device__ __forceinline__ static void load(const uint8_t* b, int g, Raw& r) {
        mx_ld8<AL, L, UA>(b, OFF + 8 * g, r.x0, r.x1);
        uint32_t dd[1];
        mx_span<2, AL, L, UA>(b, 0, dd);
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

}  // namespace pyrite
