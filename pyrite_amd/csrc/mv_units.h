// Per-type "unit" decoders for the fp32 dequant-matvec (VALU path).
//
// A unit is the slice of one block a lane owns: 32 weights (one whole block)
// for the 32-element formats, 64 weights (a quarter super-block) for the
// 256-element formats, 4 elements for the plain types.  A unit is decoded for
// R rows that share the same columns, against B activation vectors, with the
// block scale factored out of the inner loop:
//     sum_i (d*sc*q_i - dmin*m) x_i = d*sc * sum_i q_i x_i - dmin*m * sum_i x_i
// q_i are converted with v_cvt_f32_ubyte{0..3}; sum_i x_i over every 16
// columns is precomputed per workgroup in LDS (xs16).  Element order inside a
// unit follows each block layout (pyrite/kernels/native.c:129-437).
//
// bound() accumulates, per row and batch vector, an upper bound of the sum of
// the magnitudes of every product dot() forms for the unit (codes, offsets and
// minima counted separately, as dot() multiplies them), using per-16-column
// sums of |x|.  The fp32 rounding error of the matvec is at most
// gamma_depth times this sum; the LM-head argmax uses it to decide which rows
// can still hold the maximum of the exact logits.
#pragma once

#include <type_traits>

#include "common.h"

namespace pyrite {

typedef __attribute__((address_space(3))) float lds_f;

typedef float f4n __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) f4n lds_f4;

__device__ __forceinline__ float4 ld_x4(const lds_f* p) {
    const f4n v = *(const lds_f4*)(p);
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_x4(lds_f* p, float4 v) {
    *(lds_f4*)(p) = f4n{v.x, v.y, v.z, v.w};
}

// Activations seen by one unit.  With XL the activations are staged in LDS
// with 4 floats of padding after every PADI floats (PADI = the unit stride of
// the format, so consecutive lanes read distinct bank groups); ptr(b, off)
// maps a column offset inside the current block to the (padded) address.
// Block starts are multiples of PADI, so padding is additive across them.
template <bool XL, int PADI>
struct XView {
    using P = typename std::conditional<XL, const lds_f*, const float*>::type;
    P x;                // activations of column 0 of this block, batch 0
    size_t ldx;         // floats between batch rows
    const lds_f* xs16;  // LDS: sum of each 16 columns, batch 0, from column 0 of this block
    const lds_f* xa16;  // LDS: sum of |x| over each 16 columns (same indexing; bound pass only)
    int ld16;           // floats between batch rows in xs16 / xa16
    __device__ __forceinline__ P ptr(int b, int off) const {
        if constexpr (XL) return x + b * ldx + off + (off / PADI) * 4;
        else return x + b * ldx + off;
    }
};

// sum over 4*NW consecutive columns of u32 codes (4 per dword) against x
template <int NW, typename PX>
__device__ __forceinline__ float dot_run(const uint32_t (&c)[NW], PX x) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < NW; ++k) s = dot_ub4(c[k], ld_x4(x + 4 * k), s);
    return s;
}

template <int T> struct Unit;

// ------------------------------------------------------------------ Q4_K
// unit c (0..3): qs[32c, 32c+32); low nibbles -> columns 64c+l (sub-block 2c),
// high nibbles -> 64c+32+l (sub-block 2c+1).  pyrite/kernels/native.c:173-197
__device__ __forceinline__ void k4_pair_regs(uint32_t s0, uint32_t s1, uint32_t s2, int c,
                                             float& sc0, float& m0, float& sc1, float& m1) {
    const uint32_t k = 16u * (c & 1);
    const uint32_t Ba = (s0 >> k) & 0xFF, Bb = (s0 >> (k + 8)) & 0xFF;
    const uint32_t Ma = (s1 >> k) & 0xFF, Mb = (s1 >> (k + 8)) & 0xFF;
    const uint32_t Ca = (s2 >> k) & 0xFF, Cb = (s2 >> (k + 8)) & 0xFF;
    uint32_t a0, a1, a2, a3;
    if (c < 2) {
        a0 = Ba & 63; a1 = Ma & 63; a2 = Bb & 63; a3 = Mb & 63;
    } else {
        a0 = (Ca & 15) | ((Ba >> 6) << 4);
        a1 = (Ca >> 4) | ((Ma >> 6) << 4);
        a2 = (Cb & 15) | ((Bb >> 6) << 4);
        a3 = (Cb >> 4) | ((Mb >> 6) << 4);
    }
    sc0 = (float)a0; m0 = (float)a1; sc1 = (float)a2; m1 = (float)a3;
}

template <> struct Unit<T_Q4_K> {
    static constexpr int P = 4, PADI = 64;
    struct Raw { uint32_t hd[4]; uint32_t q[8]; };
    template <bool AL>
    __device__ __forceinline__ static void load(const uint8_t* blk, int c, Raw& raw) {
        ld_span<16, AL>(blk, raw.hd);
        ld_span<32, AL>(blk + 16 + 32 * c, raw.q);
    }
    template <int B, int R, class XV>
    __device__ __forceinline__ static void dot(const Raw (&raw)[R], int c, const XV& xv,
                                               float (&acc)[R][B]) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const lds_f* s16 = xv.xs16 + b * xv.ld16 + 4 * c;
            const float xlo = s16[0] + s16[1], xhi = s16[2] + s16[3];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                uint32_t lo[8], hi[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) { lo[k] = oand(raw[r].q[k], 0x0F0F0F0Fu); hi[k] = oand(raw[r].q[k], 0xF0F0F0F0u); }
                const float slo = dot_run<8>(lo, xv.ptr(b, 64 * c));
                const float shi = dot_run<8>(hi, xv.ptr(b, 64 * c + 32));
                float sc0, m0, sc1, m1;
                k4_pair_regs(raw[r].hd[1], raw[r].hd[2], raw[r].hd[3], c, sc0, m0, sc1, m1);
                const float d = half_bits_to_float(raw[r].hd[0]), dmin = half_bits_to_float(raw[r].hd[0] >> 16);
                acc[r][b] += d * (sc0 * slo + sc1 * 0.0625f * shi) - dmin * (m0 * xlo + m1 * xhi);
            }
        }
    }
    // leaves: d*sc*q*x (q <= 15) and dmin*m*x
    template <int B, int R, class XV>
    __device__ __forceinline__ static void bound(const Raw (&raw)[R], int c, const XV& xv, float (&bacc)[R][B]) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float sc0, m0, sc1, m1;
            k4_pair_regs(raw[r].hd[1], raw[r].hd[2], raw[r].hd[3], c, sc0, m0, sc1, m1);
            const float d = fabsf(half_bits_to_float(raw[r].hd[0])), dm = fabsf(half_bits_to_float(raw[r].hd[0] >> 16));
            const float k0 = d * sc0 * 15.f + dm * m0, k1 = d * sc1 * 15.f + dm * m1;
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const lds_f* a = xv.xa16 + b * xv.ld16 + 4 * c;
                bacc[r][b] += k0 * (a[0] + a[1]) + k1 * (a[2] + a[3]);
            }
        }
    }
};

// ------------------------------------------------------------------ Q5_K
// as Q4_K plus a fifth bit: qh[l] bit 2c (low) / 2c+1 (high).  native.c:410-437
template <> struct Unit<T_Q5_K> {
    static constexpr int P = 4, PADI = 64;
    struct Raw { uint32_t hd[4]; uint32_t q[8]; uint32_t h[8]; };
    template <bool AL>
    __device__ __forceinline__ static void load(const uint8_t* blk, int c, Raw& raw) {
        ld_span<16, AL>(blk, raw.hd);
        ld_span<32, AL>(blk + 16, raw.h);
        ld_span<32, AL>(blk + 48 + 32 * c, raw.q);
    }
    template <int B, int R, class XV>
    __device__ __forceinline__ static void dot(const Raw (&raw)[R], int c, const XV& xv,
                                               float (&acc)[R][B]) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const auto x = xv.ptr(b, 64 * c), xh = xv.ptr(b, 64 * c + 32);
            const lds_f* s16 = xv.xs16 + b * xv.ld16 + 4 * c;
            const float xlo = s16[0] + s16[1], xhi = s16[2] + s16[3];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                uint32_t lo[8], hi[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    lo[k] = oandor(raw[r].q[k], 0x0F0F0F0Fu, ((raw[r].h[k] >> (2 * c)) & 0x01010101u) << 4);
                    hi[k] = oandor(raw[r].q[k] >> 4, 0x0F0F0F0Fu, ((raw[r].h[k] >> (2 * c + 1)) & 0x01010101u) << 4);
                }
                const float slo = dot_run<8>(lo, x);
                const float shi = dot_run<8>(hi, xh);
                float sc0, m0, sc1, m1;
                k4_pair_regs(raw[r].hd[1], raw[r].hd[2], raw[r].hd[3], c, sc0, m0, sc1, m1);
                const float d = half_bits_to_float(raw[r].hd[0]), dmin = half_bits_to_float(raw[r].hd[0] >> 16);
                acc[r][b] += d * (sc0 * slo + sc1 * shi) - dmin * (m0 * xlo + m1 * xhi);
            }
        }
    }
    // leaves: d*sc*q*x (q <= 31) and dmin*m*x
    template <int B, int R, class XV>
    __device__ __forceinline__ static void bound(const Raw (&raw)[R], int c, const XV& xv, float (&bacc)[R][B]) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float sc0, m0, sc1, m1;
            k4_pair_regs(raw[r].hd[1], raw[r].hd[2], raw[r].hd[3], c, sc0, m0, sc1, m1);
            const float d = fabsf(half_bits_to_float(raw[r].hd[0])), dm = fabsf(half_bits_to_float(raw[r].hd[0] >> 16));
            const float k0 = d * sc0 * 31.f + dm * m0, k1 = d * sc1 * 31.f + dm * m1;
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const lds_f* a = xv.xa16 + b * xv.ld16 + 4 * c;
                bacc[r][b] += k0 * (a[0] + a[1]) + k1 * (a[2] + a[3]);
            }
        }
    }
};

// ------------------------------------------------------------------ Q6_K
// unit u = (h, r') = (u >> 1, u & 1): columns 128h + 32g + 16r' + l, g = 0..3,
// l = 0..15.  ql bytes 64h+16r'+l (g even) and 64h+32+16r'+l (g odd), nibble
// g >> 1; qh byte 32h+16r'+l bits 2g; scale 8h + 2g + r'.  native.c:199-225
template <> struct Unit<T_Q6_K> {
    static constexpr int P = 4, PADI = 128;
    struct Raw { uint32_t A[4]; uint32_t Bq[4]; uint32_t H[4]; uint32_t S[2]; uint32_t D[1]; };
    template <bool AL>
    __device__ __forceinline__ static void load(const uint8_t* blk, int u, Raw& raw) {
        const int h = u >> 1, rr = u & 1;
        ld_span<16, AL, true>(blk + 64 * h + 16 * rr, raw.A);
        ld_span<16, AL, true>(blk + 64 * h + 32 + 16 * rr, raw.Bq);
        ld_span<16, AL, true>(blk + 128 + 32 * h + 16 * rr, raw.H);
        ld_span<8, AL, true>(blk + 192 + 8 * h, raw.S);
        ld_span<2, AL, true>(blk + 208, raw.D);
    }
    template <int B, int R, class XV>
    __device__ __forceinline__ static void dot(const Raw (&raw)[R], int u, const XV& xv,
                                               float (&acc)[R][B]) {
        const int h = u >> 1, rr = u & 1;
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int xo = 128 * h + 16 * rr;
            const lds_f* s16 = xv.xs16 + b * xv.ld16 + 8 * h + rr;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float tot = 0.f;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    uint32_t c[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const uint32_t lq = (g & 1) ? raw[r].Bq[k] : raw[r].A[k];
                        c[k] = oandor((g & 2) ? (lq >> 4) : lq, 0x0F0F0F0Fu,
                                      ((raw[r].H[k] >> (2 * g)) & 0x03030303u) << 4);
                    }
                    const float sg = dot_run<4>(c, xv.ptr(b, xo + 32 * g));
                    const uint32_t sw = raw[r].S[g >> 1] >> (8 * (rr + 2 * (g & 1)));
                    const float sc = (float)(int)(int8_t)(sw & 0xFF);
                    tot += sc * (sg - 32.f * s16[2 * g]);
                }
                acc[r][b] += half_bits_to_float(raw[r].D[0]) * tot;
            }
        }
    }
    // leaves: d*sc*q*x (q <= 63) and d*sc*32*x
    template <int B, int R, class XV>
    __device__ __forceinline__ static void bound(const Raw (&raw)[R], int u, const XV& xv, float (&bacc)[R][B]) {
        const int h = u >> 1, rr = u & 1;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float d = fabsf(half_bits_to_float(raw[r].D[0])) * 95.f;
            float k[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint32_t sw = raw[r].S[g >> 1] >> (8 * (rr + 2 * (g & 1)));
                k[g] = d * fabsf((float)(int)(int8_t)(sw & 0xFF));
            }
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const lds_f* a = xv.xa16 + b * xv.ld16 + 8 * h + rr;
                bacc[r][b] += k[0] * a[0] + k[1] * a[2] + k[2] * a[4] + k[3] * a[6];
            }
        }
    }
};

// ------------------------------------------------------------------ Q2_K
// unit (h, r'): qs bytes 32h+16r'+l hold the 2-bit codes of columns
// 128h + 32g + 16r' + l at bits 2g; scale byte 8h + 2g + r' (low nibble scale,
// high nibble min); d, dmin at 80, 82.  native.c:381-408
template <> struct Unit<T_Q2_K> {
    static constexpr int P = 4, PADI = 128;
    struct Raw { uint32_t Q[4]; uint32_t S[2]; uint32_t D[1]; };
    template <bool AL>
    __device__ __forceinline__ static void load(const uint8_t* blk, int u, Raw& raw) {
        const int h = u >> 1, rr = u & 1;
        ld_span<16, AL>(blk + 16 + 32 * h + 16 * rr, raw.Q);
        ld_span<8, AL>(blk + 8 * h, raw.S);
        ld_span<4, AL>(blk + 80, raw.D);
    }
    template <int B, int R, class XV>
    __device__ __forceinline__ static void dot(const Raw (&raw)[R], int u, const XV& xv,
                                               float (&acc)[R][B]) {
        const int h = u >> 1, rr = u & 1;
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int xo = 128 * h + 16 * rr;
            const lds_f* s16 = xv.xs16 + b * xv.ld16 + 8 * h + rr;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float ts = 0.f, tm = 0.f;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    uint32_t c[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k) c[k] = oand(raw[r].Q[k] >> (2 * g), 0x03030303u);
                    const float sg = dot_run<4>(c, xv.ptr(b, xo + 32 * g));
                    const uint32_t sb = (raw[r].S[g >> 1] >> (8 * (rr + 2 * (g & 1)))) & 0xFF;
                    ts += (float)(sb & 15) * sg;
                    tm += (float)(sb >> 4) * s16[2 * g];
                }
                acc[r][b] += half_bits_to_float(raw[r].D[0]) * ts - half_bits_to_float(raw[r].D[0] >> 16) * tm;
            }
        }
    }
    // leaves: d*sc*q*x (q <= 3) and dmin*m*x
    template <int B, int R, class XV>
    __device__ __forceinline__ static void bound(const Raw (&raw)[R], int u, const XV& xv, float (&bacc)[R][B]) {
        const int h = u >> 1, rr = u & 1;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float d = fabsf(half_bits_to_float(raw[r].D[0])) * 3.f, dm = fabsf(half_bits_to_float(raw[r].D[0] >> 16));
            float k[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint32_t sb = (raw[r].S[g >> 1] >> (8 * (rr + 2 * (g & 1)))) & 0xFF;
                k[g] = d * (float)(sb & 15) + dm * (float)(sb >> 4);
            }
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const lds_f* a = xv.xa16 + b * xv.ld16 + 8 * h + rr;
                bacc[r][b] += k[0] * a[0] + k[1] * a[2] + k[2] * a[4] + k[3] * a[6];
            }
        }
    }
};

// ------------------------------------------------------------------ Q3_K
// unit (h, r'): 2-bit codes at qs byte 32h+16r'+l bits 2g, high bit at hmask
// byte 16r'+l bit 4h+g (clear = subtract 4), 6-bit scale j = 8h+2g+r' from the
// 12 packed bytes at 96, d at 108.  native.c:129-171
template <> struct Unit<T_Q3_K> {
    static constexpr int P = 4, PADI = 128;
    struct Raw { uint32_t Q[4]; uint32_t M[4]; uint32_t S[3]; uint32_t D[1]; };
    template <bool AL>
    __device__ __forceinline__ static void load(const uint8_t* blk, int u, Raw& raw) {
        const int h = u >> 1, rr = u & 1;
        ld_span<16, AL, true>(blk + 32 + 32 * h + 16 * rr, raw.Q);
        ld_span<16, AL, true>(blk + 16 * rr, raw.M);
        ld_span<12, AL, true>(blk + 96, raw.S);
        ld_span<2, AL, true>(blk + 108, raw.D);
    }
    template <int B, int R, class XV>
    __device__ __forceinline__ static void dot(const Raw (&raw)[R], int u, const XV& xv,
                                               float (&acc)[R][B]) {
        const int h = u >> 1, rr = u & 1;
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int xo = 128 * h + 16 * rr;
            const lds_f* s16 = xv.xs16 + b * xv.ld16 + 8 * h + rr;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float tot = 0.f;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    uint32_t c[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        c[k] = oandor(raw[r].Q[k] >> (2 * g), 0x03030303u,
                                      ((raw[r].M[k] >> (4 * h + g)) & 0x01010101u) << 2);
                    const float sg = dot_run<4>(c, xv.ptr(b, xo + 32 * g));
                    // j = 8h + 2g + r': low nibble from byte 2g + r' (h selects the nibble),
                    // top two bits from byte 8 + (2g + r') % 4 at bit 2 * (2h + g / 2)
                    const uint32_t lb = (raw[r].S[g >> 1] >> (8 * (rr + 2 * (g & 1)))) & 0xFF;
                    const uint32_t low4 = h ? (lb >> 4) : (lb & 15);
                    const uint32_t hb = (raw[r].S[2] >> (8 * ((2 * g + rr) & 3))) & 0xFF;
                    const uint32_t hi2 = (hb >> (2 * (2 * h + (g >> 1)))) & 3;
                    const float sc = (float)(int)(low4 | (hi2 << 4)) - 32.f;
                    tot += sc * (sg - 4.f * s16[2 * g]);
                }
                acc[r][b] += half_bits_to_float(raw[r].D[0]) * tot;
            }
        }
    }
    // leaves: d*sc*c*x (c <= 7) and d*sc*4*x
    template <int B, int R, class XV>
    __device__ __forceinline__ static void bound(const Raw (&raw)[R], int u, const XV& xv, float (&bacc)[R][B]) {
        const int h = u >> 1, rr = u & 1;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float d = fabsf(half_bits_to_float(raw[r].D[0])) * 11.f;
            float k[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint32_t lb = (raw[r].S[g >> 1] >> (8 * (rr + 2 * (g & 1)))) & 0xFF;
                const uint32_t low4 = h ? (lb >> 4) : (lb & 15);
                const uint32_t hb = (raw[r].S[2] >> (8 * ((2 * g + rr) & 3))) & 0xFF;
                const uint32_t hi2 = (hb >> (2 * (2 * h + (g >> 1)))) & 3;
                k[g] = d * fabsf((float)(int)(low4 | (hi2 << 4)) - 32.f);
            }
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const lds_f* a = xv.xa16 + b * xv.ld16 + 8 * h + rr;
                bacc[r][b] += k[0] * a[0] + k[1] * a[2] + k[2] * a[4] + k[3] * a[6];
            }
        }
    }
};

// ------------------------------------------------------------------ IQ4_XS
// unit u: sub-blocks 2u and 2u+1; qs[16 ib + j] low nibble -> column 32ib + j,
// high -> 32ib + 16 + j; 6-bit scale ls from scales_l / scales_h, value
// d*(ls-32)*K[n].  native.c:364-379
template <> struct Unit<T_IQ4_XS> {
    static constexpr int P = 4, PADI = 64;
    struct Raw { uint32_t hd[2]; uint32_t q[8]; };
    template <bool AL>
    __device__ __forceinline__ static void load(const uint8_t* blk, int u, Raw& raw) {
        ld_span<8, AL>(blk, raw.hd);
        ld_span<32, AL>(blk + 8 + 32 * u, raw.q);
    }
    template <int B, int R, class XV>
    __device__ __forceinline__ static void dot(const Raw (&raw)[R], int u, const XV& xv,
                                               float (&acc)[R][B]) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const lds_f* s16 = xv.xs16 + b * xv.ld16 + 4 * u;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t sl = (raw[r].hd[1] >> (8 * u)) & 0xFF;
                const uint32_t sh = raw[r].hd[0] >> 16;
                float tot = 0.f;
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    const int ib = 2 * u + s;
                    const uint32_t ls = ((sl >> (4 * s)) & 15) | (((sh >> (2 * ib)) & 3u) << 4);
                    uint32_t lo[4], hi[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        lo[k] = iq4_lut4(raw[r].q[4 * s + k] & 0x0F0F0F0Fu);
                        hi[k] = iq4_lut4((raw[r].q[4 * s + k] >> 4) & 0x0F0F0F0Fu);
                    }
                    const float sv = dot_run<4>(lo, xv.ptr(b, 64 * u + 32 * s)) + dot_run<4>(hi, xv.ptr(b, 64 * u + 32 * s + 16));
                    const float xs = s16[2 * s] + s16[2 * s + 1];
                    tot += ((float)(int)ls - 32.f) * (sv - 128.f * xs);
                }
                acc[r][b] += half_bits_to_float(raw[r].hd[0]) * tot;
            }
        }
    }
    // leaves: d*(ls-32)*(K+128)*x (K+128 <= 241) and d*(ls-32)*128*x
    template <int B, int R, class XV>
    __device__ __forceinline__ static void bound(const Raw (&raw)[R], int u, const XV& xv, float (&bacc)[R][B]) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t sl = (raw[r].hd[1] >> (8 * u)) & 0xFF;
            const uint32_t sh = raw[r].hd[0] >> 16;
            const float d = fabsf(half_bits_to_float(raw[r].hd[0])) * 369.f;
            float k[2];
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                const int ib = 2 * u + s2;
                const uint32_t ls = ((sl >> (4 * s2)) & 15) | (((sh >> (2 * ib)) & 3u) << 4);
                k[s2] = d * fabsf((float)(int)ls - 32.f);
            }
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const lds_f* a = xv.xa16 + b * xv.ld16 + 4 * u;
                bacc[r][b] += k[0] * (a[0] + a[1]) + k[1] * (a[2] + a[3]);
            }
        }
    }
};

// ------------------------------------------------------------------ 32-element blocks
// One unit per block.  NB = bytes of the block, OFF = byte offset of qs[0].
template <int T> struct Small;
template <> struct Small<T_Q4_0> { static constexpr int NB = 18; };
template <> struct Small<T_Q4_1> { static constexpr int NB = 20; };
template <> struct Small<T_Q5_0> { static constexpr int NB = 22; };
template <> struct Small<T_Q5_1> { static constexpr int NB = 24; };
template <> struct Small<T_Q8_0> { static constexpr int NB = 34; };
template <> struct Small<T_Q8_1> { static constexpr int NB = 36; };
template <> struct Small<T_IQ4_NL> { static constexpr int NB = 18; };

// dword k of a byte stream that starts `off` (even) bytes into w[]
template <int N>
__device__ __forceinline__ uint32_t at_off(const uint32_t (&w)[N], int k, int off) {
    const int i = off / 4 + k;
    return (off & 2) ? __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2u) : w[i];
}

#define PYRITE_SMALL_UNIT(T)                                                                         \
    template <> struct Unit<T> {                                                                     \
        static constexpr int P = 1, PADI = 32;                                                       \
        static constexpr int NB = Small<T>::NB;                                                      \
        struct Raw { uint32_t w[(NB + 3) / 4]; };                                                    \
        template <bool AL>                                                                           \
        __device__ __forceinline__ static void load(const uint8_t* blk, int, Raw& raw) {             \
            ld_span<NB, AL>(blk, raw.w);                                                             \
        }                                                                                            \
        template <int B, int R, class XV>                                                            \
        __device__ __forceinline__ static void dot(const Raw (&raw)[R], int, const XV& xv,           \
                                                   float (&acc)[R][B]) {                             \
            _Pragma("unroll") for (int b = 0; b < B; ++b) {                                          \
                const auto x0 = xv.ptr(b, 0), x16 = xv.ptr(b, 16);                                   \
                const lds_f* s16 = xv.xs16 + b * xv.ld16;                                            \
                const float xs = s16[0] + s16[1];                                                    \
                _Pragma("unroll") for (int r = 0; r < R; ++r)                                        \
                    acc[r][b] += small_dot<T>(raw[r].w, x0, x16, xs);                                \
            }                                                                                        \
        }                                                                                            \
        template <int B, int R, class XV>                                                            \
        __device__ __forceinline__ static void bound(const Raw (&raw)[R], int, const XV& xv,         \
                                                     float (&bacc)[R][B]) {                          \
            _Pragma("unroll") for (int r = 0; r < R; ++r) {                                          \
                const float k = small_coef<T>(raw[r].w);                                             \
                _Pragma("unroll") for (int b = 0; b < B; ++b) {                                      \
                    const lds_f* a = xv.xa16 + b * xv.ld16;                                          \
                    bacc[r][b] += k * (a[0] + a[1]);                                                 \
                }                                                                                    \
            }                                                                                        \
        }                                                                                            \
    };

// Q4_0: d | qs[16]; d * (q - 8).  native.c:281-288
template <typename PX>
__device__ __forceinline__ float small_dot_T_Q4_0(const uint32_t (&w)[5], PX x, PX x16, float xs) {
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t v = at_off(w, k, 2);
        lo[k] = oand(v, 0x0F0F0F0Fu);
        hi[k] = oand(v, 0xF0F0F0F0u);
    }
    const float s = dot_run<4>(lo, x) + 0.0625f * dot_run<4>(hi, x16);
    return half_bits_to_float(w[0]) * (s - 8.f * xs);
}
// IQ4_NL: d | qs[16]; d * K[n].  native.c:351-358
template <typename PX>
__device__ __forceinline__ float small_dot_T_IQ4_NL(const uint32_t (&w)[5], PX x, PX x16, float xs) {
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t v = at_off(w, k, 2);
        lo[k] = iq4_lut4(v & 0x0F0F0F0Fu);
        hi[k] = iq4_lut4((v >> 4) & 0x0F0F0F0Fu);
    }
    const float s = dot_run<4>(lo, x) + dot_run<4>(hi, x16);
    return half_bits_to_float(w[0]) * (s - 128.f * xs);
}
// Q4_1: d | m | qs[16]; d*q + m.  native.c:290-298
template <typename PX>
__device__ __forceinline__ float small_dot_T_Q4_1(const uint32_t (&w)[5], PX x, PX x16, float xs) {
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        lo[k] = oand(w[1 + k], 0x0F0F0F0Fu);
        hi[k] = oand(w[1 + k], 0xF0F0F0F0u);
    }
    const float s = dot_run<4>(lo, x) + 0.0625f * dot_run<4>(hi, x16);
    return half_bits_to_float(w[0]) * s + half_bits_to_float(w[0] >> 16) * xs;
}
// Q5_0: d | qh | qs[16]; d * (q5 - 16).  native.c:300-314
template <typename PX>
__device__ __forceinline__ float small_dot_T_Q5_0(const uint32_t (&w)[6], PX x, PX x16, float xs) {
    const uint32_t qh = at_off(w, 0, 2);
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t v = at_off(w, k, 6);
        lo[k] = oandor(v, 0x0F0F0F0Fu, spread4(qh >> (4 * k)) << 4);
        hi[k] = oandor(v >> 4, 0x0F0F0F0Fu, spread4(qh >> (16 + 4 * k)) << 4);
    }
    const float s = dot_run<4>(lo, x) + dot_run<4>(hi, x16);
    return half_bits_to_float(w[0]) * (s - 16.f * xs);
}
// Q5_1: d | m | qh | qs[16]; d*q5 + m.  native.c:316-328
template <typename PX>
__device__ __forceinline__ float small_dot_T_Q5_1(const uint32_t (&w)[6], PX x, PX x16, float xs) {
    const uint32_t qh = w[1];
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t v = w[2 + k];
        lo[k] = oandor(v, 0x0F0F0F0Fu, spread4(qh >> (4 * k)) << 4);
        hi[k] = oandor(v >> 4, 0x0F0F0F0Fu, spread4(qh >> (16 + 4 * k)) << 4);
    }
    const float s = dot_run<4>(lo, x) + dot_run<4>(hi, x16);
    return half_bits_to_float(w[0]) * s + half_bits_to_float(w[0] >> 16) * xs;
}
// Q8_0: d | i8 qs[32]; codes biased by +128 (xor 0x80) for unsigned conversion.  native.c:330-336
template <typename PX>
__device__ __forceinline__ float small_dot_T_Q8_0(const uint32_t (&w)[9], PX x, PX x16, float xs) {
    uint32_t c[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) c[k] = at_off(w, k, 2) ^ 0x80808080u;
    const float s = dot_run<8>(c, x);
    return half_bits_to_float(w[0]) * (s - 128.f * xs);
}
// Q8_1: d | s | i8 qs[32].  native.c:338-344
template <typename PX>
__device__ __forceinline__ float small_dot_T_Q8_1(const uint32_t (&w)[9], PX x, PX x16, float xs) {
    uint32_t c[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) c[k] = w[1 + k] ^ 0x80808080u;
    const float s = dot_run<8>(c, x);
    return half_bits_to_float(w[0]) * (s - 128.f * xs);
}

// Magnitude coefficient of a 32-element block for bound(): every product the
// block's small_dot forms for column i is at most coef * |x_i|.
template <int T, int N>
__device__ __forceinline__ float small_coef(const uint32_t (&w)[N]) {
    const float d = fabsf(half_bits_to_float(w[0]));
    if constexpr (T == T_Q4_0) return d * 23.f;                  // q <= 15, offset 8
    if constexpr (T == T_IQ4_NL) return d * 369.f;               // K + 128 <= 241, offset 128
    if constexpr (T == T_Q4_1) return d * 15.f + fabsf(half_bits_to_float(w[0] >> 16));
    if constexpr (T == T_Q5_0) return d * 47.f;                  // q <= 31, offset 16
    if constexpr (T == T_Q5_1) return d * 31.f + fabsf(half_bits_to_float(w[0] >> 16));
    if constexpr (T == T_Q8_0 || T == T_Q8_1) return d * 383.f;  // q + 128 <= 255, offset 128
    return 0.f;
}

template <int T, int N, typename PX>
__device__ __forceinline__ float small_dot(const uint32_t (&w)[N], PX x, PX x16, float xs) {
    if constexpr (T == T_Q4_0) return small_dot_T_Q4_0(w, x, x16, xs);
    if constexpr (T == T_IQ4_NL) return small_dot_T_IQ4_NL(w, x, x16, xs);
    if constexpr (T == T_Q4_1) return small_dot_T_Q4_1(w, x, x16, xs);
    if constexpr (T == T_Q5_0) return small_dot_T_Q5_0(w, x, x16, xs);
    if constexpr (T == T_Q5_1) return small_dot_T_Q5_1(w, x, x16, xs);
    if constexpr (T == T_Q8_0) return small_dot_T_Q8_0(w, x, x16, xs);
    if constexpr (T == T_Q8_1) return small_dot_T_Q8_1(w, x, x16, xs);
    return 0.f;
}

PYRITE_SMALL_UNIT(T_Q4_0)
PYRITE_SMALL_UNIT(T_Q4_1)
PYRITE_SMALL_UNIT(T_Q5_0)
PYRITE_SMALL_UNIT(T_Q5_1)
PYRITE_SMALL_UNIT(T_Q8_0)
PYRITE_SMALL_UNIT(T_Q8_1)
PYRITE_SMALL_UNIT(T_IQ4_NL)
#undef PYRITE_SMALL_UNIT

// ------------------------------------------------------------------ plain types
// Four consecutive elements per unit (the last unit of a row may be partial).
template <int T>
__device__ __forceinline__ float plain_elem(const uint8_t* p) {
    if constexpr (T == T_F32) return __uint_as_float(*reinterpret_cast<const uint32_t*>(p));
    if constexpr (T == T_F16) return half_bits_to_float(*reinterpret_cast<const uint16_t*>(p));
    if constexpr (T == T_BF16) return bf16_bits_to_float(*reinterpret_cast<const uint16_t*>(p));
    if constexpr (T == T_I8) return (float)(int)*reinterpret_cast<const int8_t*>(p);
    if constexpr (T == T_I16) return (float)(int)*reinterpret_cast<const int16_t*>(p);
    if constexpr (T == T_I32) return (float)*reinterpret_cast<const int32_t*>(p);
    if constexpr (T == T_I64) return (float)(double)*reinterpret_cast<const long long*>(p);
    if constexpr (T == T_F64) return (float)*reinterpret_cast<const double*>(p);
    return 0.f;
}

}  // namespace pyrite
