// MFMA dequant-GEMM for prefill-sized batches (gfx950):
//   Y[t][r] = sum_c dequant(W)[r][c] * X[t][c]   for t < batch
// (pyrite/kernels/native.c:518-555 applied to every token; fp32 accumulation).
//
// Operands and exact fp16 fragments are those of mx_traits.h: A = activations
// (MFMA row m = 2t + p, fp16 hi (p = 0) and lo (p = 1) parts of x[t]), B =
// weights built exactly from the block codes, D = per lane row r0 + n of W and
// token-parts 4g..4g+3.  The block scales are applied once per block (epi).
//
// Schedule: a workgroup owns 128 rows of W (each of its 4 waves 32 rows = two
// 16-row MFMA tiles) and 32 tokens (four 8-token A sub-tiles).  It walks K in
// chunks of 8 steps (256 columns): the chunk's activations are converted to
// fp16 hi/lo fragments in LDS once for the workgroup, and each wave decodes
// each weight block once into B fragments and multiplies them against all
// four token sub-tiles.  A wave loads its next block while it computes the
// current one.  Workgroups with the same rows and consecutive token tiles are
// adjacent in the grid, so the weights they share are read from HBM once.
// Each token's activations are staged scaled by a per-(token, chunk) power of
// two that brings their largest finite |x| into [2^14, 2^15) (no fp16
// overflow, full hi/lo precision at any scale); the block epilogue multiplies
// it back (exact).
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "dispatch.h"
#include "mx_traits.h"

namespace pyrite {

constexpr int kMgRows = 128;      // rows per workgroup
constexpr int kMgTok = 32;        // tokens per workgroup
constexpr int kMgSub = kMgTok / 8;
constexpr int kMgChunkSteps = 8;  // 32-column steps per staged chunk

struct MgArgs {
    const uint8_t* W;
    unsigned long long row_bytes;
    const float* X;
    unsigned long long ldx;
    float* Y;
    unsigned long long ldy;
    int rows, cols, batch;
    int row_tiles, tok_tiles;
};

__device__ __forceinline__ void mg_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int T, bool AL>
__global__ __launch_bounds__(256) void mg_kernel(const MgArgs a) {
    using F = Mx<T>;
    constexpr int BPC = kMgChunkSteps / F::STEPS > 0 ? kMgChunkSteps / F::STEPS : 1;  // blocks per chunk
    constexpr int CS = BPC * F::STEPS;                                               // steps per chunk
    constexpr int XI = CS * 4 * kMgTok / 256;  // staged items (8 values of one token) per thread
    __shared__ uint4 frag[CS * 4 * 64];
    __shared__ unsigned tok_max[2][kMgTok];  // per chunk parity: largest finite |x| per token

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, n = lane & 15;
    const int rt = blockIdx.x / a.tok_tiles, tt = blockIdx.x - rt * a.tok_tiles;
    const int tok0 = tt * kMgTok;
    const long long r0 = (long long)rt * kMgRows + 32 * w + n, r1 = r0 + 16;
    const uint8_t* rp0 = a.W + (r0 < a.rows ? r0 : a.rows - 1) * a.row_bytes;
    const uint8_t* rp1 = a.W + (r1 < a.rows ? r1 : a.rows - 1) * a.row_bytes;
    const int nblk = a.cols / F::BS;
    const int nchunk = (nblk + BPC - 1) / BPC;
    // staging role: token tl, column group xg (8 columns) of steps xs0 + 2k
    const int tl = tid & 31, xg = (tid >> 5) & 3, xs0 = tid >> 7;
    const bool tok_ok = tok0 + tl < a.batch;
    const float* xrow = a.X + (unsigned long long)(tok_ok ? tok0 + tl : 0) * a.ldx;

    f4v acc[kMgSub][2];
#pragma unroll
    for (int s = 0; s < kMgSub; ++s) acc[s][0] = acc[s][1] = f4v{0.f, 0.f, 0.f, 0.f};
    if (tid < kMgTok) tok_max[0][tid] = 0u;

    typename F::Raw ca, cb, na, nb;
    F::template load<AL>(rp0, g, ca);
    F::template load<AL>(rp1, g, cb);

    for (int ch = 0; ch < nchunk; ++ch) {
        const int b0 = ch * BPC;
        const int b1 = b0 + BPC < nblk ? b0 + BPC : nblk;
        const int s0 = b0 * F::STEPS, ns = (b1 - b0) * F::STEPS;
        unsigned* tmax = tok_max[ch & 1];
        // Stage the chunk: activations into registers, each token's largest
        // finite |x| into LDS, then fp16 hi/lo fragments of x * 2^-e with the
        // token's normalising exponent e (the epilogue multiplies by 2^e).
        float xv[XI][8];
        float mx = 0.f;
#pragma unroll
        for (int k = 0; k < XI; ++k) {
            const int st = xs0 + 2 * k;
            if (tok_ok && st < ns) {
                const float* q = xrow + mx_col<F>(s0 + st, xg);
                const float4 u = ld_x4(q), v = ld_x4(q + 4);
                xv[k][0] = u.x; xv[k][1] = u.y; xv[k][2] = u.z; xv[k][3] = u.w;
                xv[k][4] = v.x; xv[k][5] = v.y; xv[k][6] = v.z; xv[k][7] = v.w;
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) xv[k][i] = 0.f;
            }
            mx = fmaxf(mx, finite_max8(xv[k]));
        }
        mg_barrier();  // the previous chunk's fragments and maxima are consumed
        if (tid < kMgTok) tok_max[(ch + 1) & 1][tid] = 0u;
        if (mx > 0.f) atomicMax(&tmax[tl], __float_as_uint(mx));
        mg_barrier();
        {
            const int e = norm_exp(__uint_as_float(tmax[tl]));
            uint4* fp = frag + xg * 64 + (tl >> 3) * 16 + 2 * (tl & 7);
#pragma unroll
            for (int k = 0; k < XI; ++k) {
                const int st = xs0 + 2 * k;
                if (st < ns) {
                    uint4 hi, lo;
                    split8(xv[k], e, hi, lo);
                    fp[st * 256] = hi;
                    fp[st * 256 + 1] = lo;
                }
            }
        }
        mg_barrier();
        // the exponents of this lane's D rows (tokens 2g and 2g + 1 of each sub-tile)
        int te[kMgSub][2];
#pragma unroll
        for (int s = 0; s < kMgSub; ++s) {
            te[s][0] = norm_exp(__uint_as_float(tmax[s * 8 + 2 * g]));
            te[s][1] = norm_exp(__uint_as_float(tmax[s * 8 + 2 * g + 1]));
        }

        for (int b = b0; b < b1; ++b) {
            // next block (of this chunk or the next), clamped to the last block
            const int bn = b + 1 < nblk ? b + 1 : nblk - 1;
            F::template load<AL>(rp0 + (size_t)bn * F::BPB, g, na);
            F::template load<AL>(rp1 + (size_t)bn * F::BPB, g, nb);

            f4v D[kMgSub][2][F::NACC];
#pragma unroll
            for (int s = 0; s < kMgSub; ++s)
#pragma unroll
                for (int p = 0; p < F::NACC; ++p) D[s][0][p] = D[s][1][p] = f4v{0.f, 0.f, 0.f, 0.f};
            const uint4* fb = frag + (size_t)(b - b0) * F::STEPS * 4 * 64;
            typename MxPreOf<F>::type pa, pb;
            mx_prep<F>(ca, g, pa);
            mx_prep<F>(cb, g, pb);
#pragma unroll
            for (int st = 0; st < F::STEPS; ++st) {
                uint32_t ba[F::NACC][4], bb[F::NACC][4];
                mx_frag<F>(ca, pa, st, g, ba);
                mx_frag<F>(cb, pb, st, g, bb);
#pragma unroll
                for (int s = 0; s < kMgSub; ++s) {
                    const uint4 av = fb[(st * 4 + g) * 64 + s * 16 + n];
                    const uint32_t aw[4] = {av.x, av.y, av.z, av.w};
                    const h8v A = __builtin_bit_cast(h8v, aw);
#pragma unroll
                    for (int p = 0; p < F::NACC; ++p) {
                        D[s][0][p] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(h8v, ba[p]),
                                                                           D[s][0][p], 0, 0, 0);
                        D[s][1][p] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(h8v, bb[p]),
                                                                           D[s][1][p], 0, 0, 0);
                    }
                }
            }
#pragma unroll
            for (int s = 0; s < kMgSub; ++s) {
#pragma unroll
                for (int p = 0; p < F::NACC; ++p) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        f4v& q = D[s][h][p];
                        q[0] = __builtin_amdgcn_ldexpf(q[0], te[s][0]);
                        q[1] = __builtin_amdgcn_ldexpf(q[1], te[s][0]);
                        q[2] = __builtin_amdgcn_ldexpf(q[2], te[s][1]);
                        q[3] = __builtin_amdgcn_ldexpf(q[3], te[s][1]);
                    }
                }
                F::epi(ca, D[s][0], acc[s][0]);
                F::epi(cb, D[s][1], acc[s][1]);
            }
            ca = na;
            cb = nb;
        }
    }

    // D rows 4g..4g+3 = (token 2g: hi, lo), (token 2g + 1: hi, lo) of each sub-tile
#pragma unroll
    for (int s = 0; s < kMgSub; ++s) {
        const int t0 = tok0 + s * 8 + 2 * g;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const long long row = h ? r1 : r0;
            if (row >= a.rows) continue;
            const f4v v = acc[s][h];
            if (t0 < a.batch) a.Y[(unsigned long long)t0 * a.ldy + row] = v[0] + v[1];
            if (t0 + 1 < a.batch) a.Y[(unsigned long long)(t0 + 1) * a.ldy + row] = v[2] + v[3];
        }
    }
}

template <int T, bool AL>
static hipError_t mg_launch_t(const MgArgs& a, hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
    const unsigned wgs = (unsigned)((long long)a.row_tiles * a.tok_tiles);
    if (e0 || e1)
        hipExtLaunchKernelGGL((mg_kernel<T, AL>), dim3(wgs), dim3(256), 0, s, e0, e1, 0, a);
    else
        hipLaunchKernelGGL((mg_kernel<T, AL>), dim3(wgs), dim3(256), 0, s, a);
    return hipGetLastError();
}

int mg_launch(int type, const MatvecArgs& m, size_t batch, bool al, hipStream_t stream, hipEvent_t start,
              hipEvent_t stop) {
    const TypeGeo g = type_geo(type);
    MgArgs a;
    a.W = static_cast<const uint8_t*>(m.w);
    a.row_bytes = m.cols / g.bs * g.bpb;
    a.X = m.x;
    a.ldx = m.ldx;
    a.Y = m.y;
    a.ldy = m.ldy;
    a.rows = (int)m.rows;
    a.cols = (int)m.cols;
    if (batch > 0x7FFFFFFF) return -2;
    a.batch = (int)batch;
    a.row_tiles = (int)((m.rows + kMgRows - 1) / kMgRows);
    a.tok_tiles = (int)((batch + kMgTok - 1) / kMgTok);
    if ((long long)a.row_tiles * a.tok_tiles > 0x7FFFFFFFLL) return -2;
    hipError_t e = hipSuccess;
#define PYRITE_CASE(T)                                                                         \
    case T:                                                                                  \
        e = (al && Geo<T>::bpb % 4 == 0) ? mg_launch_t<T, (Geo<T>::bpb % 4 == 0)>(a, stream, start, stop) \
                                         : mg_launch_t<T, false>(a, stream, start, stop);    \
        break;
    switch (type) {
        PYRITE_CASE(T_Q4_0) PYRITE_CASE(T_Q4_1) PYRITE_CASE(T_Q5_0) PYRITE_CASE(T_Q5_1)
        PYRITE_CASE(T_Q8_0) PYRITE_CASE(T_Q8_1) PYRITE_CASE(T_Q2_K) PYRITE_CASE(T_Q3_K)
        PYRITE_CASE(T_Q4_K) PYRITE_CASE(T_Q5_K) PYRITE_CASE(T_Q6_K) PYRITE_CASE(T_IQ4_NL)
        PYRITE_CASE(T_IQ4_XS)
    default: return -1;
    }
#undef PYRITE_CASE
    return e == hipSuccess ? 0 : -4;
}

}  // namespace pyrite
