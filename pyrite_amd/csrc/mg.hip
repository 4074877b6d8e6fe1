// MFMA dequant-GEMM for prefill-sized batches (gfx950):
//   Y[t][r] = sum_c dequant(W)[r][c] * X[t][c]   for t < batch
// (pyrite/kernels/native.c:518-555 applied to every token; fp32 accumulation).
//
// Operands of v_mfma_f32_16x16x32_f16 (lane l: m or n = l % 16, K-slot group
// g = l / 16): A = activations of 16 tokens (row m = token), one fragment for
// the fp16 "hi" parts of x * 2^-e_t and one for the "lo" parts; B = weights
// built exactly from the block codes (mx_traits.h); D = per lane weight row
// r0 + n and tokens 4g..4g+3.  The hi and the lo fragment are multiplied by
// the same B into the same accumulator, so a block's D holds one value per
// (token, row) and the block scales are applied once per block.
//
// Three launches:
//   mg_exp_kernel   one workgroup per token: the power of two e_t that brings
//                   the token's largest finite |x| into [2^14, 2^15);
//   mg_frag_kernel  x[t] * 2^-e_t as fp16 hi and lo A fragments, written in
//                   the order the GEMM reads them: XF[((xs * Gp + f) * 2 + p)
//                   * 64 + lane] is lane `lane`'s 16 bytes of part p (0 hi,
//                   1 lo) of fragment step xs for tokens 16f..16f+15 (1 KiB
//                   per fragment).  Fragment steps are the 32-column steps,
//                   and for formats with per-sub-block mins (MINSUM) one
//                   more per block: the tokens' sums over each 32-column
//                   sub-block times 2^-e_t-5, hi parts in K-slots 0..7 and lo
//                   parts in K-slots 8..15 of part 0;
//   mg_kernel       the GEMM.  A workgroup of 8 waves owns 256 rows of one
//                   matrix (32 per wave = two 16-row MFMA tiles) and 16 * TG
//                   tokens.  K is walked in chunks of 8 steps: the chunk's
//                   fragments go from XF into LDS by direct global -> LDS
//                   loads (no registers), one chunk ahead.  Each wave builds
//                   each weight block's B fragments once (codes loaded one
//                   block ahead into registers), reads the next step's A
//                   fragments from LDS while it multiplies the current ones,
//                   and multiplies every B against all TG token groups.
//                   MINSUM formats take their min term as one MFMA per block
//                   against the staged sums.  The result is scaled by 2^e_t
//                   once, at the end.
// Two waves per SIMD (at most 256 registers each) let one wave's fragment
// building run under the other's MFMAs.  Workgroups are mapped so that all
// token tiles of one row tile run on one XCD, next to each other: their
// shared weights are read into that XCD's L2 once.  Up to four matrices with
// the same activations and columns share a launch (row tiles concatenated).
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <type_traits>

#include "dispatch.h"
#include "mx_traits.h"

namespace pyrite {

constexpr int kMgWaves = 8;
constexpr int kMgWaveTiles = 2;                         // 16-row tiles per wave
constexpr int kMgRows = 16 * kMgWaveTiles * kMgWaves;   // rows per workgroup
constexpr int kMgChunk = 8;                             // 32-column steps staged per chunk
constexpr int kMgMaxMats = 4;

template <class F, class = void> struct MgMinSum : std::false_type {};
template <class F> struct MgMinSum<F, std::void_t<decltype(F::MINSUM)>> : std::bool_constant<F::MINSUM> {};

// fragment steps per block: the 32-column steps, plus the sums step (MINSUM)
template <class F>
constexpr int mg_xs_per_block() { return F::STEPS + (MgMinSum<F>::value ? 1 : 0); }

// 16-token groups per workgroup: up to 4 for MINSUM formats (one accumulator
// per block), 2 for the others (two), so that a wave fits in 256 registers.
// Launches whose 32-token workgroups fit in one pass over the CUs take 2.
template <class F>
constexpr int mg_tg_max() { return MgMinSum<F>::value ? 4 : 2; }

struct MgMat {
    const uint8_t* W;
    unsigned long long row_bytes;
    float* Y;
    unsigned long long ldy;
    int rows;
    int tile0;  // first row tile of this matrix in the launch
};

struct MgArgs {
    MgMat m[kMgMaxMats];
    int nmat;
    const uint4* XF;
    const int* texp;
    int Gp;  // 16-token groups per fragment step in XF (token tiles * TG)
    int cols, batch;
    int row_tiles, tok_tiles;
    int ksplit, kblocks;  // K parts and blocks per part (split K when the tiles alone leave CUs idle)
    int reduce;           // 1: the launch after a split-K launch, summing its parts into y
    float* part;          // [ksplit][row_tiles * tok_tiles][512 threads][TG * 2 * 4] partial sums
};

// ---------------------------------------------------------------- activations
// One workgroup per token: its largest finite |x|, every load issued before
// the reduction.
__global__ __launch_bounds__(256) void mg_exp_kernel(const float* __restrict__ X, unsigned long long ldx, int cols,
                                                     int* __restrict__ texp) {
    __shared__ float red[4];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float* row = X + (unsigned long long)t * ldx;
    float m = 0.f;
    for (int c0 = 4 * tid; c0 < cols; c0 += 1024 * 8) {
        float4 v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int c = c0 + 1024 * k;
            v[k] = c < cols ? ld_x4(row + c) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float a[4] = {fabsf(v[k].x), fabsf(v[k].y), fabsf(v[k].z), fabsf(v[k].w)};
#pragma unroll
            for (int i = 0; i < 4; ++i) m = fmaxf(m, a[i] <= 3.402823466e38f ? a[i] : 0.f);
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    if (tid == 0) texp[t] = norm_exp(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
}

// Workgroup (16-token group f, 256-column window sb): the 16 tokens' window
// is read row by row into LDS, then item (step s, K-slot group g, token m)
// writes the hi and lo 16 bytes of its 8 columns as lane 16 g + m of parts 0
// and 1 (two items per thread).  MINSUM formats (256-column blocks, K-slot
// map 1) also write the block's sums step: in part 0, lane group 0 holds the
// hi and lane group 1 the lo parts of the token's eight sub-block sums (times
// 2^-e_t-5), the other lanes and part 1 zeros.
template <int T>
__global__ __launch_bounds__(256) void mg_frag_kernel(const float* __restrict__ X, unsigned long long ldx, int cols,
                                                      int batch, const int* __restrict__ texp, uint4* __restrict__ XF,
                                                      int Gp) {
    using F = Mx<T>;
    constexpr bool MS = MgMinSum<F>::value;
    constexpr int KM = MxKMode<F>::value;
    constexpr int XPB = mg_xs_per_block<F>();
    constexpr int LD = 256 + 4;  // LDS row pitch (floats)
    static_assert(!MS || (F::STEPS == 8 && KM == 1), "sums step: 256-column blocks, K-slot map 1");
    __shared__ float xs[16 * LD];
    __shared__ float sums[MS ? 128 : 1];
    const int tid = threadIdx.x, nsteps = cols / 32, sg = (nsteps + 7) / 8;
    const int f = blockIdx.x / sg, sb = blockIdx.x - f * sg;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int q = tid + 256 * k, tr = q >> 6, c = 256 * sb + 4 * (q & 63);
        float4 u = make_float4(0.f, 0.f, 0.f, 0.f);
        if (16 * f + tr < batch && c < cols) u = ld_x4(X + (unsigned long long)(16 * f + tr) * ldx + c);
        *reinterpret_cast<float4*>(xs + tr * LD + 4 * (q & 63)) = u;
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int it = tid + 256 * h, sl = it >> 6, g = (it >> 4) & 3, m = it & 15;
        const int t = 16 * f + m;
        if (8 * sb + sl < nsteps) {
            const int off = KM == 1 ? 64 * g + 8 * sl : 32 * sl + 8 * g;
            const float4 u = *reinterpret_cast<const float4*>(xs + m * LD + off);
            const float4 w = *reinterpret_cast<const float4*>(xs + m * LD + off + 4);
            const float v[8] = {u.x, u.y, u.z, u.w, w.x, w.y, w.z, w.w};
            uint4 hi, lo;
            split8(v, t < batch ? texp[t] : 0, hi, lo);
            const int xstep = MS ? sb * XPB + sl : 8 * sb + sl;
            uint4* o = XF + ((size_t)xstep * Gp + f) * 128 + 16 * g + m;
            o[0] = hi;
            o[64] = lo;
        }
    }
    if constexpr (MS) {
        if (tid < 128) {
            // sub-block j = tid & 7 of token tid >> 3: columns 32 j .. 32 j + 31
            const float* q = xs + (tid >> 3) * LD + 32 * (tid & 7);
            float acc = 0.f;
#pragma unroll
            for (int k = 0; k < 32; k += 4) {
                const float4 v = *reinterpret_cast<const float4*>(q + k);
                acc += (v.x + v.y) + (v.z + v.w);
            }
            sums[tid] = acc;
        }
        __syncthreads();
        if (tid < 128) {
            const int p = tid >> 6, ln = tid & 63, g = ln >> 4, m = ln & 15;
            uint4 r = make_uint4(0u, 0u, 0u, 0u);
            if (p == 0 && g < 2) {
                const int tk = 16 * f + m;
                float sv[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) sv[j] = sums[m * 8 + j];
                uint4 hi, lo;
                split8(sv, (tk < batch ? texp[tk] : 0) + 5, hi, lo);
                r = g ? lo : hi;
            }
            XF[((size_t)(sb * XPB + 8) * Gp + f) * 128 + tid] = r;
        }
    }
}

// ---------------------------------------------------------------- GEMM
typedef __attribute__((address_space(3))) void lds_void;

// 64 lanes x 16 bytes from src (per lane) to dst .. dst + 1 KiB (wave-uniform
// LDS address, in M0).  Issued as inline assembly: the compiler then does not
// treat every later LDS read as a possible reader of this copy (it would put
// a wait for all outstanding loads before each, and so wait for the next
// chunk's copies before computing this one).  Completion is waited for
// explicitly (mg_wait_all) before the barrier that publishes the chunk.
__device__ __forceinline__ void lds_load_1k(const uint4* src, uint4* dst) {
    const uint32_t m = __builtin_amdgcn_readfirstlane(
        static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void*)(dst))));
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m) : "memory", "m0");
}
// s_waitcnt vmcnt(0) (expcnt and lgkmcnt unconstrained) as a builtin the
// compiler's own wait placement sees: it then knows every earlier load is done
__device__ __forceinline__ void mg_wait_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

__device__ __forceinline__ h8v as_h8(const uint4 v) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    return __builtin_bit_cast(h8v, w);
}

template <int T, bool AL, int TG>
__global__ __launch_bounds__(kMgWaves * 64) void mg_kernel(const MgArgs a) {
    using F = Mx<T>;
    constexpr bool MS = MgMinSum<F>::value;
    constexpr int NT = kMgWaveTiles;
    constexpr int NA = MS ? 1 : F::NACC;                                 // accumulators per block
    constexpr int BPC = F::STEPS >= kMgChunk ? 1 : kMgChunk / F::STEPS;  // blocks per chunk
    constexpr int XPB = mg_xs_per_block<F>();
    constexpr int CX = BPC * XPB;    // fragment steps per chunk
    constexpr int FS = 2 * TG;       // fragments per fragment step (groups x hi/lo)
    constexpr int CF = CX * FS;      // fragments per chunk
    // Super-block formats other than MINSUM ones (unaligned 84- to 210-byte
    // blocks): each wave copies its 32 rows' next block into its own LDS
    // region with aligned 16-byte direct loads (the 16-byte pieces that
    // overlap the block: never past the page of its last byte), and its
    // lanes read their spans from there.  Other formats load their spans
    // straight into registers, one block ahead.
    constexpr bool WL = F::BS == 256 && !MS;
    constexpr int WP = WL ? (15 + F::BPB + 4 + 15) / 16 : 1;  // 16-byte pieces per row region
    constexpr bool UA = !AL && F::BS == 256;
    __shared__ uint4 abuf[2][CF * 64];
    __shared__ uint4 wbuf[WL ? kMgWaves * 16 * NT * WP : 1];

    // XCD-aware order: workgroup b runs on XCD b % 8; logical tile L counts
    // each XCD's workgroups contiguously, so the token tiles of a row tile
    // share an XCD and run next to each other.
    const int N = a.row_tiles * a.tok_tiles * (a.reduce ? 1 : a.ksplit);
    const int bx = blockIdx.x, xcd = bx & 7, per = N >> 3, rem = N & 7;
    const int L = xcd * per + (xcd < rem ? xcd : rem) + (bx >> 3);
    // K part outermost: the workgroups of one part and row tile stay adjacent
    const int kp = L / (a.row_tiles * a.tok_tiles), Lt = L - kp * (a.row_tiles * a.tok_tiles);
    const int rt = Lt / a.tok_tiles, tt = Lt - rt * a.tok_tiles;

    // matrix of this row tile (workgroup-uniform)
    const uint8_t* W = a.m[0].W;
    unsigned long long row_bytes = a.m[0].row_bytes, ldy = a.m[0].ldy;
    float* Y = a.m[0].Y;
    int rows = a.m[0].rows, tile0 = 0;
#pragma unroll
    for (int k = 1; k < kMgMaxMats; ++k) {
        if (k < a.nmat && rt >= a.m[k].tile0) {
            W = a.m[k].W;
            row_bytes = a.m[k].row_bytes;
            ldy = a.m[k].ldy;
            Y = a.m[k].Y;
            rows = a.m[k].rows;
            tile0 = a.m[k].tile0;
        }
    }

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, n = lane & 15;
    const long long rbase = (long long)(rt - tile0) * kMgRows + 16 * NT * w + n;
    const uint8_t* rp[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const long long r = rbase + 16 * i;
        rp[i] = W + (r < rows ? r : rows - 1) * row_bytes;
    }
    // D rows 4g..4g+3 = tokens 4g..4g+3 of each group
    auto write_out = [&](auto value) {  // value(f, i, k): the (token, row) sum before scaling
#pragma unroll
        for (int f = 0; f < TG; ++f) {
            const int t0 = (tt * TG + f) * 16 + 4 * g;
            int ex[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) ex[k] = t0 + k < a.batch ? a.texp[t0 + k] : 0;
#pragma unroll
            for (int i = 0; i < NT; ++i) {
                const long long row = rbase + 16 * i;
                if (row >= rows) continue;
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (t0 + k < a.batch)
                        Y[(unsigned long long)(t0 + k) * ldy + row] = __builtin_amdgcn_ldexpf(value(f, i, k), ex[k]);
            }
        }
    };
    // Split K: a part's sums go to the part buffer with plain stores (thread
    // tid's TG x NT x 4 values, 16 bytes per (group, tile)); the launch after
    // it (reduce mode, one workgroup per tile) adds the parts in part order
    // (deterministic) and writes y.
    constexpr int PE = TG * NT * 4;
    const size_t ntile = (size_t)a.row_tiles * a.tok_tiles;
    const size_t pstride = ntile * (kMgWaves * 64) * PE;  // floats per K part
    if (a.reduce) {
        const float* col0 = a.part + ((size_t)Lt * (kMgWaves * 64) + tid) * PE;
        f4v tot[TG][NT];
#pragma unroll
        for (int f = 0; f < TG; ++f)
#pragma unroll
            for (int i = 0; i < NT; ++i) tot[f][i] = f4v{0.f, 0.f, 0.f, 0.f};
        for (int q = 0; q < a.ksplit; ++q) {
#pragma unroll
            for (int f = 0; f < TG; ++f)
#pragma unroll
                for (int i = 0; i < NT; ++i)
                    tot[f][i] += *reinterpret_cast<const f4v*>(col0 + (size_t)q * pstride + (f * NT + i) * 4);
        }
        write_out([&](int f, int i, int k) { return tot[f][i][k]; });
        return;
    }

    // this workgroup's K blocks [blo, bhi)
    const int nblk_all = a.cols / F::BS;
    const int blo = kp * a.kblocks;
    const int bhi = blo + a.kblocks < nblk_all ? blo + a.kblocks : nblk_all;
    const int nblk = bhi - blo;
    const int nchunk = (nblk + BPC - 1) / BPC;
    const int nxs = bhi * XPB;
    // this workgroup's groups are contiguous in each fragment step
    const uint4* xsrc = a.XF + (size_t)tt * FS * 64 + lane;

    // the chunk's fragments: fragment j = (fragment step j / FS, group and part j % FS)
    constexpr int KPW = (CF + kMgWaves - 1) / kMgWaves;  // copies per wave and chunk
    auto stage_k = [&](int ch, int buf, int k) {
        const int x0 = blo * XPB + ch * CX;
        const int nx = nxs - x0 < CX ? nxs - x0 : CX;
        const int j = w + kMgWaves * k;
        const int xl = j / FS, fl = j - xl * FS;
        if (j < CF && xl < nx) lds_load_1k(xsrc + ((size_t)(x0 + xl) * a.Gp * 2 + fl) * 64, &abuf[buf][j * 64]);
    };
    auto stage = [&](int ch, int buf) {
#pragma unroll
        for (int k = 0; k < KPW; ++k) stage_k(ch, buf, k);
    };

    // WL: this wave's row region; lane (row q / WP, piece q % WP) of copy k, q = 64 k + lane
    uint4* wreg = wbuf + w * 16 * NT * WP;
    auto wstage = [&](int blk) {
#pragma unroll
        for (int k = 0; k < (16 * NT * WP + 63) / 64; ++k) {
            const int q = 64 * k + lane, r = q / WP, pc = q - r * WP;
            const long long row = rbase - n + r;
            const uint8_t* bp = W + (row < rows ? row : rows - 1) * row_bytes + (size_t)blk * F::BPB;
            const uint8_t* a0 = bp - (reinterpret_cast<uintptr_t>(bp) & 15u);
            if (r < 16 * NT && a0 + 16 * pc < bp + F::BPB)
                lds_load_1k(reinterpret_cast<const uint4*>(a0) + pc, wreg + 64 * k);
        }
    };
    // WL: the block's bytes of tile i's row in the wave's region
    auto wrow = [&](int i, int blk) {
        const uintptr_t o = reinterpret_cast<uintptr_t>(rp[i] + (size_t)blk * F::BPB) & 15u;
        return reinterpret_cast<const uint8_t*>(wreg + (16 * i + n) * WP) + o;
    };

    typename F::Raw ca[NT], na[NT];
    if constexpr (WL) {
        wstage(blo);
    } else {
#pragma unroll
        for (int i = 0; i < NT; ++i) F::template load<AL, false, UA>(rp[i] + (size_t)blo * F::BPB, g, ca[i]);
    }
    stage(0, 0);

    f4v acc[TG][NT];
#pragma unroll
    for (int f = 0; f < TG; ++f)
#pragma unroll
        for (int i = 0; i < NT; ++i) acc[f][i] = f4v{0.f, 0.f, 0.f, 0.f};

    for (int ch = 0; ch < nchunk; ++ch) {
        // this chunk's fragments have landed (all waves), and every wave is
        // done with the buffer the next chunk goes into
        mg_wait_all();
        __syncthreads();
        if (ch + 1 < nchunk) stage(ch + 1, (ch + 1) & 1);
        const uint4* ab = abuf[ch & 1] + lane;
        const int b0 = blo + ch * BPC;
        const int b1 = b0 + BPC < bhi ? b0 + BPC : bhi;
        for (int b = b0; b < b1; ++b) {
            const int bn = b + 1 < bhi ? b + 1 : bhi - 1;
            if constexpr (WL) {
                // this block's spans out of the wave's region (landed: the
                // chunk began with vmcnt(0)), then the next block into it
#pragma unroll
                for (int i = 0; i < NT; ++i) F::template load<false, true>(wrow(i, b), g, ca[i]);
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                if (b + 1 < bhi) wstage(b + 1);
            } else {
#pragma unroll
                for (int i = 0; i < NT; ++i)
                    F::template load<AL, false, UA>(rp[i] + (size_t)bn * F::BPB, g, na[i]);
            }
            // keep the next block's loads here, a whole block ahead of their use
            __builtin_amdgcn_sched_barrier(0);
            typename MxPreOf<F>::type pre[NT];
#pragma unroll
            for (int i = 0; i < NT; ++i) mx_prep<F>(ca[i], g, pre[i]);
            // fragment (step st, group f, part p) of this block at fb[(st * FS + 2 f + p) * 64]
            const uint4* fb = ab + (b - b0) * XPB * FS * 64;
            f4v D[TG][NT][NA];
            // A fragments of the current step, and of the next one in flight
            uint4 Av[2][FS];
#pragma unroll
            for (int q = 0; q < FS; ++q) Av[0][q] = fb[q * 64];
#pragma unroll
            for (int st = 0; st < F::STEPS; ++st) {
                const int cur = st & 1;
                if (st + 1 < F::STEPS) {
#pragma unroll
                    for (int q = 0; q < FS; ++q) Av[cur ^ 1][q] = fb[((st + 1) * FS + q) * 64];
                } else if constexpr (MS) {
                    // the sums step: part 0 of each group
#pragma unroll
                    for (int f = 0; f < TG; ++f) Av[cur ^ 1][2 * f] = fb[(F::STEPS * FS + 2 * f) * 64];
                }
                uint32_t B[NT][NA][4];
#pragma unroll
                for (int i = 0; i < NT; ++i) {
                    if constexpr (MS) F::frag_main(ca[i], pre[i], st, B[i][0]);
                    else mx_frag<F>(ca[i], pre[i], st, g, B[i]);
                }
                // hi parts of every group first, then the lo parts: the two
                // products into one accumulator are never back to back
#pragma unroll
                for (int pt = 0; pt < 2; ++pt)
#pragma unroll
                    for (int f = 0; f < TG; ++f) {
                        const h8v A = as_h8(Av[cur][2 * f + pt]);
#pragma unroll
                        for (int i = 0; i < NT; ++i)
#pragma unroll
                            for (int p = 0; p < NA; ++p)
                                D[f][i][p] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                    A, __builtin_bit_cast(h8v, B[i][p]),
                                    (st == 0 && pt == 0) ? f4v{0.f, 0.f, 0.f, 0.f} : D[f][i][p], 0, 0, 0);
                    }
            }
            if constexpr (MS) {
                // acc += d D - dmin (sum_j 32 m_j * 2^-5 S_j), the sums' hi and
                // lo parts in K-slots 0..7 and 8..15 against 32 m_j in both
                constexpr int cm = F::STEPS & 1;  // Av buffer holding the sums
                float dm[NT];
                uint32_t Bm[NT][4];
#pragma unroll
                for (int i = 0; i < NT; ++i) {
                    const float d = F::dscale(ca[i]);
                    dm[i] = -F::mscale(ca[i]);
                    F::min_frag(ca[i], g, Bm[i]);
#pragma unroll
                    for (int f = 0; f < TG; ++f) {
                        f4v& q = acc[f][i];
#pragma unroll
                        for (int k = 0; k < 4; ++k) q[k] = fmaf(d, D[f][i][0][k], q[k]);
                    }
                }
#pragma unroll
                for (int f = 0; f < TG; ++f) {
                    const h8v A = as_h8(Av[cm][2 * f]);
#pragma unroll
                    for (int i = 0; i < NT; ++i)
                        D[f][i][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            A, __builtin_bit_cast(h8v, Bm[i]), f4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                }
#pragma unroll
                for (int f = 0; f < TG; ++f)
#pragma unroll
                    for (int i = 0; i < NT; ++i) {
                        f4v& q = acc[f][i];
#pragma unroll
                        for (int k = 0; k < 4; ++k) q[k] = fmaf(dm[i], D[f][i][0][k], q[k]);
                    }
            } else {
#pragma unroll
                for (int f = 0; f < TG; ++f)
#pragma unroll
                    for (int i = 0; i < NT; ++i) F::epi(ca[i], D[f][i], acc[f][i]);
            }
            if constexpr (!WL) {
#pragma unroll
                for (int i = 0; i < NT; ++i) ca[i] = na[i];
            }
        }
    }

    if (a.ksplit == 1) {
        write_out([&](int f, int i, int k) { return acc[f][i][k]; });
        return;
    }
    float* mine = a.part + (size_t)kp * pstride + ((size_t)Lt * (kMgWaves * 64) + tid) * PE;
#pragma unroll
    for (int f = 0; f < TG; ++f)
#pragma unroll
        for (int i = 0; i < NT; ++i) *reinterpret_cast<f4v*>(mine + (f * NT + i) * 4) = acc[f][i];
}

// ---------------------------------------------------------------- launch
// Activation fragments and exponents, one per device, grown on demand (never
// during stream capture; a replaced block stays allocated for graphs captured
// before).  Launches on one device must be ordered on one stream.
struct MgWorkspace {
    void* block = nullptr;
    size_t cap = 0;  // bytes
};
static MgWorkspace g_mg_ws[64];
// Split-K partial sums, one buffer per device; launches that split K on one
// device must be ordered on one stream.
static MgWorkspace g_mg_part[64];

// K parts of a launch whose tiles alone give `tiles` workgroups.  A launch of
// fewer than 192 tiles (under a pass over the 256 CUs) is split into the part
// count that minimises passes x blocks per part (one block added for
// the partial sums and their reduce launch), each part at least one staging
// chunk (bpc blocks) and two blocks long; larger launches are not split.
static void mg_split(long long tiles, int nblk, int bpc, int* ksplit, int* kblocks) {
    *ksplit = 1;
    *kblocks = nblk;
    if (tiles >= 192 || tiles < 1) return;
    const int kmin = bpc > 2 ? bpc : 2;
    long long best = nblk;  // one pass, whole rows
    for (int ks = 2; ks <= 64 && (nblk + ks - 1) / ks >= kmin; ++ks) {
        const int kb = (nblk + ks - 1) / ks, parts = (nblk + kb - 1) / kb;
        const long long cost = (tiles * parts + 255) / 256 * kb + 1;
        if (cost < best) {
            best = cost;
            *ksplit = parts;
            *kblocks = kb;
        }
    }
}

template <int T, bool AL, int TG>
static hipError_t mg_launch_t(MgArgs& a, const float* X, unsigned long long ldx, hipStream_t s, hipEvent_t e0,
                              hipEvent_t e1) {
    using F = Mx<T>;
    const int nsteps = a.cols / 32, nblk = a.cols / F::BS;
    const size_t frag_bytes = (size_t)nblk * mg_xs_per_block<F>() * a.Gp * 2048;
    const size_t need = frag_bytes + ((size_t)a.batch * sizeof(int) + 255) / 256 * 256;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    MgWorkspace& ws = g_mg_ws[dev];
    if (need > ws.cap && (e = workspace_grow(&ws.block, &ws.cap, need, false, s)) != hipSuccess) return e;
    uint4* XF = static_cast<uint4*>(ws.block);
    int* texp = reinterpret_cast<int*>(static_cast<uint8_t*>(ws.block) + frag_bytes);
    a.XF = XF;
    a.texp = texp;
    a.part = nullptr;
    a.reduce = 0;
    if (a.ksplit > 1) {
        const size_t ntile = (size_t)a.row_tiles * a.tok_tiles;
        const size_t pbytes = (size_t)a.ksplit * ntile * (kMgWaves * 64) * (TG * kMgWaveTiles * 4) * sizeof(float);
        MgWorkspace& wp = g_mg_part[dev];
        if (pbytes > wp.cap && (e = workspace_grow(&wp.block, &wp.cap, pbytes, false, s)) != hipSuccess) return e;
        a.part = static_cast<float*>(wp.block);
    }
    const dim3 gexp(a.batch), gfrag((unsigned)((long long)a.Gp * ((nsteps + 7) / 8)));
    if (e0)
        hipExtLaunchKernelGGL(mg_exp_kernel, gexp, dim3(256), 0, s, e0, nullptr, 0, X, ldx, a.cols, texp);
    else
        hipLaunchKernelGGL(mg_exp_kernel, gexp, dim3(256), 0, s, X, ldx, a.cols, texp);
    hipLaunchKernelGGL((mg_frag_kernel<T>), gfrag, dim3(256), 0, s, X, ldx, a.cols, a.batch, (const int*)texp, XF,
                       a.Gp);
    const unsigned ntile = (unsigned)((long long)a.row_tiles * a.tok_tiles);
    const unsigned wgs = ntile * (unsigned)a.ksplit;
    hipEvent_t ec = a.ksplit > 1 ? nullptr : e1;  // the launch that ends the set records the stop event
    if (ec)
        hipExtLaunchKernelGGL((mg_kernel<T, AL, TG>), dim3(wgs), dim3(kMgWaves * 64), 0, s, nullptr, ec, 0, a);
    else
        hipLaunchKernelGGL((mg_kernel<T, AL, TG>), dim3(wgs), dim3(kMgWaves * 64), 0, s, a);
    if (a.ksplit > 1) {
        MgArgs r = a;
        r.reduce = 1;
        if (e1)
            hipExtLaunchKernelGGL((mg_kernel<T, AL, TG>), dim3(ntile), dim3(kMgWaves * 64), 0, s, nullptr, e1, 0, r);
        else
            hipLaunchKernelGGL((mg_kernel<T, AL, TG>), dim3(ntile), dim3(kMgWaves * 64), 0, s, r);
    }
    return hipGetLastError();
}

// 16-token groups per workgroup for a launch of `row_tiles` row tiles
template <int T>
static int mg_tg_for(long long row_tiles, size_t batch) {
    constexpr int TM = mg_tg_max<Mx<T>>();
    // 32-token tiles when they still fit in one pass over the 256 CUs
    if (TM == 4 && row_tiles * (long long)((batch + 31) / 32) <= 256) return 2;
    return TM;
}

template <int T, bool AL>
static hipError_t mg_launch_tg(MgArgs& a, int tg, const float* X, unsigned long long ldx, hipStream_t s,
                               hipEvent_t e0, hipEvent_t e1) {
    if constexpr (mg_tg_max<Mx<T>>() == 4)
        if (tg == 4) return mg_launch_t<T, AL, 4>(a, X, ldx, s, e0, e1);
    return mg_launch_t<T, AL, 2>(a, X, ldx, s, e0, e1);
}

// Workgroups the GEMM launches would have for these matrices (one per
// 256-row tile, token tile and K part, sized as mg_group_launch sizes them),
// and the most blocks a workgroup walks (*kblocks).
long long mg_workgroups(int type, const MatvecArgs* mats, size_t n, size_t batch, int* kblocks) {
    const TypeGeo geo = type_geo(type);
    const int bpc = geo.bs >= 256 ? 1 : 256 / geo.bs;
    long long total = 0;
    *kblocks = 0;
    size_t i = 0;
    while (i < n) {
        size_t j = i + 1;
        while (j < n && j - i < (size_t)kMgMaxMats && mats[j].x == mats[i].x && mats[j].ldx == mats[i].ldx &&
               mats[j].cols == mats[i].cols)
            ++j;
        long long tiles = 0;
        for (size_t k = i; k < j; ++k) tiles += (long long)((mats[k].rows + kMgRows - 1) / kMgRows);
        int tg = 2;
#define PYRITE_CASE(T) case T: tg = mg_tg_for<T>(tiles, batch); break;
        switch (type) {
            PYRITE_CASE(T_Q4_0) PYRITE_CASE(T_Q4_1) PYRITE_CASE(T_Q5_0) PYRITE_CASE(T_Q5_1)
            PYRITE_CASE(T_Q8_0) PYRITE_CASE(T_Q8_1) PYRITE_CASE(T_Q2_K) PYRITE_CASE(T_Q3_K)
            PYRITE_CASE(T_Q4_K) PYRITE_CASE(T_Q5_K) PYRITE_CASE(T_Q6_K) PYRITE_CASE(T_IQ4_NL)
            PYRITE_CASE(T_IQ4_XS)
        default: break;
        }
#undef PYRITE_CASE
        const long long wt = tiles * (long long)((batch + 16 * tg - 1) / (16 * tg));
        int ks = 1, kb = 0;
        mg_split(wt, (int)(mats[i].cols / geo.bs), bpc, &ks, &kb);
        if (kb > *kblocks) *kblocks = kb;
        total += wt * ks;
        i = j;
    }
    return total;
}

// One launch set per run of consecutive matrices with the same activations
// and columns (at most kMgMaxMats each).
int mg_group_launch(int type, const MatvecArgs* mats, size_t n, size_t batch, bool al, hipStream_t stream,
                    hipEvent_t start, hipEvent_t stop) {
    const TypeGeo geo = type_geo(type);
    if (batch > 0x7FFFFFFF) return -2;
    size_t i = 0;
    while (i < n) {
        size_t j = i + 1;
        while (j < n && j - i < (size_t)kMgMaxMats && mats[j].x == mats[i].x && mats[j].ldx == mats[i].ldx &&
               mats[j].cols == mats[i].cols)
            ++j;
        MgArgs a{};
        a.nmat = (int)(j - i);
        long long tiles = 0;
        for (size_t k = i; k < j; ++k) {
            MgMat& d = a.m[k - i];
            d.W = static_cast<const uint8_t*>(mats[k].w);
            d.row_bytes = mats[k].cols / geo.bs * geo.bpb;
            d.Y = mats[k].y;
            d.ldy = mats[k].ldy;
            d.rows = (int)mats[k].rows;
            d.tile0 = (int)tiles;
            tiles += (long long)((mats[k].rows + kMgRows - 1) / kMgRows);
        }
        int tg = 0;
#define PYRITE_CASE(T) case T: tg = mg_tg_for<T>(tiles, batch); break;
        switch (type) {
            PYRITE_CASE(T_Q4_0) PYRITE_CASE(T_Q4_1) PYRITE_CASE(T_Q5_0) PYRITE_CASE(T_Q5_1)
            PYRITE_CASE(T_Q8_0) PYRITE_CASE(T_Q8_1) PYRITE_CASE(T_Q2_K) PYRITE_CASE(T_Q3_K)
            PYRITE_CASE(T_Q4_K) PYRITE_CASE(T_Q5_K) PYRITE_CASE(T_Q6_K) PYRITE_CASE(T_IQ4_NL)
            PYRITE_CASE(T_IQ4_XS)
        default: return -1;
        }
#undef PYRITE_CASE
        a.cols = (int)mats[i].cols;
        a.batch = (int)batch;
        a.row_tiles = (int)tiles;
        a.tok_tiles = (int)((batch + 16 * tg - 1) / (16 * tg));
        a.Gp = a.tok_tiles * tg;
        mg_split(tiles * a.tok_tiles, (int)(mats[i].cols / geo.bs), geo.bs >= 256 ? 1 : 256 / geo.bs, &a.ksplit,
                 &a.kblocks);
        if (tiles * a.tok_tiles * a.ksplit > 0x7FFFFFFFLL || (long long)a.Gp * ((a.cols / 32 + 7) / 8) > 0x7FFFFFFFLL)
            return -2;
        hipEvent_t e0 = i == 0 ? start : nullptr, e1 = j == n ? stop : nullptr;
        hipError_t e = hipSuccess;
#define PYRITE_CASE(T)                                                                                     \
    case T:                                                                                                \
        e = (al && Geo<T>::bpb % 4 == 0)                                                                   \
                ? mg_launch_tg<T, (Geo<T>::bpb % 4 == 0)>(a, tg, mats[i].x, mats[i].ldx, stream, e0, e1)  \
                : mg_launch_tg<T, false>(a, tg, mats[i].x, mats[i].ldx, stream, e0, e1);                   \
        break;
        switch (type) {
            PYRITE_CASE(T_Q4_0) PYRITE_CASE(T_Q4_1) PYRITE_CASE(T_Q5_0) PYRITE_CASE(T_Q5_1)
            PYRITE_CASE(T_Q8_0) PYRITE_CASE(T_Q8_1) PYRITE_CASE(T_Q2_K) PYRITE_CASE(T_Q3_K)
            PYRITE_CASE(T_Q4_K) PYRITE_CASE(T_Q5_K) PYRITE_CASE(T_Q6_K) PYRITE_CASE(T_IQ4_NL)
            PYRITE_CASE(T_IQ4_XS)
        default: return -1;
        }
#undef PYRITE_CASE
        if (e != hipSuccess) return -4;
        i = j;
    }
    return 0;
}

}  // namespace pyrite
