// VALU dequant-matvec kernel templates and their launch planning, shared by
// matvec.hip (plain matvec) and lmhead.hip (matvec with per-row error bounds).
//
// Y[b][row] = sum_c dequant(W)[row][c] * X[b][c] for every row of a verbatim
// GGUF matrix (rows x row_bytes), fp32 accumulation.  Mirrors the semantics of
// pyrite_matvec (pyrite/kernels/native.c:518-555) with fp32 instead of fp64
// arithmetic and a different summation order.
//
// Work decomposition: a workgroup is 4 (or 8, 16) wave64s.  A wave is split into
// 64/LPR row slots of LPR lanes (LPR = lanes per row, a power of two chosen so
// a row's units fill it); each slot owns R consecutive rows and its lanes
// stride over the units of those rows (a unit = one block, or a quarter of a
// 256-element super-block).  Lanes load whole units with dword-aligned 16-byte
// loads, decode in registers and accumulate in fp32; the slot then reduces
// with DPP lane sums.  Per-16-column sums of X (needed by formats with a block
// minimum or code offset) are built once per workgroup in LDS.
#pragma once

#include <hip/hip_ext.h>
#include <stdlib.h>

#include <type_traits>

#include "common.h"
#include "dispatch.h"
#include "mv_units.h"

namespace pyrite {

// One matrix of a grouped launch.  wg_begin is the first workgroup (blockIdx.x)
// assigned to this matrix; matrices occupy consecutive workgroup ranges.
struct MvDesc {
    const uint8_t* W;
    unsigned long long row_bytes;
    const float* X;
    unsigned long long ldx;
    float* Y;
    unsigned long long ldy;
    int rows;
    int cols;
    int lpr_log2;
    int wg_begin;  // first workgroup of this matrix
    int wg_count;  // workgroups assigned; each loops over row groups wg, wg + wg_count, ...
    int pad;
    float* Bnd;    // bound pass only: per-row magnitude sums, laid out like Y
    const int* xrow;   // XGather: token row of each batch vector (negative: zeros)
    const float* X2;   // XSwiglu: the up-projection rows (X holds the gate rows)
};

// How a workgroup fetches 16 activations (vector b, columns 16j..16j+15)
// when it stages them: fetch() issues the loads into F, finish() turns F into
// the 16 values.  XDirect: row b of X.  XGather: row xrow[b] of X, or zeros.
// XSwiglu: silu(X[b]) * X2[b] (pyrite/tensor_ops.py:509-510: v / (1 +
// exp(-v)) for v > -60, else 0) in fp32, as the MFMA experts compute it (a
// relative error of a few fp32 ulps, far inside the matvec tolerance).
struct XDirect {
    struct F { float4 v[4]; };
    __device__ __forceinline__ static void fetch(const MvDesc& d, int b, int j, F& f) {
        const float* p = d.X + b * d.ldx + 16 * j;
        f.v[0] = ld_x4(p); f.v[1] = ld_x4(p + 4); f.v[2] = ld_x4(p + 8); f.v[3] = ld_x4(p + 12);
    }
    __device__ __forceinline__ static void finish(const F& f, float4 (&v)[4]) {
        v[0] = f.v[0]; v[1] = f.v[1]; v[2] = f.v[2]; v[3] = f.v[3];
    }
};
struct XGather {
    struct F { float4 v[4]; bool missing; };
    __device__ __forceinline__ static void fetch(const MvDesc& d, int b, int j, F& f) {
        const int t = d.xrow[b];
        f.missing = t < 0;  // a missing row reads row 0 (always present) and becomes zeros
        const float* p = d.X + (unsigned long long)(f.missing ? 0 : t) * d.ldx + 16 * j;
        f.v[0] = ld_x4(p); f.v[1] = ld_x4(p + 4); f.v[2] = ld_x4(p + 8); f.v[3] = ld_x4(p + 12);
    }
    __device__ __forceinline__ static void finish(const F& f, float4 (&v)[4]) {
        const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = f.missing ? z : f.v[k];
    }
};
struct XSwiglu {
    struct F { float4 g[4], u[4]; };
    __device__ __forceinline__ static float act(float g, float u) {
        return g > -60.f ? g / (1.f + expf(-g)) * u : 0.f;
    }
    __device__ __forceinline__ static void fetch(const MvDesc& d, int b, int j, F& f) {
        const float* pg = d.X + b * d.ldx + 16 * j;
        const float* pu = d.X2 + b * d.ldx + 16 * j;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            f.g[k] = ld_x4(pg + 4 * k);
            f.u[k] = ld_x4(pu + 4 * k);
        }
    }
    __device__ __forceinline__ static void finish(const F& f, float4 (&v)[4]) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
            v[k] = make_float4(act(f.g[k].x, f.u[k].x), act(f.g[k].y, f.u[k].y), act(f.g[k].z, f.u[k].z),
                               act(f.g[k].w, f.u[k].w));
    }
};

constexpr int kMaxGroup = 16;

// Workgroup shape: 4 waves, or 8-16 where the staged activations would limit
// the workgroups per CU (see launch_group_r).
constexpr int kMvWaves = 4;
constexpr int kMvThreads = 64 * kMvWaves;
struct MvGroup {
    int n;
    MvDesc d[kMaxGroup];
};

// An empty use of every register of a loaded unit: the compiler must wait for
// the unit's loads before it, on every path that reaches it.
template <int R, class Raw>
__device__ __forceinline__ void consume(const Raw (&raw)[R]) {
    static_assert(sizeof(Raw) % 4 == 0, "units are whole dwords");
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t* w = reinterpret_cast<const uint32_t*>(&raw[r]);
#pragma unroll
        for (int i = 0; i < (int)(sizeof(Raw) / 4); ++i) asm volatile("" ::"v"(w[i]));
    }
}

// What a slot's leader lane does with each finished row: NoObs stores the
// logits (and bounds) to d.Y / d.Bnd; another observer (the fused LM head)
// may store them its own way and watch the values go by.  Called for rows
// below d.rows only.
struct NoObs {
    template <int B, int R>
    __device__ __forceinline__ void row(const MvDesc& d, long long r, int ri, const float (&acc)[R][B],
                                        const float (&bacc)[R][B], bool bd) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            d.Y[b * d.ldy + r] = acc[ri][b];
            if (bd) d.Bnd[b * d.ldy + r] = bacc[ri][b];
        }
    }
};

// XL: activations staged in LDS (padded, see XView) instead of read from
// global memory by every unit; used when B * cols fits the LDS budget.
// BD: also accumulate each row's magnitude sum (Unit::bound, or sum |w||x| for
// plain types) and store it to d.Bnd.
template <int T, int B, int R, bool AL, bool XL, bool BD, class XS = XDirect, int NW = kMvWaves, class OB = NoObs>
__device__ __forceinline__ void mv_body(const MvDesc& d, long long wg, float* smem, OB& ob) {
    static_assert(XL || std::is_same<XS, XDirect>::value, "indirect activations need LDS staging");
    constexpr int BS = Geo<T>::bs, BPB = Geo<T>::bpb;
    const uint8_t* __restrict__ W = d.W;
    const float* __restrict__ X = d.X;
    const int rows = d.rows, cols = d.cols, lpr_log2 = d.lpr_log2;
    const unsigned long long ldx = d.ldx;
    const int n16 = cols >> 4;

    // wave (and so wrow0 and the loop exits) in scalar registers: the loop
    // branches stay uniform instead of exec-masked
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int LPR = 1 << lpr_log2, nslot = 64 >> lpr_log2;
    const int slot = lane >> lpr_log2, li = lane & (LPR - 1);
    const long long rows_per_wg = (long long)NW * nslot * R;
    const long long wave_rows = (long long)nslot * R;
    const long long stride_rows = (long long)d.wg_count * rows_per_wg;  // rows between row groups of this workgroup
    long long wrow0 = (wg * NW + wave) * wave_rows;                       // first row of this wave (wave-uniform)
    long long row0 = wrow0 + (long long)slot * R;                         // first row of this lane's slot

    float acc[R][B], bacc[R][B];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < B; ++b) acc[r][b] = bacc[r][b] = 0.f;

    // reduce the slot's partial sums, store rows row0..row0+R-1, clear acc
    auto flush = [&](long long r0) {
        group_sum(acc, lpr_log2);
        if constexpr (BD) group_sum(bacc, lpr_log2);
        if (li == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (r0 + r < rows) ob.template row<B, R>(d, r0 + r, r, acc, bacc, BD);
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int b = 0; b < B; ++b) acc[r][b] = bacc[r][b] = 0.f;
    };

    if constexpr (BS > 1) {
        // Software pipeline over the lane's (row group, unit) sequence: the
        // next unit's weights (possibly of the next row group) are loaded
        // before the current unit is decoded, so every lane keeps two units
        // of loads in flight.  The unit count per row group is wave-uniform
        // (KU), which keeps the reduction converged.
        using Un = Unit<T>;
        using Raw = typename Un::Raw;
        constexpr int P = Un::P;
        static_assert((P & (P - 1)) == 0, "units per block must be a power of two");
        constexpr int PL = P == 4 ? 2 : 0;
        constexpr int PADI = Un::PADI;
        const int U = (cols / BS) * P;
        const int KU = (U + LPR - 1) >> lpr_log2;
        // Row pointers (clamped to the last row) of the current and the next row group.
        auto row_ptrs = [&](long long r0, const uint8_t* (&rp)[R]) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const long long rr = (r0 + r < rows) ? r0 + r : (long long)rows - 1;
                rp[r] = W + rr * d.row_bytes;
            }
        };
        const uint8_t* rp_cur[R];
        const uint8_t* rp_nxt[R];
        row_ptrs(row0, rp_cur);
        row_ptrs(row0 + stride_rows, rp_nxt);
        // Loads are issued unconditionally (unit index clamped to the row's
        // last unit, rows clamped to the last row) so that every path through
        // the loop has the same number of loads in flight and the waits before
        // a decode cover only the older loads.
        auto load_item = [&](Raw (&dst)[R], const uint8_t* const (&rp)[R], int u) {
            const unsigned uu = (unsigned)(u < U ? u : U - 1);
            const unsigned blk = uu >> PL, part = uu & (P - 1);
#pragma unroll
            for (int r = 0; r < R; ++r) Un::template load<AL>(rp[r] + (size_t)blk * BPB, (int)part, dst[r]);
        };
        // Per-16-column sums of X (and of |X| for BD; with XL, the padded copy
        // of X) in LDS, one pass.  The thread's first 16 activations are
        // loaded before the first weights, so waiting for them does not wait
        // for the weights (loads complete in order).
        lds_f* xs16 = (lds_f*)(smem);  // address-space cast: smem is LDS
        const int ldxl = cols + (cols / PADI) * 4;
        const int n16r = (B * n16 + 3) & ~3;
        lds_f* xa16 = xs16 + n16r;
        lds_f* xl = xs16 + (BD ? 2 * n16r : n16r);
        const int i0 = (int)threadIdx.x < B * n16 ? (int)threadIdx.x : 0;
        typename XS::F xf0;
        XS::fetch(d, i0 / n16, i0 - (i0 / n16) * n16, xf0);

        Raw ra[R], rb[R];
        load_item(ra, rp_cur, li);  // first weights in flight while the activations are staged

        for (int i = threadIdx.x; i < B * n16; i += blockDim.x) {
            const int b = i / n16, j = i - b * n16;
            float4 v4[4];
            if (i == (int)threadIdx.x) {
                XS::finish(xf0, v4);
            } else {
                typename XS::F xf;
                XS::fetch(d, b, j, xf);
                XS::finish(xf, v4);
            }
            const float4 a = v4[0], c = v4[1], e = v4[2], f = v4[3];
            xs16[i] = (((a.x + a.y) + (a.z + a.w)) + ((c.x + c.y) + (c.z + c.w))) +
                      (((e.x + e.y) + (e.z + e.w)) + ((f.x + f.y) + (f.z + f.w)));
            if constexpr (BD)
                xa16[i] = (((fabsf(a.x) + fabsf(a.y)) + (fabsf(a.z) + fabsf(a.w))) +
                           ((fabsf(c.x) + fabsf(c.y)) + (fabsf(c.z) + fabsf(c.w)))) +
                          (((fabsf(e.x) + fabsf(e.y)) + (fabsf(e.z) + fabsf(e.w))) +
                           ((fabsf(f.x) + fabsf(f.y)) + (fabsf(f.z) + fabsf(f.w))));
            if constexpr (XL) {
                // 16 columns never straddle a pad (PADI is a multiple of 16)
                lds_f* q = xl + b * ldxl + 16 * j + (16 * j / PADI) * 4;
                st_x4(q, a); st_x4(q + 4, c); st_x4(q + 8, e); st_x4(q + 12, f);
            }
        }
        __syncthreads();
        if (wrow0 >= rows) return;

        XView<XL, PADI> xv;
        xv.ldx = XL ? (size_t)ldxl : (size_t)ldx;
        xv.ld16 = n16;
        auto dot_item = [&](const Raw (&src)[R], int u) {
            const unsigned blk = (unsigned)u >> PL, part = (unsigned)u & (P - 1);
            if constexpr (XL) xv.x = xl + blk * BS + (blk * BS / PADI) * 4;
            else xv.x = X + (size_t)blk * BS;
            xv.xs16 = xs16 + blk * (BS / 16);
            Un::template dot<B, R>(src, (int)part, xv, acc);
            if constexpr (BD) {
                xv.xa16 = xa16 + blk * (BS / 16);
                Un::template bound<B, R>(src, (int)part, xv, bacc);
            }
        };
        int k = 0;
        // one pipeline step: decode cur (unit k), with unit k+1 loaded into nxt; true when done
        auto step = [&](Raw (&cur)[R], Raw (&nxt)[R]) -> bool {
            const int u = li + (k << lpr_log2);
            const bool adv = (k + 1 == KU);
            const int un = adv ? li : u + LPR;
            const uint8_t* rpl[R];
#pragma unroll
            for (int r = 0; r < R; ++r) rpl[r] = adv ? rp_nxt[r] : rp_cur[r];
            load_item(nxt, rpl, un);
            if (u < U) dot_item(cur, u);
            // Every path waits for cur's loads here (a no-op after a decode).
            // Without it the path that skips the decode leaves them pending,
            // and the compiler's merged wait at the loop top drains nxt too.
            consume(cur);
            if (adv) {
                flush(row0);
                wrow0 += stride_rows;
                if (wrow0 >= rows) {
                    consume(nxt);  // likewise for the exit edge the loop shares with its latch
                    return true;
                }
                row0 += stride_rows;
#pragma unroll
                for (int r = 0; r < R; ++r) rp_cur[r] = rp_nxt[r];
                row_ptrs(row0 + stride_rows, rp_nxt);
                k = 0;
            } else {
                ++k;
            }
            return false;
        };
        for (;;) {
            if (step(ra, rb)) break;
            if (step(rb, ra)) break;
        }
    } else {
        if (wrow0 >= rows) return;
        for (;;) {
            const int U = (cols + 3) >> 2;
            const uint8_t* rp[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const long long rr = (row0 + r < rows) ? row0 + r : (long long)rows - 1;
                rp[r] = W + rr * d.row_bytes;
            }
            for (int u = li; u < U; u += LPR) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int col = 4 * u + e;
                    if (col < cols) {
#pragma unroll
                        for (int r = 0; r < R; ++r) {
                            const float w = plain_elem<T>(rp[r] + (size_t)col * BPB);
#pragma unroll
                            for (int b = 0; b < B; ++b) {
                                acc[r][b] = fmaf(w, X[b * ldx + col], acc[r][b]);
                                if constexpr (BD) bacc[r][b] = fmaf(fabsf(w), fabsf(X[b * ldx + col]), bacc[r][b]);
                            }
                        }
                    }
                }
            }
            flush(row0);
            wrow0 += stride_rows;
            if (wrow0 >= rows) break;
            row0 += stride_rows;
        }
    }
}

// NW waves per workgroup: 4, or 8-16 for launches whose staged activations
// would otherwise limit the workgroups per CU (long rows): then one copy of x
// in LDS serves 8-16 waves.
// XS: how activations are fetched while staged (XDirect; XSwiglu stages
// silu(gate) * up for a down projection, which needs XL).
template <int T, int B, int R, bool AL, bool XL, bool BD, int NW = kMvWaves, class XS = XDirect>
__global__ __launch_bounds__(64 * NW) void mv_kernel(const MvGroup g) {
    extern __shared__ float smem[];
    int i = 0;
    while (i + 1 < g.n && (int)blockIdx.x >= g.d[i + 1].wg_begin) ++i;
    NoObs ob;
    mv_body<T, B, R, AL, XL, BD, XS, NW>(g.d[i], (long long)blockIdx.x - g.d[i].wg_begin, smem, ob);
}

// ---------------------------------------------------------------- launcher

static int log2_ceil(long long v) {
    int l = 0;
    while ((1LL << l) < v) ++l;
    return l;
}

template <int T>
static long long units_per_row(int cols) {
    constexpr int BS = Geo<T>::bs;
    if constexpr (BS > 1) return (long long)(cols / BS) * Unit<T>::P;
    else return (cols + 3) / 4;
}

// A launch uses at most as many workgroups as the device holds at once
// (persistent workgroups): each loops over row groups, so the per-workgroup
// prologue (activations and their 16-column sums staged in LDS) is paid once
// per resident workgroup instead of once per row group.
struct DevInfo {
    int cus;
    size_t lds_per_cu;
};
static const DevInfo& dev_info() {
    static const DevInfo info = [] {
        DevInfo i{256, 160 * 1024};
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess) {
            if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) i.cus = v;
            if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) == hipSuccess && v > 0)
                i.lds_per_cu = (size_t)v;
        }
        return i;
    }();
    return info;
}

// Workgroups of one kernel instance resident per CU, from its register use.
template <int T, int B, int R, bool AL, bool XL, bool BD, int NW = kMvWaves, class XS = XDirect>
static int wgs_per_cu_regs() {
    static const int n = [] {
        int v = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, mv_kernel<T, B, R, AL, XL, BD, NW, XS>, 64 * NW, 0) !=
                hipSuccess ||
            v < 1)
            v = 1;
        return v;
    }();
    return n;
}

// PYRITE_MATVEC_WAVES=4 keeps every VALU launch on 4-wave workgroups.
static int matvec_waves_env() {
    static const int v = [] {
        const char* e = getenv("PYRITE_MATVEC_WAVES");
        return e ? atoi(e) : 0;
    }();
    return v;
}

// Optional tuning override of the units per lane (PYRITE_MATVEC_KU = 1, 2,
// 4, 8 or 16); unset means "choose".
static int ku_override() {
    static const int v = [] {
        const char* e = getenv("PYRITE_MATVEC_KU");
        return e ? atoi(e) : 0;
    }();
    return v;
}

// Slot geometry for one matrix: lanes per row = the row's units split over
// KU units per lane, KU = 1 for short rows (up to 32 units) and 2 otherwise,
// capped at 64 lanes.  Measured on MI355X, short rows (LM head, 1024-column
// projections) are fastest with one unit per lane (most slots in flight);
// longer rows gain a little from amortising the per-row reduction over two.
static int plan_lpr(long long U) {
    int ku = U <= 32 ? 1 : 2;
    if (const int forced = ku_override()) ku = forced;
    const long long per_lane = (U + ku - 1) / ku;
    return log2_ceil(per_lane < 64 ? per_lane : 64);
}

template <int T, int B, int R, bool AL, bool XL, bool BD, int NW = kMvWaves, class XS = XDirect>
static long long resident_wgs(size_t lds) {
    const DevInfo& di = dev_info();
    long long per_cu = wgs_per_cu_regs<T, B, R, AL, XL, BD, NW, XS>();
    if (lds > 0 && (long long)(di.lds_per_cu / lds) < per_cu) per_cu = (long long)(di.lds_per_cu / lds);
    if (per_cu < 1) per_cu = 1;
    return per_cu * di.cus;
}

// LDS bytes of a launch: per-16-column sums (of x, and of |x| with BD), plus
// the padded activations when staged.
template <int T, int B, bool BD>
static size_t lds_bytes(int max_cols, bool xl) {
    if constexpr (Geo<T>::bs == 1) {
        return 0;
    } else {
        const size_t n16r = ((size_t)B * (max_cols / 16) + 3) & ~size_t(3);
        size_t n = (BD ? 2 : 1) * n16r * sizeof(float);
        if (xl) {
            constexpr int PADI = Unit<T>::PADI;
            n += (size_t)B * (max_cols + (max_cols / PADI) * 4) * sizeof(float);
        }
        return n;
    }
}
template <int T, int B, bool BD>
static bool use_xl(int max_cols) {
    return Geo<T>::bs > 1 && lds_bytes<T, B, BD>(max_cols, true) <= 65536;
}
// The plain matvec also stages batch-1/2 activations of long rows in up to
// kMvXlMax bytes of LDS (one 8- or 16-wave workgroup per CU; the launch
// raises the kernel's dynamic LDS limit).
constexpr int kMvXlMax = 144 * 1024;
template <int T, int B, bool BD>
static bool use_xl_mv(int max_cols) {
    if (use_xl<T, B, BD>(max_cols)) return true;
    return Geo<T>::bs > 1 && B <= 2 && !BD && lds_bytes<T, B, BD>(max_cols, true) <= (size_t)kMvXlMax;
}

// Slot shape of one matrix (rows per slot R, lanes per row), a function of
// the matrix only, so a matrix gives bit-identical results whether it is
// launched alone or in a group.  One row per slot.
struct MatShape {
    int R;
    int lpr_log2;
};
template <int T, int B, bool AL>
static MatShape mat_shape(int rows, int cols) {
    (void)rows;
    return MatShape{1, plan_lpr(units_per_row<T>(cols))};
}

// Fill wg_begin / wg_count (lpr_log2 is already set) and return the total
// number of workgroups (at most cap).  Each matrix gets workgroups in
// proportion to its weight bytes, never more than it has row groups.
static long long plan_group(MvGroup& g, int R, long long cap, int nw = kMvWaves) {
    double total_bytes = 0;
    for (int i = 0; i < g.n; ++i) total_bytes += (double)g.d[i].rows * (double)g.d[i].row_bytes;
    long long wg = 0;
    for (int i = 0; i < g.n; ++i) {
        const double frac = ((double)g.d[i].rows * (double)g.d[i].row_bytes) / (total_bytes > 0 ? total_bytes : 1.0);
        long long share = (long long)((double)cap * frac);
        if (share < 1) share = 1;
        const long long rows_per_wg = (long long)nw * (64 >> g.d[i].lpr_log2) * R;
        const long long need = (g.d[i].rows + rows_per_wg - 1) / rows_per_wg;
        const long long cnt = need < share ? need : share;
        g.d[i].wg_begin = (int)wg;
        g.d[i].wg_count = (int)cnt;
        wg += cnt;
    }
    return wg;
}

// Optional start/stop events are recorded by the launch itself
// (hipExtLaunchKernelGGL), so they bracket the kernel's execution on the GPU.
struct LaunchEvents {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};

template <int T, int B, int R, bool AL, bool XL, bool BD, int NW, class XS = XDirect>
static hipError_t launch_group_w(MvGroup g, size_t lds, hipStream_t stream, LaunchEvents ev) {
    if (lds > 65536) {
        static const hipError_t attr =
            hipFuncSetAttribute(reinterpret_cast<const void*>(&mv_kernel<T, B, R, AL, XL, BD, NW, XS>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, kMvXlMax);
        if (attr != hipSuccess) return attr;
    }
    const long long wgs = plan_group(g, R, resident_wgs<T, B, R, AL, XL, BD, NW, XS>(lds), NW);
    if (wgs <= 0 || wgs > 0x7FFFFFFF) return hipErrorInvalidValue;
    if (ev.start || ev.stop)
        hipExtLaunchKernelGGL((mv_kernel<T, B, R, AL, XL, BD, NW, XS>), dim3((unsigned)wgs), dim3(64 * NW),
                              (uint32_t)lds, stream, ev.start, ev.stop, 0, g);
    else
        hipLaunchKernelGGL((mv_kernel<T, B, R, AL, XL, BD, NW, XS>), dim3((unsigned)wgs), dim3(64 * NW), lds, stream,
                           g);
    return hipGetLastError();
}

// Staged activations that hold a CU below the workgroups its registers allow
// (long rows) switch batch-1 launches to 16-wave workgroups and batch-2
// launches to 8-wave ones (16 waves would cap them at 128 VGPRs and spill).
template <int T, int B, int R, bool AL, bool XL, bool BD, class XS = XDirect>
static hipError_t launch_group_r(MvGroup g, size_t lds, hipStream_t stream, LaunchEvents ev) {
    if constexpr (XL && B <= 2 && !BD) {
        constexpr int NW = B == 1 ? 16 : 8;
        const DevInfo& di = dev_info();
        const long long by_regs = wgs_per_cu_regs<T, B, R, AL, XL, BD, kMvWaves, XS>();
        if (lds > 0 && (long long)(di.lds_per_cu / lds) < by_regs && lds <= di.lds_per_cu &&
            matvec_waves_env() != 4 && wgs_per_cu_regs<T, B, R, AL, XL, BD, NW, XS>() >= 1)
            return launch_group_w<T, B, R, AL, XL, BD, NW, XS>(g, lds, stream, ev);
    }
    return launch_group_w<T, B, R, AL, XL, BD, kMvWaves, XS>(g, lds, stream, ev);
}

template <int T, int B, int R, bool AL, bool BD, class XS = XDirect>
static hipError_t launch_group_rx(const MvGroup& g, hipStream_t stream, LaunchEvents ev) {
    int max_cols = 0;
    for (int i = 0; i < g.n; ++i) max_cols = g.d[i].cols > max_cols ? g.d[i].cols : max_cols;
    if constexpr (Geo<T>::bs > 1) {
        if (use_xl_mv<T, B, BD>(max_cols))
            return launch_group_r<T, B, R, AL, true, BD, XS>(g, lds_bytes<T, B, BD>(max_cols, true), stream, ev);
    }
    if constexpr (std::is_same<XS, XDirect>::value)
        return launch_group_r<T, B, R, AL, false, BD>(g, lds_bytes<T, B, BD>(max_cols, false), stream, ev);
    else
        return hipErrorInvalidValue;  // indirect activations are only staged
}

template <int T, int B, bool AL, bool BD, class XS = XDirect>
static hipError_t launch_group(const MvGroup& g, hipStream_t stream, LaunchEvents ev) {
    MvGroup sg = g;
    for (int i = 0; i < sg.n; ++i) sg.d[i].lpr_log2 = mat_shape<T, B, AL>(sg.d[i].rows, sg.d[i].cols).lpr_log2;
    return launch_group_rx<T, B, 1, AL, BD, XS>(sg, stream, ev);
}

// Batch chunks 1, 2, 4 and 8; the SwiGLU-staged down projection (XSwiglu)
// exists for chunks of 1 and 2 and the block formats.
template <int T, bool AL, bool BD, class XS = XDirect>
static hipError_t launch_type(int batch, const MvGroup& g, hipStream_t s, LaunchEvents ev) {
    if constexpr (std::is_same<XS, XDirect>::value) {
        switch (batch) {
        case 1: return launch_group<T, 1, AL, BD>(g, s, ev);
        case 2: return launch_group<T, 2, AL, BD>(g, s, ev);
        case 4: return launch_group<T, 4, AL, BD>(g, s, ev);
        case 8: return launch_group<T, 8, AL, BD>(g, s, ev);
        default: return hipErrorInvalidValue;
        }
    } else if constexpr (Geo<T>::bs > 1 && !BD) {
        switch (batch) {
        case 1: return launch_group<T, 1, AL, BD, XS>(g, s, ev);
        case 2: return launch_group<T, 2, AL, BD, XS>(g, s, ev);
        default: return hipErrorInvalidValue;
        }
    } else {
        return hipErrorInvalidValue;
    }
}

// PYRITE_MATVEC_PATH=valu keeps matvecs on the VALU kernels (no MFMA).
static char matvec_path_env() {
    static const char c = [] {
        const char* v = getenv("PYRITE_MATVEC_PATH");
        return v ? v[0] : '\0';
    }();
    return c;
}

// Largest instantiated batch chunk (8, 4, 2, 1) not above `left` whose
// staged activations (column sums and the padded copy) fit LDS; else the
// largest whose column sums alone fit (activations then read from memory per
// unit, which is slower than two launches that stage them: measured 45 vs
// 2 x 17.5 us for a 4096 x 14336 Q6_K matrix at batch 2); 0 if none.
template <int T, bool BD>
static int valu_chunk_t(size_t left, size_t max_cols) {
    if constexpr (Geo<T>::bs == 1) {
        return left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
    } else {
        if (left >= 8 && use_xl_mv<T, 8, BD>((int)max_cols)) return 8;
        if (left >= 4 && use_xl_mv<T, 4, BD>((int)max_cols)) return 4;
        if (left >= 2 && use_xl_mv<T, 2, BD>((int)max_cols)) return 2;
        if (use_xl_mv<T, 1, BD>((int)max_cols)) return 1;
        const size_t sums1 = (BD ? 2 : 1) * (max_cols / 16) * sizeof(float);
        for (int cand : {8, 4, 2, 1})
            if ((size_t)cand <= left && cand * sums1 <= 65536) return cand;
        return 0;
    }
}
template <bool BD>
static int valu_chunk(int type, size_t left, size_t max_cols) {
#define PYRITE_CASE(T) \
    case T: return valu_chunk_t<T, BD>(left, max_cols);
    switch (type) {
        PYRITE_FOR_EACH_TYPE(PYRITE_CASE)
    default: return 0;
    }
#undef PYRITE_CASE
}

// Whether a chunk of c (1 or 2) vectors of max_cols columns stages its
// activations in LDS (the SwiGLU-staged matvec requires it).
static bool valu_staged(int type, int c, size_t max_cols) {
#define PYRITE_CASE(T) \
    case T: return c == 1 ? use_xl_mv<T, 1, false>((int)max_cols) : use_xl_mv<T, 2, false>((int)max_cols);
    switch (type) {
        PYRITE_FOR_EACH_TYPE(PYRITE_CASE)
    default: return false;
    }
#undef PYRITE_CASE
}

// VALU launches over batch chunks and groups of kMaxGroup matrices; bnd
// (BD only) holds one bound buffer per matrix, laid out like its y.
// XSwiglu: mats[i].x holds the gate rows and up[i] the up rows (same ldx);
// chunks are at most 2 vectors and must stage their activations in LDS.
template <bool BD, class XS = XDirect>
static int valu_group_launch(int type, const TypeGeo& g, bool al, const MatvecArgs* mats, float* const* bnd,
                             size_t n, size_t batch, size_t max_cols, hipStream_t stream, hipEvent_t start,
                             hipEvent_t stop, const float* const* up = nullptr) {
    constexpr bool kSwiglu = !std::is_same<XS, XDirect>::value;
    size_t done = 0;
    while (done < batch) {
        const int c = valu_chunk<BD>(type, kSwiglu && batch - done > 2 ? 2 : batch - done, max_cols);
        if (c == 0 || (kSwiglu && (c > 2 || !valu_staged(type, c, max_cols)))) return -2;
        for (size_t base = 0; base < n; base += kMaxGroup) {
            LaunchEvents ev;
            if (done == 0 && base == 0) ev.start = start;
            if (done + c >= batch && base + kMaxGroup >= n) ev.stop = stop;
            MvGroup grp;
            grp.n = (int)((n - base) < (size_t)kMaxGroup ? (n - base) : (size_t)kMaxGroup);
            for (int i = 0; i < grp.n; ++i) {
                const MatvecArgs& m = mats[base + i];
                MvDesc& dd = grp.d[i];
                dd.W = static_cast<const uint8_t*>(m.w);
                dd.row_bytes = m.cols / g.bs * g.bpb;
                dd.X = m.x + done * m.ldx;
                dd.ldx = m.ldx;
                dd.Y = m.y + done * m.ldy;
                dd.ldy = m.ldy;
                dd.rows = (int)m.rows;
                dd.cols = (int)m.cols;
                dd.pad = 0;
                dd.Bnd = BD ? bnd[base + i] + done * m.ldy : nullptr;
                dd.X2 = kSwiglu ? up[base + i] + done * m.ldx : nullptr;
            }
            hipError_t e = hipSuccess;
#define PYRITE_CASE(T)                                                                       \
    case T:                                                                                \
        e = al ? launch_type<T, (Geo<T>::bpb % 4 == 0), BD, XS>(c, grp, stream, ev)        \
               : launch_type<T, false, BD, XS>(c, grp, stream, ev);                        \
        break;
            switch (type) {
                PYRITE_FOR_EACH_TYPE(PYRITE_CASE)
            default: return -1;
            }
#undef PYRITE_CASE
            if (e != hipSuccess) return -4;
        }
        done += c;
    }
    return 0;
}

// Validate a group of same-type matrices (codes of pyrite/kernels/native.c:
// 496-525); on success sets *al (all weight buffers 4-byte aligned and the
// block size a multiple of 4) and *max_cols.
static int validate_group(const TypeGeo& g, const MatvecArgs* mats, size_t n, size_t batch, bool* al,
                          size_t* max_cols) {
    if (!g.valid) return -1;
    if (n == 0 || batch == 0) return -2;
    const bool quant = g.bs > 1;
    *al = (g.bpb % 4 == 0);
    *max_cols = 0;
    for (size_t i = 0; i < n; ++i) {
        const MatvecArgs& m = mats[i];
        if (m.rows == 0 || m.cols == 0 || m.cols % g.bs != 0) return -2;
        if (m.rows > 0x7FFFFFFF || m.cols > 0x7FFFFFFF) return -2;
        const size_t row_bytes = m.cols / g.bs * g.bpb;
        if (m.w_len != m.rows * row_bytes) return -3;
        if (!m.w || !m.x || !m.y || m.ldx < m.cols || m.ldy < m.rows) return -3;
        if (quant && ((reinterpret_cast<uintptr_t>(m.x) & 15u) || (m.ldx & 3u))) return -3;
        if (!quant && (reinterpret_cast<uintptr_t>(m.w) % g.bpb)) return -3;
        if (reinterpret_cast<uintptr_t>(m.w) & 3u) *al = false;
        if (m.cols > *max_cols) *max_cols = m.cols;
    }
    return 0;
}

}  // namespace pyrite
