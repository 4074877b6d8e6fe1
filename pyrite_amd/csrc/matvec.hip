// Fused GGML dequantize x matvec for gfx950 (VALU path, batch 1..8).
//
// Y[b][row] = sum_c dequant(W)[row][c] * X[b][c] for every row of a verbatim
// GGUF matrix (rows x row_bytes), fp32 accumulation.  Mirrors the semantics of
// pyrite_matvec (pyrite/kernels/native.c:518-555) with fp32 instead of fp64
// arithmetic and a different summation order.
//
// Work decomposition: a workgroup is 4 wave64s.  A wave is split into
// 64/LPR row slots of LPR lanes (LPR = lanes per row, a power of two chosen so
// a row's units fill it); each slot owns R consecutive rows and its lanes
// stride over the units of those rows (a unit = one block, or a quarter of a
// 256-element super-block).  Lanes load whole units with dword-aligned 16-byte
// loads, decode in registers and accumulate in fp32; the slot then reduces
// with lane shuffles.  Per-16-column sums of X (needed by formats with a block
// minimum or code offset) are built once per workgroup in LDS.
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
};

constexpr int kMaxGroup = 16;
struct MvGroup {
    int n;
    MvDesc d[kMaxGroup];
};

// XL: activations staged in LDS (padded, see XView) instead of read from
// global memory by every unit; used when B * cols fits the LDS budget.
template <int T, int B, bool AL, bool XL>
__device__ __forceinline__ void mv_body(const MvDesc& d, long long wg, float* smem) {
    constexpr int R = (B <= 2) ? 2 : 1;
    constexpr int BS = Geo<T>::bs, BPB = Geo<T>::bpb;
    const uint8_t* __restrict__ W = d.W;
    const float* __restrict__ X = d.X;
    const int rows = d.rows, cols = d.cols, lpr_log2 = d.lpr_log2;
    const unsigned long long ldx = d.ldx;
    const int n16 = cols >> 4;
    lds_f* xs16 = (lds_f*)(smem);  // address-space cast: smem is LDS
    if constexpr (BS > 1) {
        for (int i = threadIdx.x; i < B * n16; i += blockDim.x) {
            const int b = i / n16, j = i - b * n16;
            const float* p = X + b * ldx + 16 * j;
            const float4 a = ld_x4(p), c = ld_x4(p + 4), e = ld_x4(p + 8), f = ld_x4(p + 12);
            xs16[i] = (((a.x + a.y) + (a.z + a.w)) + ((c.x + c.y) + (c.z + c.w))) +
                      (((e.x + e.y) + (e.z + e.w)) + ((f.x + f.y) + (f.z + f.w)));
        }
    }
    constexpr int PADI = [] {
        if constexpr (BS > 1) return Unit<T>::PADI;
        else return 32;
    }();
    const int ldxl = cols + (cols / PADI) * 4;
    lds_f* xl = xs16 + ((B * n16 + 3) & ~3);
    if constexpr (XL) {
        const int q = cols >> 2;
        for (int i = threadIdx.x; i < B * q; i += blockDim.x) {
            const int b = i / q, e = (i - b * q) * 4;
            st_x4(xl + b * ldxl + e + (e / PADI) * 4, ld_x4(X + b * ldx + e));
        }
    }
    if constexpr (BS > 1) __syncthreads();

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int LPR = 1 << lpr_log2, nslot = 64 >> lpr_log2;
    const int slot = lane >> lpr_log2, li = lane & (LPR - 1);
    const long long rows_per_wg = 4LL * nslot * R;
    for (long long rg = wg; rg * rows_per_wg < rows; rg += d.wg_count) {
        const long long wave_row0 = (rg * 4 + wave) * nslot * R;
        if (wave_row0 >= rows) break;
        const long long row0 = wave_row0 + (long long)slot * R;

        float acc[R][B];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int b = 0; b < B; ++b) acc[r][b] = 0.f;

        const uint8_t* rp[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const long long rr = (row0 + r < rows) ? row0 + r : (long long)rows - 1;
            rp[r] = W + rr * d.row_bytes;
        }

        if constexpr (BS > 1) {
            constexpr int P = Unit<T>::P;
            const int U = (cols / BS) * P;
            XView<XL, PADI> xv;
            xv.ldx = XL ? (size_t)ldxl : (size_t)ldx;
            xv.ld16 = n16;
            for (int u = li; u < U; u += LPR) {
                const int blk = u / P, part = u - blk * P;
                const uint8_t* bp[R];
#pragma unroll
                for (int r = 0; r < R; ++r) bp[r] = rp[r] + (size_t)blk * BPB;
                if constexpr (XL) xv.x = xl + blk * BS + (blk * BS / PADI) * 4;
                else xv.x = X + (size_t)blk * BS;
                xv.xs16 = xs16 + blk * (BS / 16);
                Unit<T>::template run<B, R, AL>(bp, part, xv, acc);
            }
        } else {
            const int U = (cols + 3) >> 2;
            for (int u = li; u < U; u += LPR) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int col = 4 * u + e;
                    if (col < cols) {
#pragma unroll
                        for (int r = 0; r < R; ++r) {
                            const float w = plain_elem<T>(rp[r] + (size_t)col * BPB);
#pragma unroll
                            for (int b = 0; b < B; ++b) acc[r][b] = fmaf(w, X[b * ldx + col], acc[r][b]);
                        }
                    }
                }
            }
        }

        for (int off = LPR >> 1; off > 0; off >>= 1)
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int b = 0; b < B; ++b) acc[r][b] += __shfl_xor(acc[r][b], off, 64);

        if (li == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (row0 + r < rows)
#pragma unroll
                    for (int b = 0; b < B; ++b) d.Y[b * d.ldy + row0 + r] = acc[r][b];
        }
    }
}

template <int T, int B, bool AL, bool XL>
__global__ __launch_bounds__(256) void mv_kernel(const MvGroup g) {
    extern __shared__ float smem[];
    int i = 0;
    while (i + 1 < g.n && (int)blockIdx.x >= g.d[i + 1].wg_begin) ++i;
    mv_body<T, B, AL, XL>(g.d[i], (long long)blockIdx.x - g.d[i].wg_begin, smem);
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

// Workgroups per launch to aim for: 8 per CU on a 256-CU MI355X.  A
// workgroup loops over row groups, so the per-workgroup prologue (x sums in
// LDS) is paid once per workgroup, not once per 8 rows.
constexpr long long kTargetWgs = 2048;

// Fill lpr_log2 / wg_begin / wg_count for B and return the total number of
// workgroups.  Each matrix gets workgroups in proportion to its weight bytes.
template <int T, int B>
static long long plan_group(MvGroup& g) {
    const int R = (B <= 2) ? 2 : 1;
    double total_bytes = 0;
    for (int i = 0; i < g.n; ++i) total_bytes += (double)g.d[i].rows * (double)g.d[i].row_bytes;
    long long wg = 0;
    for (int i = 0; i < g.n; ++i) {
        const long long U = units_per_row<T>(g.d[i].cols);
        g.d[i].lpr_log2 = log2_ceil(U < 64 ? U : 64);
        const long long rows_per_wg = 4LL * (64 >> g.d[i].lpr_log2) * R;
        const long long need = (g.d[i].rows + rows_per_wg - 1) / rows_per_wg;
        long long share = (long long)((double)kTargetWgs * ((double)g.d[i].rows * (double)g.d[i].row_bytes) /
                                      (total_bytes > 0 ? total_bytes : 1.0)) + 1;
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

template <int T, int B, bool AL, bool XL>
static hipError_t launch_group_x(const MvGroup& g, long long wgs, size_t lds, hipStream_t stream, LaunchEvents ev) {
    if (ev.start || ev.stop)
        hipExtLaunchKernelGGL((mv_kernel<T, B, AL, XL>), dim3((unsigned)wgs), dim3(256), (uint32_t)lds, stream,
                              ev.start, ev.stop, 0, g);
    else
        hipLaunchKernelGGL((mv_kernel<T, B, AL, XL>), dim3((unsigned)wgs), dim3(256), lds, stream, g);
    return hipGetLastError();
}

template <int T, int B, bool AL>
static hipError_t launch_group(MvGroup g, size_t lds, hipStream_t stream, LaunchEvents ev) {
    const long long wgs = plan_group<T, B>(g);
    if (wgs <= 0 || wgs > 0x7FFFFFFF) return hipErrorInvalidValue;
    if constexpr (Geo<T>::bs > 1 && B <= 2) {
        // stage the activations in LDS when they fit next to the column sums
        constexpr int PADI = Unit<T>::PADI;
        int max_cols = 0;
        for (int i = 0; i < g.n; ++i) max_cols = g.d[i].cols > max_cols ? g.d[i].cols : max_cols;
        const size_t xl = (size_t)B * (max_cols + (max_cols / PADI) * 4) * sizeof(float);
        const size_t lds_x = ((lds / sizeof(float) + 3) & ~size_t(3)) * sizeof(float) + xl;
        if (lds_x <= 65536) return launch_group_x<T, B, AL, true>(g, wgs, lds_x, stream, ev);
    }
    return launch_group_x<T, B, AL, false>(g, wgs, lds, stream, ev);
}

template <int T, bool AL>
static hipError_t launch_type(int batch, const MvGroup& g, size_t lds, hipStream_t s, LaunchEvents ev) {
    switch (batch) {
    case 1: return launch_group<T, 1, AL>(g, lds, s, ev);
    case 2: return launch_group<T, 2, AL>(g, lds, s, ev);
    case 4: return launch_group<T, 4, AL>(g, lds, s, ev);
    case 8: return launch_group<T, 8, AL>(g, lds, s, ev);
    default: return hipErrorInvalidValue;
    }
}

int matvec_group_launch(int type, const MatvecArgs* mats, size_t n, size_t batch, hipStream_t stream,
                        hipEvent_t start, hipEvent_t stop) {
    const TypeGeo g = type_geo(type);
    if (!g.valid) return -1;
    if (n == 0 || batch == 0) return -2;
    const bool quant = g.bs > 1;
    bool al = (g.bpb % 4 == 0);
    size_t max_cols = 0;
    for (size_t i = 0; i < n; ++i) {
        const MatvecArgs& m = mats[i];
        if (m.rows == 0 || m.cols == 0 || m.cols % g.bs != 0) return -2;
        if (m.rows > 0x7FFFFFFF || m.cols > 0x7FFFFFFF) return -2;
        const size_t row_bytes = m.cols / g.bs * g.bpb;
        if (m.w_len != m.rows * row_bytes) return -3;
        if (!m.w || !m.x || !m.y || m.ldx < m.cols || m.ldy < m.rows) return -3;
        if (quant && ((reinterpret_cast<uintptr_t>(m.x) & 15u) || (m.ldx & 3u))) return -3;
        if (!quant && (reinterpret_cast<uintptr_t>(m.w) % g.bpb)) return -3;
        if (reinterpret_cast<uintptr_t>(m.w) & 3u) al = false;
        if (m.cols > max_cols) max_cols = m.cols;
    }
    static const int forced = [] {
        const char* v = getenv("PYRITE_MATVEC_PATH");  // "valu" forces the VALU kernels
        return (v && v[0] == 'v') ? 1 : 0;
    }();
    if (quant && !forced && batch >= 3 && mx_type_supported(type)) {
        for (size_t done = 0; done < batch; done += 8) {
            const size_t c = batch - done < 8 ? batch - done : 8;
            const int rc = mx_group_launch(type, mats, n, c, done, al, stream, done == 0 ? start : nullptr,
                                           done + c >= batch ? stop : nullptr);
            if (rc != 0) return rc;
        }
        return 0;
    }
    size_t done = 0;
    while (done < batch) {
        // largest instantiated batch chunk whose per-16-column x sums fit 64 KiB of LDS
        int c = 0;
        for (int cand : {8, 4, 2, 1}) {
            if ((size_t)cand > batch - done) continue;
            if (!quant || (size_t)cand * (max_cols / 16) * sizeof(float) <= 65536) { c = cand; break; }
        }
        if (c == 0) return -2;
        const size_t lds = quant ? (size_t)c * (max_cols / 16) * sizeof(float) : 0;
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
            }
            hipError_t e = hipSuccess;
#define PYRITE_CASE(T)                                                                       \
    case T:                                                                                \
        e = al ? launch_type<T, (Geo<T>::bpb % 4 == 0)>(c, grp, lds, stream, ev)           \
               : launch_type<T, false>(c, grp, lds, stream, ev);                           \
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

int matvec_launch(int type, const uint8_t* W, size_t w_len, size_t rows, size_t cols, const float* X, size_t ldx,
                  float* Y, size_t ldy, size_t batch, hipStream_t stream) {
    MatvecArgs m{W, w_len, rows, cols, X, ldx, Y, ldy};
    return matvec_group_launch(type, &m, 1, batch, stream, nullptr, nullptr);
}

}  // namespace pyrite
