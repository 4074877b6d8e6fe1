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
#include "common.h"
#include "dispatch.h"
#include "mv_units.h"

namespace pyrite {

template <int T, int B, bool AL>
__global__ __launch_bounds__(256) void mv_kernel(const uint8_t* __restrict__ W, unsigned long long row_bytes,
                                                 int rows, int cols, const float* __restrict__ X,
                                                 unsigned long long ldx, float* __restrict__ Y,
                                                 unsigned long long ldy, int lpr_log2) {
    constexpr int R = (B <= 2) ? 2 : 1;
    constexpr int BS = Geo<T>::bs, BPB = Geo<T>::bpb;
    extern __shared__ float xs16[];
    const int n16 = cols >> 4;
    if constexpr (BS > 1) {
        for (int i = threadIdx.x; i < B * n16; i += blockDim.x) {
            const int b = i / n16, j = i - b * n16;
            const float* p = X + b * ldx + 16 * j;
            const float4 a = ld_x4(p), c = ld_x4(p + 4), e = ld_x4(p + 8), f = ld_x4(p + 12);
            xs16[i] = (((a.x + a.y) + (a.z + a.w)) + ((c.x + c.y) + (c.z + c.w))) +
                      (((e.x + e.y) + (e.z + e.w)) + ((f.x + f.y) + (f.z + f.w)));
        }
        __syncthreads();
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int LPR = 1 << lpr_log2, nslot = 64 >> lpr_log2;
    const int slot = lane >> lpr_log2, li = lane & (LPR - 1);
    const long long wave_row0 = ((long long)blockIdx.x * 4 + wave) * nslot * R;
    if (wave_row0 >= rows) return;
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
        rp[r] = W + rr * row_bytes;
    }

    if constexpr (BS > 1) {
        constexpr int P = Unit<T>::P;
        const int U = (cols / BS) * P;
        XView xv;
        xv.ldx = ldx;
        xv.ld16 = n16;
        for (int u = li; u < U; u += LPR) {
            const int blk = u / P, part = u - blk * P;
            const uint8_t* bp[R];
#pragma unroll
            for (int r = 0; r < R; ++r) bp[r] = rp[r] + (size_t)blk * BPB;
            xv.x = X + (size_t)blk * BS;
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
                for (int b = 0; b < B; ++b) Y[b * ldy + row0 + r] = acc[r][b];
    }
}

// ---------------------------------------------------------------- launcher

static int pow2_log2_ceil(long long v) {
    int l = 0;
    while ((1LL << l) < v) ++l;
    return l;
}

template <int T, int B, bool AL>
static hipError_t launch_one(const uint8_t* W, size_t row_bytes, int rows, int cols, const float* X, size_t ldx,
                             float* Y, size_t ldy, hipStream_t stream) {
    constexpr int BS = Geo<T>::bs;
    long long U;
    if constexpr (BS > 1) U = (long long)(cols / BS) * Unit<T>::P;
    else U = (cols + 3) / 4;
    const int lpr_log2 = pow2_log2_ceil(U < 64 ? U : 64);
    const int nslot = 64 >> lpr_log2;
    const int R = (B <= 2) ? 2 : 1;
    const long long rows_per_wg = 4LL * nslot * R;
    const long long grid = (rows + rows_per_wg - 1) / rows_per_wg;
    const size_t lds = (BS > 1) ? (size_t)B * (cols / 16) * sizeof(float) : 0;
    hipLaunchKernelGGL((mv_kernel<T, B, AL>), dim3((unsigned)grid), dim3(256), lds, stream, W,
                       (unsigned long long)row_bytes, rows, cols, X, (unsigned long long)ldx, Y,
                       (unsigned long long)ldy, lpr_log2);
    return hipGetLastError();
}

template <int T, bool AL>
static hipError_t launch_type(int batch, const uint8_t* W, size_t row_bytes, int rows, int cols, const float* X,
                              size_t ldx, float* Y, size_t ldy, hipStream_t s) {
    switch (batch) {
    case 1: return launch_one<T, 1, AL>(W, row_bytes, rows, cols, X, ldx, Y, ldy, s);
    case 2: return launch_one<T, 2, AL>(W, row_bytes, rows, cols, X, ldx, Y, ldy, s);
    case 4: return launch_one<T, 4, AL>(W, row_bytes, rows, cols, X, ldx, Y, ldy, s);
    case 8: return launch_one<T, 8, AL>(W, row_bytes, rows, cols, X, ldx, Y, ldy, s);
    default: return hipErrorInvalidValue;
    }
}

// Largest batch chunk the kernels are instantiated for that fits `left` and the
// LDS budget for the per-16-column sums (64 KiB).
static int pick_chunk(int left, int cols, bool quant) {
    const int cand[4] = {8, 4, 2, 1};
    for (int c : cand) {
        if (c > left) continue;
        if (!quant || (size_t)c * (cols / 16) * sizeof(float) <= 65536) return c;
    }
    return 0;
}

int matvec_launch(int type, const uint8_t* W, size_t w_len, size_t rows, size_t cols, const float* X, size_t ldx,
                  float* Y, size_t ldy, size_t batch, hipStream_t stream) {
    const TypeGeo g = type_geo(type);
    if (!g.valid) return -1;
    if (rows == 0 || cols == 0 || batch == 0 || cols % g.bs != 0) return -2;
    if (rows > 0x7FFFFFFF || cols > 0x7FFFFFFF) return -2;
    const size_t row_bytes = cols / g.bs * g.bpb;
    if (w_len != rows * row_bytes) return -3;
    if (!W || !X || !Y || ldx < cols || ldy < rows) return -3;
    const bool quant = g.bs > 1;
    if (quant && ((reinterpret_cast<uintptr_t>(X) & 15u) || (ldx & 3u))) return -3;
    if (!quant && (reinterpret_cast<uintptr_t>(W) % g.bpb)) return -3;
    const bool al = (g.bpb % 4 == 0) && ((reinterpret_cast<uintptr_t>(W) & 3u) == 0);
    size_t done = 0;
    while (done < batch) {
        const int c = pick_chunk((int)(batch - done > 8 ? 8 : batch - done), (int)cols, quant);
        if (c == 0) return -2;
        hipError_t e = hipSuccess;
        const float* Xc = X + done * ldx;
        float* Yc = Y + done * ldy;
#define PYRITE_CASE(T)                                                                                  \
    case T:                                                                                           \
        e = (al && Geo<T>::bpb % 4 == 0)                                                              \
                ? launch_type<T, (Geo<T>::bpb % 4 == 0)>(c, W, row_bytes, (int)rows, (int)cols, Xc, ldx, Yc, ldy, stream) \
                : launch_type<T, false>(c, W, row_bytes, (int)rows, (int)cols, Xc, ldx, Yc, ldy, stream);  \
        break;
        switch (type) {
            PYRITE_FOR_EACH_TYPE(PYRITE_CASE)
        default: return -1;
        }
#undef PYRITE_CASE
        if (e != hipSuccess) return -4;
        done += c;
    }
    return 0;
}

}  // namespace pyrite
