// Exact dequantization kernels: one output element per thread, fp32 or fp64.
// fp64 output is bit-identical to pyrite_dequantize_rows
// (pyrite/kernels/native.c:557-576); fp32 output equals (float) of it.
#include "dequant.h"
#include "dispatch.h"

namespace pyrite {

template <typename T>
__global__ __launch_bounds__(256) void dq_kernel(int type, const uint8_t* __restrict__ W,
                                                 unsigned long long row_bytes, unsigned long long rows,
                                                 unsigned long long cols, int bs, int bpb, T* __restrict__ out) {
    const unsigned long long total = rows * cols;
    const unsigned long long stride = (unsigned long long)gridDim.x * blockDim.x;
    for (unsigned long long i = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const unsigned long long r = i / cols, c = i - r * cols;
        const unsigned long long blk = c / (unsigned)bs;
        const int e = (int)(c - blk * (unsigned)bs);
        out[i] = dq_elem<T>(type, W + r * row_bytes + blk * (unsigned)bpb, e);
    }
}

// fp64 matvec for the host drop-in (pyrite_matvec takes and returns doubles):
// every weight is the exact reference double (dq_elem<double>), products and
// sums are fp64, one wave per row, lanes stride over the columns and reduce
// with shuffles.  Matches the reference to fp64 rounding (order differs).
__global__ __launch_bounds__(256) void mv64_kernel(int type, const uint8_t* __restrict__ W,
                                                   unsigned long long row_bytes, unsigned long long rows,
                                                   unsigned long long cols, int bs, int bpb,
                                                   const double* __restrict__ X, double* __restrict__ Y) {
    const int lane = threadIdx.x & 63;
    const unsigned long long row = (unsigned long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const uint8_t* rp = W + row * row_bytes;
    double acc = 0.0;
    for (unsigned long long c = lane; c < cols; c += 64) {
        const unsigned long long blk = c / (unsigned)bs;
        const double v = dq_elem<double>(type, rp + blk * (unsigned)bpb, (int)(c - blk * (unsigned)bs));
        acc = fma(v, X[c], acc);
    }
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (lane == 0) Y[row] = acc;
}

int matvec64_launch(int type, const uint8_t* W, size_t w_len, size_t rows, size_t cols, const double* X,
                    double* Y, hipStream_t stream) {
    const TypeGeo g = type_geo(type);
    if (!g.valid) return -1;
    if (rows == 0 || cols == 0 || cols % g.bs != 0) return -2;
    const size_t row_bytes = cols / g.bs * g.bpb;
    if (w_len != rows * row_bytes || !W || !X || !Y) return -3;
    const unsigned long long blocks = (rows + 3) / 4;
    if (blocks > 0x7FFFFFFFULL) return -2;
    hipLaunchKernelGGL(mv64_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, type, W,
                       (unsigned long long)row_bytes, (unsigned long long)rows, (unsigned long long)cols, g.bs,
                       g.bpb, X, Y);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int dequant_launch(int type, const uint8_t* W, size_t w_len, size_t rows, size_t cols, void* out, int out_f64,
                   hipStream_t stream) {
    const TypeGeo g = type_geo(type);
    if (!g.valid) return -1;
    if (rows == 0 || cols == 0 || cols % g.bs != 0) return -2;
    const size_t row_bytes = cols / g.bs * g.bpb;
    if (row_bytes > SIZE_MAX / rows) return -2;
    if (w_len != rows * row_bytes || cols > SIZE_MAX / rows) return -3;
    if (!W || !out) return -3;
    const unsigned long long total = (unsigned long long)rows * cols;
    unsigned long long blocks = (total + 255) / 256;
    if (blocks > 65536ULL * 8) blocks = 65536ULL * 8;
    if (out_f64)
        hipLaunchKernelGGL(dq_kernel<double>, dim3((unsigned)blocks), dim3(256), 0, stream, type, W,
                           (unsigned long long)row_bytes, (unsigned long long)rows, (unsigned long long)cols, g.bs,
                           g.bpb, static_cast<double*>(out));
    else
        hipLaunchKernelGGL(dq_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, stream, type, W,
                           (unsigned long long)row_bytes, (unsigned long long)rows, (unsigned long long)cols, g.bs,
                           g.bpb, static_cast<float*>(out));
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace pyrite
