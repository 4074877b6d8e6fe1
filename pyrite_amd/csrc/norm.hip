// RMSNorm on the device: y = x * (1 / sqrt(sum(x^2) / n + eps)) * w
// (pyrite/tensor_ops.py:502-506, pyrite/executor.py:621-624), one workgroup per
// vector.  The sum of squares, the scale and both products are computed in
// fp64 as the reference does (its sum is sequential; this one is a tree, so
// the scale can differ from the reference's in the last fp64 bit), and each
// output is rounded once to fp32.
#include "dispatch.h"

namespace pyrite {

__global__ __launch_bounds__(256) void rms_norm_kernel(const float* __restrict__ X, unsigned long long ldx,
                                                       const float* __restrict__ Wt, int n, double eps,
                                                       float* __restrict__ Y, unsigned long long ldy) {
    const float* x = X + (unsigned long long)blockIdx.x * ldx;
    float* y = Y + (unsigned long long)blockIdx.x * ldy;
    double ss = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) {
        const double v = x[i];
        ss = fma(v, v, ss);
    }
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    __shared__ double part[4];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (part[0] + part[1]) + (part[2] + part[3]);
    const double inv = 1.0 / sqrt(ss / (double)(n > 0 ? n : 1) + eps);
    for (int i = threadIdx.x; i < n; i += 256) {
        const double v = (double)x[i] * inv;
        y[i] = (float)(Wt ? v * (double)Wt[i] : v);
    }
}

int rms_norm_launch(const float* X, size_t ldx, const float* Wt, size_t n, double eps, float* Y, size_t ldy,
                    size_t batch, hipStream_t stream) {
    if (n == 0 || batch == 0 || n > 0x7FFFFFFF || batch > 0x7FFFFFFF) return -2;
    if (!X || !Y || ldx < n || ldy < n) return -3;
    hipLaunchKernelGGL(rms_norm_kernel, dim3((unsigned)batch), dim3(256), 0, stream, X,
                       (unsigned long long)ldx, Wt, (int)n, eps, Y, (unsigned long long)ldy);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace pyrite
