// The operations around the matvecs of one decode layer, so that a layer runs
// on the device from its input to its output:
//
//   add_rms_norm_kernel   h' = h + delta (the residual add) and rms_norm(h'),
//                         one pass (pyrite/executor.py:795-811,
//                         pyrite/dense.py:497-513)
//   matvec_swiglu_launch  the dense FFN's down projection, W . (silu(gate) *
//                         up), with the activation formed while the VALU
//                         matvec stages its input (pyrite/dense.py:473-495)
//   attn_prep_kernel,     single-token attention over an fp32 KV cache:
//   attn_split_kernel,    QK-norm and NEOX RoPE, append K/V, scores, softmax,
//   attn_combine_kernel   weighted values (pyrite/executor.py:627-646,
//                         685-755; the cache is LayerKV, :79-141)
//
// Attention numerics: the reference keeps q in fp64 and K/V as fp32
// (array('f')), computes the scores, the softmax and the weighted sum in
// fp64.  Here QK-norm and RoPE run in fp64 and are rounded once to fp32 (the
// cached K is rounded exactly as the reference stores it); scores and the
// per-chunk softmax are fp64; each 256-token chunk's weighted values are
// summed in fp32 and the chunks are combined in fp64.
#include <math.h>

#include "dispatch.h"
#include "mv_kernel.h"

namespace pyrite {

// ---------------------------------------------------------------- residual add + RMSNorm

// One workgroup per vector: Hout = H + D (fp32), N = Hout * (1 / sqrt(sum(Hout^2) / n + eps)) * Wt
// with the sum, the scale and the products in fp64 and one rounding to fp32.
// Hout may alias H.
__global__ __launch_bounds__(256) void add_rms_norm_kernel(const float* H, unsigned long long ldh,
                                                           const float* __restrict__ D, unsigned long long ldd,
                                                           const float* __restrict__ Wt, int n, double eps,
                                                           float* Hout, unsigned long long ldo,
                                                           float* __restrict__ N, unsigned long long ldn) {
    const unsigned long long b = blockIdx.x;
    const float* h = H + b * ldh;
    const float* d = D + b * ldd;
    float* ho = Hout + b * ldo;
    float* y = N + b * ldn;
    double ss = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = h[i] + d[i];
        ho[i] = v;
        ss = fma((double)v, (double)v, ss);
    }
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    __shared__ double part[4];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (part[0] + part[1]) + (part[2] + part[3]);
    const double inv = 1.0 / sqrt(ss / (double)n + eps);
    // each thread re-reads only the values it wrote itself
    for (int i = threadIdx.x; i < n; i += 256) {
        const double v = (double)ho[i] * inv;
        y[i] = (float)(Wt ? v * (double)Wt[i] : v);
    }
}

int add_rms_norm_launch(const float* H, size_t ldh, const float* D, size_t ldd, const float* Wt, size_t n,
                        double eps, float* Hout, size_t ldo, float* N, size_t ldn, size_t batch,
                        hipStream_t stream) {
    if (n == 0 || batch == 0 || n > 0x7FFFFFFF || batch > 0x7FFFFFFF) return -2;
    if (!H || !D || !Hout || !N || ldh < n || ldd < n || ldo < n || ldn < n) return -3;
    hipLaunchKernelGGL(add_rms_norm_kernel, dim3((unsigned)batch), dim3(256), 0, stream, H,
                       (unsigned long long)ldh, D, (unsigned long long)ldd, Wt, (int)n, eps, Hout,
                       (unsigned long long)ldo, N, (unsigned long long)ldn);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// ---------------------------------------------------------------- SwiGLU down projection

int matvec_swiglu_launch(int type, const uint8_t* W, size_t w_len, size_t rows, size_t cols, const float* G,
                         const float* U, size_t ldx, float* Y, size_t ldy, size_t batch, hipStream_t stream) {
    const TypeGeo g = type_geo(type);
    MatvecArgs m{W, w_len, rows, cols, G, ldx, Y, ldy};
    bool al = false;
    size_t max_cols = 0;
    if (const int rc = validate_group(g, &m, 1, batch, &al, &max_cols)) return rc;
    if (g.bs == 1) return -1;  // plain-type weights: no staged path
    if (!U || (reinterpret_cast<uintptr_t>(U) & 15u)) return -3;
    const float* ups[1] = {U};
    return valu_group_launch<false, XSwiglu>(type, g, al, &m, nullptr, 1, batch, max_cols, stream, nullptr, nullptr,
                                             ups);
}

// ---------------------------------------------------------------- attention decode

constexpr int kAttnChunk = 256;     // tokens per split workgroup (one per lane)
constexpr int kAttnMaxDim = 256;    // head_dim and value_dim
constexpr int kAttnMaxGroup = 16;   // query heads per kv head

struct AttnArgs {
    int n_heads, n_kv, head_dim, value_dim, rotary_dim, group;
    double theta, eps, scale;
    long long position;
    const float* q_norm;
    const float* k_norm;
    float* k_cache;   // [capacity][n_kv * head_dim]
    float* v_cache;   // [capacity][n_kv * value_dim]
    int slot, n_ctx, n_chunks;
    const float* q;   // [n_heads * head_dim]
    const float* k;   // [n_kv * head_dim]
    const float* v;   // [n_kv * value_dim]
    float* qr;        // workspace: [n_heads * head_dim] normed, rotated queries
    double* part_m;   // workspace: [n_chunks][n_heads] chunk maximum of the scaled scores
    double* part_l;   // workspace: [n_chunks][n_heads] chunk sum of exp(score - max)
    float* part_o;    // workspace: [n_chunks][n_heads][value_dim] chunk weighted values
    float* out;       // [n_heads * value_dim]
};

// One workgroup per query head (blockIdx.x < n_heads) or kv head: optional
// RMSNorm over the head (fp64, as rms_norm), then NEOX RoPE of its first
// rotary_dim values: for i < rotary_dim / 2, (x_i, x_{i+half}) rotated by
// position * theta^(-2i / rotary_dim).  Queries go to qr, keys (rounded to
// fp32) and values to the cache slot.
__global__ __launch_bounds__(256) void attn_prep_kernel(const AttnArgs a) {
    __shared__ double xs[kAttnMaxDim];
    __shared__ double part[4];
    const int hb = blockIdx.x;
    const bool is_q = hb < a.n_heads;
    const int head = is_q ? hb : hb - a.n_heads;
    const int hd = a.head_dim;
    const float* src = is_q ? a.q + (long long)head * hd : a.k + (long long)head * hd;
    const float* nw = is_q ? a.q_norm : a.k_norm;
    const int tid = threadIdx.x;
    double x = tid < hd ? (double)src[tid] : 0.0;
    if (nw) {
        double ss = x * x;
        for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
        if ((tid & 63) == 0) part[tid >> 6] = ss;
        __syncthreads();
        ss = (part[0] + part[1]) + (part[2] + part[3]);
        const double inv = 1.0 / sqrt(ss / (double)hd + a.eps);
        if (tid < hd) x = x * inv * (double)nw[tid];
    }
    if (tid < hd) xs[tid] = x;
    __syncthreads();
    const int half = a.rotary_dim / 2;
    if (tid < hd) {
        double y = x;
        if (tid < 2 * half) {
            const int i = tid < half ? tid : tid - half;
            const double freq = pow(a.theta, -2.0 * (double)i / (double)a.rotary_dim);
            const double angle = (double)a.position * freq;
            const double c = cos(angle), s = sin(angle);
            const double x0 = xs[i], x1 = xs[i + half];
            y = tid < half ? x0 * c - x1 * s : x0 * s + x1 * c;
        }
        if (is_q) {
            a.qr[(long long)head * hd + tid] = (float)y;
        } else {
            a.k_cache[(long long)a.slot * a.n_kv * hd + (long long)head * hd + tid] = (float)y;
        }
    }
    if (!is_q)
        for (int j = tid; j < a.value_dim; j += 256)
            a.v_cache[(long long)a.slot * a.n_kv * a.value_dim + (long long)head * a.value_dim + j] =
                a.v[(long long)head * a.value_dim + j];
}

// Workgroup (chunk c, kv head g): tokens [c * 256, min(n_ctx, (c + 1) * 256)),
// one per thread, against the group's query heads.  Scores in fp64
// (scale / sqrt(head_dim) applied as the reference does, after the dot
// product), the chunk's maximum and sum of exp(score - max) per head, then
// each output value of a head summed over the chunk's tokens in fp32.
__global__ __launch_bounds__(256) void attn_split_kernel(const AttnArgs a) {
    __shared__ float qs[kAttnMaxGroup * kAttnMaxDim];
    __shared__ float ps[kAttnMaxGroup][kAttnChunk];
    __shared__ double red[kAttnMaxGroup][4];
    const int c = blockIdx.x, g = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = a.group, hd = a.head_dim, vd = a.value_dim;
    const int h0 = g * G;
    for (int i = tid; i < G * hd; i += 256) qs[i] = a.qr[(long long)h0 * hd + i];
    __syncthreads();
    const int t0 = c * kAttnChunk;
    const int t = t0 + tid;
    const bool live = t < a.n_ctx;
    double s[kAttnMaxGroup];
#pragma unroll
    for (int h = 0; h < kAttnMaxGroup; ++h) s[h] = 0.0;
    if (live) {
        const float* kr = a.k_cache + (long long)t * a.n_kv * hd + (long long)g * hd;
        for (int d = 0; d < hd; d += 2) {
            const float2 k2 = *reinterpret_cast<const float2*>(kr + d);
#pragma unroll
            for (int h = 0; h < kAttnMaxGroup; ++h)
                if (h < G) {
                    s[h] = fma((double)qs[h * hd + d], (double)k2.x, s[h]);
                    s[h] = fma((double)qs[h * hd + d + 1], (double)k2.y, s[h]);
                }
        }
    }
    // chunk maximum and exp-sum per head
    double mloc[kAttnMaxGroup];
#pragma unroll
    for (int h = 0; h < kAttnMaxGroup; ++h) {
        if (h >= G) break;
        double v = live ? s[h] * a.scale : -INFINITY;
        s[h] = v;
        for (int off = 32; off > 0; off >>= 1) v = fmax(v, __shfl_xor(v, off, 64));
        if (lane == 0) red[h][wave] = v;
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < kAttnMaxGroup; ++h) {
        if (h >= G) break;
        mloc[h] = fmax(fmax(red[h][0], red[h][1]), fmax(red[h][2], red[h][3]));
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < kAttnMaxGroup; ++h) {
        if (h >= G) break;
        const double p = live ? exp(s[h] - mloc[h]) : 0.0;
        ps[h][tid] = (float)p;
        double v = p;
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        if (lane == 0) red[h][wave] = v;
    }
    __syncthreads();
    if (tid < G) {
        const long long o = (long long)c * a.n_heads + h0 + tid;
        a.part_m[o] = mloc[tid];
        a.part_l[o] = (red[tid][0] + red[tid][1]) + (red[tid][2] + red[tid][3]);
    }
    // weighted values: thread -> (head, value index) pairs, tokens of the chunk in order
    const int nt = a.n_ctx - t0 < kAttnChunk ? a.n_ctx - t0 : kAttnChunk;
    const float* vbase = a.v_cache + (long long)t0 * a.n_kv * vd + (long long)g * vd;
    for (int i = tid; i < G * vd; i += 256) {
        const int h = i / vd, j = i - h * vd;
        float acc = 0.f;
        for (int tt = 0; tt < nt; ++tt) acc = fmaf(ps[h][tt], vbase[(long long)tt * a.n_kv * vd + j], acc);
        a.part_o[((long long)c * a.n_heads + h0 + h) * vd + j] = acc;
    }
}

// One workgroup per query head: combine the chunks, out = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c.
__global__ __launch_bounds__(256) void attn_combine_kernel(const AttnArgs a) {
    const int h = blockIdx.x;
    double M = -INFINITY;
    for (int c = 0; c < a.n_chunks; ++c) M = fmax(M, a.part_m[(long long)c * a.n_heads + h]);
    double L = 0.0;
    for (int c = 0; c < a.n_chunks; ++c) {
        const long long o = (long long)c * a.n_heads + h;
        L += exp(a.part_m[o] - M) * a.part_l[o];
    }
    for (int j = threadIdx.x; j < a.value_dim; j += 256) {
        double acc = 0.0;
        for (int c = 0; c < a.n_chunks; ++c) {
            const long long o = (long long)c * a.n_heads + h;
            acc += exp(a.part_m[o] - M) * (double)a.part_o[o * a.value_dim + j];
        }
        a.out[(long long)h * a.value_dim + j] = (float)(acc / L);
    }
}

struct AttnWorkspace {
    void* base = nullptr;
    size_t cap = 0;
};

static thread_local const char* g_attn_err = nullptr;
const char* attn_last_error() { return g_attn_err; }

int attention_decode_launch(const AttnLayer& L, const float* q, const float* k, const float* v, size_t position,
                            size_t slot, size_t n_ctx, float* out, hipStream_t stream) {
    g_attn_err = nullptr;
    if (!q || !k || !v || !out || !L.k_cache || !L.v_cache) return -3;
    if (L.n_heads == 0 || L.n_kv_heads == 0 || L.n_heads % L.n_kv_heads != 0 ||
        L.n_heads / L.n_kv_heads > (size_t)kAttnMaxGroup || L.head_dim == 0 || L.head_dim > (size_t)kAttnMaxDim ||
        (L.head_dim & 1) || L.value_dim == 0 || L.value_dim > (size_t)kAttnMaxDim || L.rotary_dim > L.head_dim ||
        (L.rotary_dim & 1) || L.capacity == 0 || L.capacity > 0x7FFFFFF || n_ctx == 0 || n_ctx > L.capacity ||
        slot >= n_ctx || L.n_heads > 0xFFFF || position > 0x7FFFFFFFFFFFull || !(L.rope_theta > 0.0)) {
        g_attn_err = "attention: unsupported shape (n_heads a multiple of n_kv_heads, at most 16 query heads per "
                     "kv head, head_dim even and <= 256, value_dim <= 256, rotary_dim even and <= head_dim, "
                     "0 < n_ctx <= capacity, slot < n_ctx)";
        return -2;
    }
    if ((reinterpret_cast<uintptr_t>(L.k_cache) & 7u)) return -3;  // float2 key loads
    AttnArgs a;
    a.n_heads = (int)L.n_heads;
    a.n_kv = (int)L.n_kv_heads;
    a.head_dim = (int)L.head_dim;
    a.value_dim = (int)L.value_dim;
    a.rotary_dim = (int)L.rotary_dim;
    a.group = a.n_heads / a.n_kv;
    a.theta = L.rope_theta;
    a.eps = L.eps;
    a.scale = 1.0 / sqrt((double)L.head_dim);
    a.position = (long long)position;
    a.q_norm = L.q_norm;
    a.k_norm = L.k_norm;
    a.k_cache = L.k_cache;
    a.v_cache = L.v_cache;
    a.slot = (int)slot;
    a.n_ctx = (int)n_ctx;
    a.n_chunks = (int)((n_ctx + kAttnChunk - 1) / kAttnChunk);
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    // workspace: qr, then part_m, part_l (doubles), then part_o
    const size_t nq = L.n_heads * L.head_dim, np = (size_t)a.n_chunks * L.n_heads;
    const size_t off_m = (nq * sizeof(float) + 255) & ~size_t(255);
    const size_t off_l = off_m + ((np * sizeof(double) + 255) & ~size_t(255));
    const size_t off_o = off_l + ((np * sizeof(double) + 255) & ~size_t(255));
    const size_t bytes = off_o + np * L.value_dim * sizeof(float);
    static AttnWorkspace ws[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return -4;
    if (ws[dev].cap < bytes) {
        const hipError_t e = workspace_grow(&ws[dev].base, &ws[dev].cap, bytes, false, stream);
        if (e == hipErrorStreamCaptureUnsupported) {
            g_attn_err = "attention workspace must grow, which is not allowed during stream capture; run once "
                         "before capturing";
            return -4;
        }
        if (e != hipSuccess) return -4;
    }
    char* base = static_cast<char*>(ws[dev].base);
    a.qr = reinterpret_cast<float*>(base);
    a.part_m = reinterpret_cast<double*>(base + off_m);
    a.part_l = reinterpret_cast<double*>(base + off_l);
    a.part_o = reinterpret_cast<float*>(base + off_o);
    hipLaunchKernelGGL(attn_prep_kernel, dim3((unsigned)(L.n_heads + L.n_kv_heads)), dim3(256), 0, stream, a);
    hipLaunchKernelGGL(attn_split_kernel, dim3((unsigned)a.n_chunks, (unsigned)L.n_kv_heads), dim3(256), 0, stream,
                       a);
    hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)L.n_heads), dim3(256), 0, stream, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace pyrite
