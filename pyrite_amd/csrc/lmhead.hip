// Vocabulary LM head: fp32 logits plus the exact greedy token.
//
// The reference computes every logit in fp64 (pyrite_matvec,
// pyrite/kernels/native.c:541-553, called per 128-row chunk by
// pyrite/executor.py:852-875) and takes the first index of the maximum
// (Sampler.greedy, pyrite/sampler.py:12-15).  Here:
//
// 1. The bound variant of the VALU matvec (mv_kernel<..., BD = true>) writes
//    fp32 logits y_r and, per row, S_r >= the sum of the magnitudes of all
//    products it formed.  |y_r - exact_r| <= g32 * S_r and
//    |ref_r - exact_r| <= g64 * S_r, where exact_r is the real-number dot
//    product and ref_r the reference's fp64 logit, so
//    ref_r lies in [y_r - B_r, y_r + B_r] with B_r = (g32 + g64) * S_r (plus
//    a small absolute term for underflow).
// 2. lm_argmax_kernel: L = max_r (y_r - B_r) is a lower bound of the largest
//    reference logit, so only rows with y_r + B_r >= L can hold it.  When one
//    row qualifies it is the answer.  Otherwise every qualifying row is
//    recomputed exactly as the reference does (exact fp64 weights, one product
//    per column, fp64 adds in column order) and the largest value wins, ties
//    to the lowest index.  All-zero activations give row 0 directly.
//    Logits or bounds that are not finite switch the token to a full
//    recomputation followed by Python's max() scan (first element kept unless
//    a later one compares greater).
//
// The argmax kernel runs NWG workgroups per token; each reduces a row range
// and lists its local candidates, and the last to finish (arrival counter,
// reset by that workgroup) decides.
#include <mutex>

#include "dequant.h"
#include "mv_kernel.h"

namespace pyrite {

constexpr int kLmWgs = 256;   // argmax workgroups per token
constexpr int kLmCand = 32;   // candidates kept per workgroup before it reports overflow
constexpr int kLmKept = 512;  // candidates the deciding workgroup refines from LDS

struct LmArgs {
    int type;
    int bs, bpb;
    const uint8_t* W;
    unsigned long long row_bytes;
    int rows, cols;
    const float* X;
    unsigned long long ldx;
    const float* Y;
    const float* Bnd;
    unsigned long long ldy;
    double gamma;  // B_r = gamma * S_r + abs_margin
    double abs_margin;
    int* ids;
    // workspace
    double* ws_L;            // [batch][kLmWgs]
    int* ws_cnt;             // [batch][kLmWgs]  (-1: non-finite seen)
    int* ws_cand;            // [batch][kLmWgs][kLmCand]
    double* ws_candv;        // [batch][kLmWgs][kLmCand]: y + B of each listed row
    unsigned int* ws_arrive; // [batch]
};

__device__ __forceinline__ double readlane_f64(double v, int k) {
    const unsigned long long u = (unsigned long long)__double_as_longlong(v);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)u, k);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(u >> 32), k);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// The reference's fp64 logit of one row, in its order: exact fp64 weight times
// the fp64-widened activation, added to the running sum column by column
// (pyrite/kernels/native.c:527-553).  The whole wave computes it; every lane
// returns the same value.
__device__ double ref_row(const LmArgs& a, int row, const float* x) {
    const int lane = threadIdx.x & 63;
    const uint8_t* rp = a.W + (unsigned long long)row * a.row_bytes;
    double s = 0.0;
    for (int base = 0; base < a.cols; base += 64) {
        const int c = base + lane;
        double p = 0.0;
        if (c < a.cols) {
            const int blk = c / a.bs;
            const double w = dq_elem<double>(a.type, rp + (unsigned long long)blk * a.bpb, c - blk * a.bs);
            p = __dmul_rn(w, (double)x[c]);
        }
        const int n = a.cols - base < 64 ? a.cols - base : 64;
        for (int k = 0; k < n; ++k) s = __dadd_rn(s, readlane_f64(p, k));
    }
    return s;
}

__device__ __forceinline__ bool better(double v, int r, double bv, int br) {
    return v > bv || (v == bv && r < br);
}

__device__ __forceinline__ void block_best(double& bv, int& br, double* s_bv, int* s_br) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int off = 32; off > 0; off >>= 1) {
        const double ov = __shfl_xor(bv, off, 64);
        const int orr = __shfl_xor(br, off, 64);
        if (better(ov, orr, bv, br)) { bv = ov; br = orr; }
    }
    if (lane == 0) { s_bv[wave] = bv; s_br[wave] = br; }
    __syncthreads();
    bv = s_bv[0];
    br = s_br[0];
    for (int k = 1; k < 4; ++k)
        if (better(s_bv[k], s_br[k], bv, br)) { bv = s_bv[k]; br = s_br[k]; }
}

__global__ __launch_bounds__(256) void lm_argmax_kernel(const LmArgs a) {
    const int t = blockIdx.y, w = blockIdx.x, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const float* y = a.Y + (unsigned long long)t * a.ldy;
    const float* bn = a.Bnd + (unsigned long long)t * a.ldy;
    const float* x = a.X + (unsigned long long)t * a.ldx;
    const int chunk = (a.rows + kLmWgs - 1) / kLmWgs;
    const double g = a.gamma, am = a.abs_margin;
    auto range = [&](int k, int& q0, int& q1) {
        q0 = k * chunk < a.rows ? k * chunk : a.rows;
        q1 = q0 + chunk < a.rows ? q0 + chunk : a.rows;
    };
    auto hi = [&](int r) { return (double)y[r] + (g * (double)bn[r] + am); };
    auto lo = [&](int r) { return (double)y[r] - (g * (double)bn[r] + am); };

    __shared__ double s_red[4];
    __shared__ int s_flag[4];
    __shared__ int s_cnt, s_nref, s_one, s_last;  // s_cnt: local candidate count (pass 2)
    __shared__ int s_kept[kLmKept];
    __shared__ double s_bv[4];
    __shared__ int s_br[4];

    int r0, r1;
    range(w, r0, r1);
    // pass 1: local lower bound L_w = max (y - B); any non-finite value flags the token
    double lmax = -INFINITY;
    int nf = 0;
    for (int r = r0 + tid; r < r1; r += 256) {
        const double l = lo(r);
        if (!isfinite(y[r]) || !isfinite(l)) nf = 1;
        lmax = fmax(lmax, l);
    }
    for (int off = 32; off > 0; off >>= 1) {
        lmax = fmax(lmax, __shfl_xor(lmax, off, 64));
        nf |= __shfl_xor(nf, off, 64);
    }
    if (lane == 0) { s_red[wave] = lmax; s_flag[wave] = nf; }
    if (tid == 0) s_cnt = 0;
    __syncthreads();
    lmax = fmax(fmax(s_red[0], s_red[1]), fmax(s_red[2], s_red[3]));
    nf = s_flag[0] | s_flag[1] | s_flag[2] | s_flag[3];

    // pass 2: rows that can still beat L_w (a superset of the token's candidates in this range)
    int* cand = a.ws_cand + ((unsigned long long)t * kLmWgs + w) * kLmCand;
    double* candv = a.ws_candv + ((unsigned long long)t * kLmWgs + w) * kLmCand;
    if (!nf) {
        const double lc = lmax - fabs(lmax) * 0x1p-50;
        for (int r = r0 + tid; r < r1; r += 256) {
            const double h = hi(r);
            if (h >= lc) {
                const int k = atomicAdd(&s_cnt, 1);
                if (k < kLmCand) { st_dev(cand + k, r); st_dev(candv + k, h); }
            }
        }
    }
    __syncthreads();
    if (tid == 0) {
        st_dev(a.ws_L + (unsigned long long)t * kLmWgs + w, lmax);
        st_dev(a.ws_cnt + (unsigned long long)t * kLmWgs + w, nf ? -1 : s_cnt);
    }
    drain_dev();  // every wave's candidate stores have completed ...
    __syncthreads();
    if (tid == 0) s_last = (arrive_dev(a.ws_arrive + t) == kLmWgs - 1);  // ... before the arrival
    __syncthreads();
    __syncthreads();
    if (!s_last) return;

    // ---- deciding workgroup of token t; thread k looks after workgroup k's range
    static_assert(kLmWgs == 256, "one thread per argmax workgroup");
    const int my_cnt = ld_dev(a.ws_cnt + (unsigned long long)t * kLmWgs + tid);
    double L = ld_dev(a.ws_L + (unsigned long long)t * kLmWgs + tid);
    int any_nf = my_cnt < 0;
    for (int off = 32; off > 0; off >>= 1) {
        L = fmax(L, __shfl_xor(L, off, 64));
        any_nf |= __shfl_xor(any_nf, off, 64);
    }
    if (lane == 0) { s_red[wave] = L; s_flag[wave] = any_nf; }
    __syncthreads();
    L = fmax(fmax(s_red[0], s_red[1]), fmax(s_red[2], s_red[3]));
    any_nf = s_flag[0] | s_flag[1] | s_flag[2] | s_flag[3];

    if (any_nf) {
        // Full recomputation, then Python's max(): the first element is kept
        // unless a later one compares strictly greater (NaN never does).
        if (wave == 0) {
            double best = 0.0;
            int bi = 0;
            for (int r = 0; r < a.rows; ++r) {
                const double v = ref_row(a, r, x);
                if (r == 0 || v > best) { best = v; bi = r; }
            }
            if (lane == 0) a.ids[t] = bi;
        }
        __syncthreads();
        if (tid == 0) st_dev(a.ws_arrive + t, 0u);
        return;
    }

    // Candidates: y + B >= L (less a relative slack for the rounding of the
    // double sums above); each is queued for recomputation.
    const double Lc = L - fabs(L) * 0x1p-50;
    if (tid == 0) { s_cnt = 0; s_nref = 0; s_one = -1; }
    __syncthreads();
    double bv = -INFINITY;
    int br = 0x7FFFFFFF;
    auto consider = [&](int r, double h) {
        if (h < Lc) return;
        s_one = r;  // any candidate; used only when there is exactly one
        const int q = atomicAdd(&s_nref, 1);
        if (q < kLmKept) s_kept[q] = r;
    };
    if (my_cnt > 0 && my_cnt <= kLmCand) {
        const unsigned long long base = ((unsigned long long)t * kLmWgs + tid) * kLmCand;
        for (int q = 0; q < my_cnt; ++q) consider(ld_dev(a.ws_cand + base + q), ld_dev(a.ws_candv + base + q));
    } else if (my_cnt > kLmCand) {
        int q0, q1;
        range(tid, q0, q1);
        for (int r = q0; r < q1; ++r) consider(r, hi(r));
    }
    __syncthreads();
    const int nref = s_nref;
    if (nref == 1) {
        if (tid == 0) { a.ids[t] = s_one; st_dev(a.ws_arrive + t, 0u); }
        return;
    }
    // All-zero activations: every reference logit is +-0, which compare
    // equal, so the first row wins.
    int nz = 0;
    for (int c = tid; c < a.cols; c += 256) nz |= (x[c] != 0.f);
    for (int off = 32; off > 0; off >>= 1) nz |= __shfl_xor(nz, off, 64);
    if (lane == 0) s_flag[wave] = nz;
    __syncthreads();
    if (!(s_flag[0] | s_flag[1] | s_flag[2] | s_flag[3])) {
        if (tid == 0) { a.ids[t] = 0; st_dev(a.ws_arrive + t, 0u); }
        return;
    }
    for (int q = wave; q < (nref < kLmKept ? nref : kLmKept); q += 4) {
        const int r = s_kept[q];
        const double v = ref_row(a, r, x);
        if (better(v, r, bv, br)) { bv = v; br = r; }
    }
    if (nref > kLmKept) {
        // more rows to recompute than fit the list: recompute every such row, one per wave
        for (int r = wave; r < a.rows; r += 4) {
            if (hi(r) < Lc) continue;  // wave-uniform
            const double v = ref_row(a, r, x);
            if (better(v, r, bv, br)) { bv = v; br = r; }
        }
    }
    block_best(bv, br, s_bv, s_br);
    if (tid == 0) {
        a.ids[t] = br == 0x7FFFFFFF ? -1 : br;
        st_dev(a.ws_arrive + t, 0u);
    }
}

// ---------------------------------------------------------------- workspace

struct LmWorkspace {
    void* bnd = nullptr;     // float [tokens][ldl]
    size_t bnd_cap = 0;      // bytes
    void* tok = nullptr;     // per token: L, cnt, cand, candv (kLmTokBytes), then arrival counters
    size_t tok_cap = 0;      // bytes
};

// Per-token workspace bytes: L (double) and cnt (int) per argmax workgroup,
// then its candidate rows (int) and their upper bounds (double).
constexpr size_t kLmTokBytes = (size_t)kLmWgs * (8 + 4 + kLmCand * (4 + 8));

// Carve the token arrays out of one block of `tokens` tokens (arrival counters last).
static void lm_carve(void* base, size_t tokens, LmArgs& a) {
    char* p = static_cast<char*>(base);
    a.ws_L = reinterpret_cast<double*>(p);
    p += tokens * kLmWgs * sizeof(double);
    a.ws_candv = reinterpret_cast<double*>(p);
    p += tokens * kLmWgs * kLmCand * sizeof(double);
    a.ws_cnt = reinterpret_cast<int*>(p);
    p += tokens * kLmWgs * sizeof(int);
    a.ws_cand = reinterpret_cast<int*>(p);
    p += tokens * kLmWgs * kLmCand * sizeof(int);
    a.ws_arrive = reinterpret_cast<unsigned int*>(p);
}

static thread_local const char* g_lm_err = nullptr;

// Per-device workspace, grown on demand (never during stream capture; a
// replaced block stays allocated for graphs captured before the growth).
// The token block is zero-filled when allocated, and every launch leaves its
// arrival counters at zero.
static int lm_workspace(size_t bnd_floats, size_t tokens, hipStream_t stream, LmWorkspace** out) {
    static LmWorkspace ws[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return -4;
    LmWorkspace& w = ws[dev];
    const size_t bb = bnd_floats * sizeof(float), tb = tokens * (kLmTokBytes + sizeof(unsigned int));
    hipError_t e = hipSuccess;
    if (bb > w.bnd_cap) e = workspace_grow(&w.bnd, &w.bnd_cap, bb, false, stream);
    if (e == hipSuccess && tb > w.tok_cap) {
        // the arrival counters sit after the token arrays, whose extent depends
        // on the capacity in tokens: grow to a whole number of tokens
        e = workspace_grow(&w.tok, &w.tok_cap, tb, true, stream);
    }
    if (e == hipErrorStreamCaptureUnsupported) {
        g_lm_err = "LM-head workspace must grow, which is not allowed during stream capture; run once before capturing";
        return -4;
    }
    if (e != hipSuccess) return -4;
    *out = &w;
    return 0;
}

const char* lm_last_error() { return g_lm_err; }

// Rounding-error budget of the VALU bound kernels: the longest chain of
// roundings from a product to the stored logit is below
// (units per lane) * 96 + 64 (unit decode chains are at most 96 long; the
// lane reduction and the column sums add less than 64).
static double lm_gamma(const TypeGeo& g, size_t cols) {
    const double u32 = 1.0 / 16777216.0, u64 = 1.0 / 9007199254740992.0;
    double units = 0, per_unit = 0;
    if (g.bs > 1) {
        units = (double)(cols / g.bs) * (g.bs == 256 ? 4 : 1);
        per_unit = 96;
    } else {
        units = (double)((cols + 3) / 4);
        per_unit = 8;
    }
    const double lanes = units < 64 ? units : 64;
    const double depth = (units / lanes + 1) * per_unit + 64;
    const double g32 = depth * u32 / (1 - depth * u32);
    const double g64 = (double)cols * u64 / (1 - (double)cols * u64);
    return (g32 + g64) * (1 + 1.0 / 1024);
}

// Zero the arrival counters of `n` tokens (a kernel, not a memset, so that it
// can be captured into a graph).
__global__ __launch_bounds__(256) void lm_clear_kernel(unsigned int* counters, int n) {
    for (int i = threadIdx.x; i < n; i += 256) counters[i] = 0u;
}

// The bound matvec, then the argmax kernel, over workspace memory the caller
// provides: bnd (floats laid out like the logits) and a token block carved by
// lm_carve for `tok_cap` tokens.  clear: zero the arrival counters first.
static int lm_head_run(int type, const TypeGeo& g, bool al, size_t max_cols, const MatvecArgs& m, int* ids,
                       size_t batch, float* bnd, void* tok, size_t tok_cap, bool clear, hipStream_t stream) {
    LmArgs a;
    lm_carve(tok, tok_cap, a);
    if (clear) {
        hipLaunchKernelGGL(lm_clear_kernel, dim3(1), dim3(256), 0, stream, a.ws_arrive, (int)batch);
        if (hipGetLastError() != hipSuccess) return -4;
    }
    if (const int rc = valu_group_launch<true>(type, g, al, &m, &bnd, 1, batch, max_cols, stream, nullptr, nullptr))
        return rc;
    a.type = type;
    a.bs = g.bs;
    a.bpb = g.bpb;
    a.W = static_cast<const uint8_t*>(m.w);
    a.row_bytes = m.cols / g.bs * g.bpb;
    a.rows = (int)m.rows;
    a.cols = (int)m.cols;
    a.X = m.x;
    a.ldx = m.ldx;
    a.Y = m.y;
    a.Bnd = bnd;
    a.ldy = m.ldy;
    a.gamma = lm_gamma(g, m.cols);
    a.abs_margin = 1e-30;
    a.ids = ids;
    hipLaunchKernelGGL(lm_argmax_kernel, dim3(kLmWgs, (unsigned)batch), dim3(256), 0, stream, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

static int lm_validate(int type, const uint8_t* W, size_t w_len, size_t rows, size_t cols, const float* X,
                       size_t ldx, float* logits, size_t ldl, int* ids, size_t batch, TypeGeo* g, MatvecArgs* m,
                       bool* al, size_t* max_cols) {
    *g = type_geo(type);
    *m = MatvecArgs{W, w_len, rows, cols, X, ldx, logits, ldl};
    if (const int rc = validate_group(*g, m, 1, batch, al, max_cols)) return rc;
    if (!ids) return -3;
    if (cols > 65536 || batch > 65535) return -2;
    return 0;
}

int lm_head_launch(int type, const uint8_t* W, size_t w_len, size_t rows, size_t cols, const float* X, size_t ldx,
                   float* logits, size_t ldl, int* ids, size_t batch, hipStream_t stream) {
    g_lm_err = nullptr;
    TypeGeo g;
    MatvecArgs m;
    bool al = false;
    size_t max_cols = 0;
    if (const int rc = lm_validate(type, W, w_len, rows, cols, X, ldx, logits, ldl, ids, batch, &g, &m, &al,
                                   &max_cols))
        return rc;
    LmWorkspace* ws = nullptr;
    if (const int rc = lm_workspace(batch * ldl, batch, stream, &ws)) return rc;
    return lm_head_run(type, g, al, max_cols, m, ids, batch, static_cast<float*>(ws->bnd), ws->tok,
                       ws->tok_cap / (kLmTokBytes + sizeof(unsigned int)), false, stream);
}

// ---------------------------------------------------------------- allocation-free variant
// The LM head for callers that cannot allocate (code under graph capture,
// serving loops): its workspace is this file-scope device array instead of
// hipMalloc'ed memory.  Layout: the token block for kLmScratchTokens tokens
// (lm_carve), then, from the next 256-byte boundary, the bound floats.  Each
// GPU holds its own copy until the process ends; every call on a GPU shares it
// (the last call's contents stay), so calls that overlap on one GPU race.
constexpr size_t kLmScratchBytes = size_t(8) << 20;
constexpr size_t kLmScratchTokens = 8;
constexpr size_t kLmScratchBndOffset =
    (kLmScratchTokens * (kLmTokBytes + sizeof(unsigned int)) + 255) & ~size_t(255);
constexpr size_t kLmScratchBndFloats = (kLmScratchBytes - kLmScratchBndOffset) / sizeof(float);
static_assert(kLmScratchBndFloats == 1894336, "the limit quoted in the error message and the header");

static __device__ __align__(256) unsigned char scratch[kLmScratchBytes];

// The device address of `scratch` on the current device (its host-side name
// is only a stand-in), looked up once per device.
static int lm_scratch(void** out) {
    static std::mutex mu;
    static void* ptr[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return -4;
    std::lock_guard<std::mutex> lock(mu);
    if (!ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
            g_lm_err = "hipGetSymbolAddress of the LM-head scratch failed";
            return -4;
        }
        ptr[dev] = p;
    }
    *out = ptr[dev];
    return 0;
}

int lm_head_noalloc_launch(int type, const uint8_t* W, size_t w_len, size_t rows, size_t cols, const float* X,
                           size_t ldx, float* logits, size_t ldl, int* ids, size_t batch, hipStream_t stream) {
    g_lm_err = nullptr;
    TypeGeo g;
    MatvecArgs m;
    bool al = false;
    size_t max_cols = 0;
    if (const int rc = lm_validate(type, W, w_len, rows, cols, X, ldx, logits, ldl, ids, batch, &g, &m, &al,
                                   &max_cols))
        return rc;
    if (batch > kLmScratchTokens || (batch - 1) * ldl + rows > kLmScratchBndFloats) {
        g_lm_err = "pyrite_dev_lm_head_argmax_noalloc: at most 8 vectors and (batch - 1) * ldl + rows <= "
                   "1894336 (the fixed 8 MiB scratch)";
        return -2;
    }
    void* base = nullptr;
    if (const int rc = lm_scratch(&base)) return rc;
    float* bnd = reinterpret_cast<float*>(static_cast<char*>(base) + kLmScratchBndOffset);
    return lm_head_run(type, g, al, max_cols, m, ids, batch, bnd, base, kLmScratchTokens, true, stream);
}

}  // namespace pyrite
