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
constexpr int kLmCand = 31;   // candidates kept per workgroup before it reports overflow
constexpr int kLmKept = 512;  // candidates the deciding workgroup refines from LDS
constexpr int kLmFan = 40;    // sub-counters of a token's arrival tree (arrive_tree)
constexpr int kLmArr = 1 + kLmFan;  // arrival counters per token: the root, then the sub-counters

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
    unsigned int* ws_arrive; // [batch][kLmArr]: root, sub-counters
    unsigned int* ws_rec;    // fused batch-1 head: kLmRecDw dwords per workgroup (aliases the arrays above)
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

// LDS of a deciding workgroup.
struct LmDecLds {
    double red[4];
    int flag[4];
    int cnt, nref, one;  // candidate count, rows queued for recomputation, any candidate
    int kept[kLmKept];
    double bv[4];
    int br[4];
};

__device__ __forceinline__ void block_best(double& bv, int& br, LmDecLds& sd) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int off = 32; off > 0; off >>= 1) {
        const double ov = __shfl_xor(bv, off, 64);
        const int orr = __shfl_xor(br, off, 64);
        if (better(ov, orr, bv, br)) { bv = ov; br = orr; }
    }
    if (lane == 0) { sd.bv[wave] = bv; sd.br[wave] = br; }
    __syncthreads();
    bv = sd.bv[0];
    br = sd.br[0];
    for (int k = 1; k < 4; ++k)
        if (better(sd.bv[k], sd.br[k], bv, br)) { bv = sd.bv[k]; br = sd.br[k]; }
}

// Block-wide max of a double and OR of a flag word (4 waves).
__device__ __forceinline__ void block_max_or(double& v, int& f, LmDecLds& sd) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int off = 32; off > 0; off >>= 1) {
        v = fmax(v, __shfl_xor(v, off, 64));
        f |= __shfl_xor(f, off, 64);
    }
    if (lane == 0) { sd.red[wave] = v; sd.flag[wave] = f; }
    __syncthreads();
    v = fmax(fmax(sd.red[0], sd.red[1]), fmax(sd.red[2], sd.red[3]));
    f = sd.flag[0] | sd.flag[1] | sd.flag[2] | sd.flag[3];
    __syncthreads();  // sd.red / sd.flag may be reused
}

// The decision for token t by one 256-thread workgroup, once every row's logit
// and bound are stored and L (the largest lower bound y - B over all rows) is
// known.  gather(consider) calls consider(row, y + B) for rows of this
// thread's share that can reach L (a superset of the candidates is fine).
// Leaves the token's arrival root at zero.  Logits and bounds are read
// with device-scope loads: they may have been stored by other workgroups of
// the same launch.
template <class Gather>
__device__ void lm_decide(const LmArgs& a, int t, double L, int any_nf, LmDecLds& sd, Gather gather) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* y = a.Y + (unsigned long long)t * a.ldy;
    const float* bn = a.Bnd + (unsigned long long)t * a.ldy;
    const float* x = a.X + (unsigned long long)t * a.ldx;
    unsigned* root = a.ws_arrive + (unsigned long long)t * kLmArr;
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
        if (tid == 0) st_dev(root, 0u);
        return;
    }

    // Candidates: y + B >= L (less a relative slack for the rounding of the
    // double sums); each is queued for recomputation.
    const double Lc = L - fabs(L) * 0x1p-50;
    if (tid == 0) { sd.cnt = 0; sd.nref = 0; sd.one = -1; }
    __syncthreads();
    auto consider = [&](int r, double h) {
        if (h < Lc) return;
        sd.one = r;  // any candidate; used only when there is exactly one
        const int q = atomicAdd(&sd.nref, 1);
        if (q < kLmKept) sd.kept[q] = r;
    };
    gather(consider);
    __syncthreads();
    const int nref = sd.nref;
    if (nref == 1) {
        if (tid == 0) { a.ids[t] = sd.one; st_dev(root, 0u); }
        return;
    }
    // All-zero activations: every reference logit is +-0, which compare
    // equal, so the first row wins.
    int nz = 0;
    for (int c = tid; c < a.cols; c += 256) nz |= (x[c] != 0.f);
    double unused = 0.0;
    block_max_or(unused, nz, sd);
    if (!nz) {
        if (tid == 0) { a.ids[t] = 0; st_dev(root, 0u); }
        return;
    }
    double bv = -INFINITY;
    int br = 0x7FFFFFFF;
    for (int q = wave; q < (nref < kLmKept ? nref : kLmKept); q += 4) {
        const int r = sd.kept[q];
        const double v = ref_row(a, r, x);
        if (better(v, r, bv, br)) { bv = v; br = r; }
    }
    if (nref > kLmKept) {
        // more rows to recompute than fit the list: recompute every such row, one per wave
        for (int r = wave; r < a.rows; r += 4) {
            const double h = (double)ld_dev(y + r) + (a.gamma * (double)ld_dev(bn + r) + a.abs_margin);
            if (h < Lc) continue;  // wave-uniform
            const double v = ref_row(a, r, x);
            if (better(v, r, bv, br)) { bv = v; br = r; }
        }
    }
    block_best(bv, br, sd);
    if (tid == 0) {
        a.ids[t] = br == 0x7FFFFFFF ? -1 : br;
        st_dev(root, 0u);
    }
}

__global__ __launch_bounds__(256) void lm_argmax_kernel(const LmArgs a) {
    const int t = blockIdx.y, w = blockIdx.x, tid = threadIdx.x;
    const float* y = a.Y + (unsigned long long)t * a.ldy;
    const float* bn = a.Bnd + (unsigned long long)t * a.ldy;
    const int chunk = (a.rows + kLmWgs - 1) / kLmWgs;
    const double g = a.gamma, am = a.abs_margin;
    auto range = [&](int k, int& q0, int& q1) {
        q0 = k * chunk < a.rows ? k * chunk : a.rows;
        q1 = q0 + chunk < a.rows ? q0 + chunk : a.rows;
    };
    auto hi = [&](int r) { return (double)y[r] + (g * (double)bn[r] + am); };
    auto lo = [&](int r) { return (double)y[r] - (g * (double)bn[r] + am); };

    __shared__ LmDecLds sd;
    __shared__ int s_cnt, s_last;  // s_cnt: local candidate count (pass 2)

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
    if (tid == 0) s_cnt = 0;
    block_max_or(lmax, nf, sd);

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
    if (tid == 0) {  // ... before the arrival
        unsigned* root = a.ws_arrive + (unsigned long long)t * kLmArr;
        s_last = arrive_tree(root + 1, root, 16, w, kLmWgs);
    }
    __syncthreads();
    if (!s_last) return;

    // ---- deciding workgroup of token t; thread k looks after workgroup k's range
    static_assert(kLmWgs == 256, "one thread per argmax workgroup");
    const int my_cnt = ld_dev(a.ws_cnt + (unsigned long long)t * kLmWgs + tid);
    double L = ld_dev(a.ws_L + (unsigned long long)t * kLmWgs + tid);
    int any_nf = my_cnt < 0;
    block_max_or(L, any_nf, sd);
    lm_decide(a, t, L, any_nf, sd, [&](auto& consider) {
        if (my_cnt > 0 && my_cnt <= kLmCand) {
            const unsigned long long base = ((unsigned long long)t * kLmWgs + tid) * kLmCand;
            for (int q = 0; q < my_cnt; ++q) consider(ld_dev(a.ws_cand + base + q), ld_dev(a.ws_candv + base + q));
        } else if (my_cnt > kLmCand) {
            int q0, q1;
            range(tid, q0, q1);
            for (int r = q0; r < q1; ++r) consider(r, hi(r));
        }
    });
}

// ---------------------------------------------------------------- fused batch-1 head
// For one vector the argmax rides on the bound matvec itself (lm_fused_kernel):
// each slot's leader lane keeps, over the rows it finishes, the largest lower
// bound y - B, and lists in the workgroup's LDS every row whose upper bound
// y + B reaches it at that moment (a superset of the rows that can reach the
// workgroup's final bound; a list that fills up marks the workgroup as
// overflowed).  When its rows are done a workgroup publishes one record -- its
// lower bound L_w and the listed rows that reach L_w -- and the last workgroup
// to arrive decides with lm_decide.  An overflowed workgroup makes the decider
// scan every row's stored logit and bound instead of the records.

constexpr int kLmWgList = 128;       // rows a workgroup lists while it runs
constexpr int kLmRecCand = 4;        // candidate rows a workgroup record holds
// Record of a workgroup, 8 qwords: L_w, h0, (count, r0), (r1, r2), (r3, 0), h1, h2, h3 -- candidate
// rows r and their y + B h, the largest h first (so a record whose h0 is below the deciding bound
// holds no candidate).  Count -1: a non-finite value seen; kLmRecCand + 1: rows not listed.
constexpr int kLmRecDw = 16;
constexpr int kLmFusedWgsMax = 2048;
constexpr int kLmRecPerThread = kLmFusedWgsMax / 256;  // records the decider's threads read each

typedef __attribute__((address_space(3))) int lds_i;
typedef __attribute__((address_space(3))) double lds_d;

struct LmObs {
    double g, am;
    lds_i* n;     // rows listed (may exceed kLmWgList: overflow)
    lds_i* lr;    // listed rows
    lds_d* lh;    // their y + B
    double lmax = -INFINITY;  // largest y - B this lane has seen
    int nf = 0;               // a non-finite logit or lower bound seen

    // Logits and bounds are stored with device-scope stores: the deciding
    // workgroup of this launch may read them.
    template <int B, int R>
    __device__ __forceinline__ void row(const MvDesc& d, long long r, int ri, const float (&acc)[R][B],
                                        const float (&bacc)[R][B], bool) {
        static_assert(B == 1 && R == 1, "one vector, one row per slot");
        const float y = acc[ri][0], s = bacc[ri][0];
        st_dev(d.Y + r, y);
        st_dev(d.Bnd + r, s);
        const double bd = g * (double)s + am;
        const double lo = (double)y - bd, hi = (double)y + bd;
        if (!isfinite(y) || !isfinite(lo)) nf = 1;
        lmax = fmax(lmax, lo);
        if (hi >= lmax - fabs(lmax) * 0x1p-50) {
            const int k = __hip_atomic_fetch_add(n, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            if (k < kLmWgList) { lr[k] = (int)r; lh[k] = hi; }
        }
    }
};

template <int T, bool AL>
__global__ __launch_bounds__(256) void lm_fused_kernel(const MvDesc d, const LmArgs a) {
    // the staged activations are read 16 bytes at a time: their base (placed
    // after the static LDS below) must be 16-byte aligned
    extern __shared__ __attribute__((aligned(16))) float smem[];
    __shared__ LmDecLds sd;
    __shared__ int s_n;
    __shared__ int s_lr[kLmWgList];
    __shared__ double s_lh[kLmWgList];
    __shared__ int s_cr[kLmRecCand];
    __shared__ double s_cv[kLmRecCand];
    __shared__ int s_last;
    const int tid = threadIdx.x;

    if (tid == 0) s_n = 0;
    __syncthreads();
    LmObs ob;
    ob.g = a.gamma;
    ob.am = a.abs_margin;
    ob.n = (lds_i*)&s_n;
    ob.lr = (lds_i*)s_lr;
    ob.lh = (lds_d*)s_lh;
    mv_body<T, 1, 1, AL, true, true, XDirect, 4, LmObs>(d, blockIdx.x, smem, ob);

    // this workgroup's record
    double lw = ob.lmax;
    int fl = ob.nf;
    if (tid == 0) sd.cnt = 0;
    block_max_or(lw, fl, sd);  // its barrier also orders the list writes before the reads below
    const int listed = s_n;
    const bool nf = fl & 1, ovf = listed > kLmWgList;
    if (!nf && !ovf && tid < listed) {
        const double lc = lw - fabs(lw) * 0x1p-50;
        if (s_lh[tid] >= lc) {
            const int k = atomicAdd(&sd.cnt, 1);
            if (k < kLmRecCand) { s_cr[k] = s_lr[tid]; s_cv[k] = s_lh[tid]; }
        }
    }
    static_assert(kLmWgList <= 256, "one thread per listed row");
    __syncthreads();
    const int cnt = nf ? -1 : (ovf || sd.cnt > kLmRecCand) ? kLmRecCand + 1 : sd.cnt;
    if (tid < kLmRecDw / 2) {
        const int nc = cnt >= 0 && cnt <= kLmRecCand ? cnt : 0;  // candidates the record lists
        int best = 0;
        for (int k = 1; k < nc; ++k) best = s_cv[k] > s_cv[best] ? k : best;
        auto row = [&](int k) {  // k-th listed row, the best first
            const int kk = k == 0 ? best : k == best ? 0 : k;
            return k < nc ? (unsigned long long)(unsigned)s_cr[kk] : 0ull;
        };
        auto hv = [&](int k) {
            const int kk = k == 0 ? best : k == best ? 0 : k;
            return k < nc ? (unsigned long long)__double_as_longlong(s_cv[kk]) : 0ull;
        };
        unsigned long long v = 0;
        switch (tid) {
        case 0: v = (unsigned long long)__double_as_longlong(lw); break;
        case 1: v = hv(0); break;
        case 2: v = (unsigned long long)(unsigned)cnt | (row(0) << 32); break;
        case 3: v = row(1) | (row(2) << 32); break;
        case 4: v = row(3); break;
        default: v = hv(tid - 4); break;
        }
        st_dev(reinterpret_cast<unsigned long long*>(a.ws_rec) + (unsigned long long)blockIdx.x * (kLmRecDw / 2) + tid,
               v);
    }
    drain_dev();  // every wave's logit, bound and record stores have completed ...
    __syncthreads();
    if (tid == 0) s_last = arrive_tree(a.ws_arrive + 1, a.ws_arrive, kLmFan, blockIdx.x, gridDim.x);  // ... before the arrival
    __syncthreads();
    if (!s_last) return;

    // ---- deciding workgroup; thread t reads records t, t + 256, ..., all
    // loads of a pass issued before any is used
    const int nwg = (int)gridDim.x;
    const unsigned long long* recs = reinterpret_cast<const unsigned long long*>(a.ws_rec);
    unsigned long long q0[kLmRecPerThread], q1[kLmRecPerThread], q2[kLmRecPerThread];
#pragma unroll
    for (int i = 0; i < kLmRecPerThread; ++i) {
        const int k = tid + 256 * i;
        const unsigned long long* p = recs + (unsigned long long)(k < nwg ? k : 0) * (kLmRecDw / 2);
        q0[i] = ld_dev(p);
        q1[i] = ld_dev(p + 1);
        q2[i] = ld_dev(p + 2);
    }
    double L = -INFINITY;
    int f = 0;
#pragma unroll
    for (int i = 0; i < kLmRecPerThread; ++i) {
        if (tid + 256 * i >= nwg) continue;
        const int c = (int)(unsigned)q2[i];
        L = fmax(L, __longlong_as_double((long long)q0[i]));
        f |= (c < 0) | ((c > kLmRecCand) << 1);
    }
    block_max_or(L, f, sd);
    const bool any_ovf = (f >> 1) & 1;
    const double Lc = L - fabs(L) * 0x1p-50;
    lm_decide(a, 0, L, f & 1, sd, [&](auto& consider) {
        if (any_ovf) {
            // some workgroup did not list all its rows: every row's stored logit and bound, 8 rows a step
            for (int r0 = 0; r0 < a.rows; r0 += 8 * 256) {
                float yv[8], bv[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int r = r0 + tid + 256 * u < a.rows ? r0 + tid + 256 * u : a.rows - 1;
                    yv[u] = ld_dev(a.Y + r);
                    bv[u] = ld_dev(a.Bnd + r);
                }
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (r0 + tid + 256 * u < a.rows)
                        consider(r0 + tid + 256 * u, (double)yv[u] + (a.gamma * (double)bv[u] + a.abs_margin));
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < kLmRecPerThread; ++i) {
            const int k = tid + 256 * i;
            const double h0 = __longlong_as_double((long long)q1[i]);
            const int c = (int)(unsigned)q2[i];
            if (k >= nwg || c < 1 || !(h0 >= Lc)) continue;  // h0 is the record's largest
            consider((int)(q2[i] >> 32), h0);
            if (c > 1) {
                const unsigned long long* p = recs + (unsigned long long)k * (kLmRecDw / 2);
                const unsigned long long r12 = ld_dev(p + 3), r3 = ld_dev(p + 4);
                const double h1 = __longlong_as_double((long long)ld_dev(p + 5));
                const double h2 = __longlong_as_double((long long)ld_dev(p + 6));
                const double h3 = __longlong_as_double((long long)ld_dev(p + 7));
                consider((int)(unsigned)r12, h1);
                if (c > 2) consider((int)(r12 >> 32), h2);
                if (c > 3) consider((int)(unsigned)r3, h3);
            }
        }
    });
}

// ---------------------------------------------------------------- workspace

struct LmWorkspace {
    void* bnd = nullptr;     // float [tokens][ldl]
    size_t bnd_cap = 0;      // bytes
    void* tok = nullptr;     // per token: L, cnt, cand, candv (kLmTokBytes); then kLmArr arrival counters per token
    size_t tok_cap = 0;      // bytes
};

// Per-token workspace bytes: L (double) and cnt (int) per argmax workgroup,
// then its candidate rows (int) and their upper bounds (double).
constexpr size_t kLmTokBytes = (size_t)kLmWgs * (8 + 4 + kLmCand * (4 + 8));
// ... and with its arrival counters
constexpr size_t kLmTokTotal = kLmTokBytes + kLmArr * sizeof(unsigned int);

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
    const size_t bb = bnd_floats * sizeof(float), tb = tokens * kLmTokTotal;
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

// Zero n arrival counters (a kernel, not a memset, so that it can be
// captured into a graph).
__global__ __launch_bounds__(256) void lm_clear_kernel(unsigned int* counters, int n) {
    for (int i = threadIdx.x; i < n; i += 256) counters[i] = 0u;
}

// PYRITE_LM_FUSED=0 keeps batch-1 heads on the two-kernel path (bound matvec,
// then lm_argmax_kernel).
static bool lm_fused_env() {
    static const bool on = [] {
        const char* e = getenv("PYRITE_LM_FUSED");
        return !(e && e[0] == '0');
    }();
    return on;
}

// Workgroups resident per CU of one fused kernel instance.
template <int T, bool AL>
static int lm_fused_per_cu(size_t lds) {
    static const int n = [lds] {
        int v = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, lm_fused_kernel<T, AL>, 256, lds) != hipSuccess || v < 1)
            v = 1;
        return v;
    }();
    return n;
}

// Launch the fused head for one vector; 1 when the matrix is not eligible
// (plain types, activations that do not fit LDS, unaligned weights of a
// dword-multiple block format), which then takes the two-kernel path.
template <int T>
static int lm_fused_launch_t(bool al, const MatvecArgs& m, float* bnd, const LmArgs& a, size_t max_recs,
                             hipStream_t stream) {
    if constexpr (Geo<T>::bs == 1) {
        return 1;
    } else {
        constexpr bool AL = Geo<T>::bpb % 4 == 0;
        if ((AL && !al) || !use_xl<T, 1, true>((int)m.cols)) return 1;
        const size_t lds = lds_bytes<T, 1, true>((int)m.cols, true);
        if (lds + 4096 > 65536) return 1;  // the kernel's own LDS (under 4 KiB) comes on top
        MvDesc d{};
        d.W = static_cast<const uint8_t*>(m.w);
        d.row_bytes = m.cols / Geo<T>::bs * Geo<T>::bpb;
        d.X = m.x;
        d.ldx = m.ldx;
        d.Y = m.y;
        d.ldy = m.ldy;
        d.rows = (int)m.rows;
        d.cols = (int)m.cols;
        d.lpr_log2 = mat_shape<T, 1, AL>(d.rows, d.cols).lpr_log2;
        d.Bnd = bnd;
        const long long rows_per_wg = (long long)kMvWaves * (64 >> d.lpr_log2);
        long long nwg = (long long)lm_fused_per_cu<T, AL>(lds) * dev_info().cus;
        const long long need = ((long long)m.rows + rows_per_wg - 1) / rows_per_wg;
        if (need < nwg) nwg = need;
        if (nwg > kLmFusedWgsMax) nwg = kLmFusedWgsMax;
        if ((size_t)nwg > max_recs) nwg = (long long)max_recs;
        if (nwg < 1) return -4;
        d.wg_begin = 0;
        d.wg_count = (int)nwg;
        hipLaunchKernelGGL((lm_fused_kernel<T, AL>), dim3((unsigned)nwg), dim3(256), lds, stream, d, a);
        return hipGetLastError() == hipSuccess ? 0 : -4;
    }
}

static int lm_fused_launch(int type, bool al, const MatvecArgs& m, float* bnd, const LmArgs& a, size_t max_recs,
                           hipStream_t stream) {
#define PYRITE_CASE(T) \
    case T: return lm_fused_launch_t<T>(al, m, bnd, a, max_recs, stream);
    switch (type) {
        PYRITE_FOR_EACH_TYPE(PYRITE_CASE)
    default: return 1;
    }
#undef PYRITE_CASE
}

// Tokens' worth of workspace the fused head's records need (its workgroup
// records alias the per-token arrays).
constexpr size_t kLmFusedTokens = (kLmFusedWgsMax * kLmRecDw * 4 + kLmTokBytes - 1) / kLmTokBytes;

// The bound matvec, then the argmax kernel (or, for one vector, the fused
// kernel that does both), over workspace memory the caller provides: bnd
// (floats laid out like the logits) and a token block carved by lm_carve for
// `tok_cap` tokens.  clear: zero the arrival counters first.
static int lm_head_run(int type, const TypeGeo& g, bool al, size_t max_cols, const MatvecArgs& m, int* ids,
                       size_t batch, float* bnd, void* tok, size_t tok_cap, bool clear, hipStream_t stream) {
    LmArgs a;
    lm_carve(tok, tok_cap, a);
    a.ws_rec = static_cast<unsigned int*>(tok);
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
    if (clear) {
        hipLaunchKernelGGL(lm_clear_kernel, dim3(1), dim3(256), 0, stream, a.ws_arrive, (int)(batch * kLmArr));
        if (hipGetLastError() != hipSuccess) return -4;
    }
    if (batch == 1 && lm_fused_env()) {
        const int rc = lm_fused_launch(type, al, m, bnd, a, tok_cap * kLmTokBytes / (kLmRecDw * 4), stream);
        if (rc != 1) return rc;
    }
    if (const int rc = valu_group_launch<true>(type, g, al, &m, &bnd, 1, batch, max_cols, stream, nullptr, nullptr))
        return rc;
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
    if (const int rc = lm_workspace(batch * ldl, batch > kLmFusedTokens ? batch : kLmFusedTokens, stream, &ws))
        return rc;
    return lm_head_run(type, g, al, max_cols, m, ids, batch, static_cast<float*>(ws->bnd), ws->tok,
                       ws->tok_cap / kLmTokTotal, false, stream);
}

// ---------------------------------------------------------------- allocation-free variant
// The LM head for callers that cannot allocate (code under graph capture,
// serving loops): its workspace is this file-scope device array instead of
// hipMalloc'ed memory.  Layout: the token block for kLmScratchTokens tokens
// (lm_carve), then, from byte kLmScratchBndOffset, the bound floats.  Each
// GPU holds its own copy until the process ends; every call on a GPU shares it
// (the last call's contents stay), so calls that overlap on one GPU race.
constexpr size_t kLmScratchBytes = size_t(8) << 20;
constexpr size_t kLmScratchTokens = 8;
constexpr size_t kLmScratchBndOffset = 811264;
static_assert(kLmScratchTokens * kLmTokTotal <= kLmScratchBndOffset, "the token block ends before the bounds");
constexpr size_t kLmScratchBndFloats = (kLmScratchBytes - kLmScratchBndOffset) / sizeof(float);
static_assert(kLmScratchBndFloats == 1894336, "the limit quoted in the error message and the header");
static_assert(kLmScratchTokens >= kLmFusedTokens, "the fused head's records fit the scratch token block");

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
