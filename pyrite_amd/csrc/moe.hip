// Qwen3-MoE FFN layer on the device, driven by device-side expert ids.
//
// Reference (all fp64, one token at a time): pyrite/executor.py:757-793
// (_moe): router logits = pyrite_matvec of ffn_gate_inp (E x H), probs =
// softmax (pyrite/tensor_ops.py:513-521), experts ranked by (-p, e), the first
// k kept, weights renormalised when norm_topk_prob and their sum is positive,
// scaled when expert_weights_scale != 1, then out = sum over the chosen slots
// (in rank order, weight 0 skipped) of w * expert(x); expert(x) =
// down . (silu(gate . x) * (up . x)) (executor.py:672-683, silu
// tensor_ops.py:509-510).  Expert e of a stacked [E][rows][cols] GGUF tensor is
// the contiguous byte slice e * rows * row_bytes (pyrite/qwen3_moe.py:364-398).
//
// Kernels, all on one stream, no host round trip:
//   moe_router_kernel   fp64 router logits (tree order) and sum |w x| per row,
//                       one expert row against four tokens per wave
//   moe_router_route_kernel  router and routing in one launch for up to 16
//                       tokens (the last of a token's workgroups routes it)
//   moe_route_kernel    per token: exact ranking (rows whose rounding
//                       interval overlaps a top-(k+1) row are recomputed in
//                       the reference's own order), softmax, top-k, weights;
//                       the last token's workgroup buckets (token, slot)
//                       pairs by expert into padded chunks of MB tokens
//   moe_mv_kernel       gate and up (one launch), then down: persistent
//                       workgroups walk (matrix, chunk, row tile) items and run
//                       the VALU matvec body on each, weights read once per
//                       chunk; the gate/up launch gathers each chunk's tokens
//                       while staging them, the down launch applies
//                       silu(gate) * up (fp32) while staging
//   moe_gather_kernel,  used instead when the staged activations would not
//   moe_swiglu_kernel   fit the LDS budget
//   moe_combine_kernel  out = sum of w * down-out in slot order (fp64 inside)
#include "dequant.h"
#include "libm_exp.h"
#include "mv_kernel.h"
#include "mx_traits.h"

namespace pyrite {

constexpr int kMoeMaxE = 1024;  // experts supported by the route kernel
constexpr int kMoeMaxK = 32;    // experts per token supported
constexpr int kMoeFusedRouteBatch = 16;  // up to this batch, router and routing share one launch

// ---------------------------------------------------------------- router

// Router logit of one (expert row, token) by one wave, fp64 products and tree
// sums, with the sum of |products| for the rounding bound.  F32 routers (the
// Qwen3 case) read 4 weights per lane per load; other types decode element by
// element.  Every lane returns the totals.
__device__ __forceinline__ void moe_router_row(int type, const uint8_t* __restrict__ rp, int H, int bs, int bpb,
                                               const float* __restrict__ x, double& acc, double& mag) {
    const int lane = threadIdx.x & 63;
    acc = 0.0;
    mag = 0.0;
    if (type == T_F32 && (H & 3) == 0 && ((reinterpret_cast<uintptr_t>(rp) | reinterpret_cast<uintptr_t>(x)) & 15) == 0) {
        const float4* w4 = reinterpret_cast<const float4*>(rp);
        const float4* x4 = reinterpret_cast<const float4*>(x);
        const int n4 = H / 4;
        // eight float4 pairs per lane requested before any is used (one
        // memory round trip for a 2048-column row instead of eight); the sum
        // order per lane stays column-ascending
        for (int c0 = lane; c0 < n4; c0 += 64 * 8) {
            float4 w[8], v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                // past the row: the last float4 again (not used below)
                const int c = c0 + 64 * k < n4 ? c0 + 64 * k : n4 - 1;
                w[k] = w4[c];
                v[k] = x4[c];
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                // no branch here: the loads above stay ahead of every use
                const bool in = c0 + 64 * k < n4;
                const double p0 = (double)w[k].x * v[k].x, p1 = (double)w[k].y * v[k].y;
                const double p2 = (double)w[k].z * v[k].z, p3 = (double)w[k].w * v[k].w;
                acc += in ? (p0 + p1) + (p2 + p3) : 0.0;
                mag += in ? (fabs(p0) + fabs(p1)) + (fabs(p2) + fabs(p3)) : 0.0;
            }
        }
    } else {
        for (int c = lane; c < H; c += 64) {
            const int blk = c / bs;
            const double p = dq_elem<double>(type, rp + (unsigned long long)blk * bpb, c - blk * bs) * (double)x[c];
            acc += p;
            mag += fabs(p);
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        acc += __shfl_xor(acc, off, 64);
        mag += __shfl_xor(mag, off, 64);
    }
}

constexpr int kMoeRouterTok = 4;  // tokens per wave of moe_router_kernel

// Workgroup (x, y): wave w computes expert row 4x + w against tokens
// 4y .. 4y + 3, each (row, token) logit and magnitude sum formed exactly as
// moe_router_row forms it.  F32 rows (the Qwen3 case) are read once for the
// four tokens: a batch of a lane's eight float4s of the row and of each
// token's activations is requested before any is used.
__global__ __launch_bounds__(256) void moe_router_kernel(int type, const uint8_t* __restrict__ W,
                                                         unsigned long long row_bytes, int E, int H, int bs, int bpb,
                                                         const float* __restrict__ X, unsigned long long ldx,
                                                         int batch, double* __restrict__ logits,
                                                         double* __restrict__ mags) {
    constexpr int NT = kMoeRouterTok;
    const int lane = threadIdx.x & 63;
    const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int t0 = blockIdx.y * NT;
    if (e >= E) return;  // wave-uniform; no barrier below
    const uint8_t* rp = W + (unsigned long long)e * row_bytes;
    const float* x0 = X + (unsigned long long)t0 * ldx;
    double acc[NT], mag[NT];
    const bool f32 = type == T_F32 && (H & 3) == 0 && (ldx & 3) == 0 &&
                     ((reinterpret_cast<uintptr_t>(rp) | reinterpret_cast<uintptr_t>(x0)) & 15) == 0;
    if (f32) {
        const float4* w4 = reinterpret_cast<const float4*>(rp);
        const int n4 = H / 4;
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = mag[t] = 0.0;
        for (int c0 = lane; c0 < n4; c0 += 64 * 8) {
            float4 w[8], v[NT][8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                // past the row: the last float4 again (not used below)
                const int c = c0 + 64 * k < n4 ? c0 + 64 * k : n4 - 1;
                w[k] = w4[c];
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    // tokens past the batch read the last token (not stored)
                    const int tt = t0 + t < batch ? t0 + t : batch - 1;
                    v[t][k] = reinterpret_cast<const float4*>(X + (unsigned long long)tt * ldx)[c];
                }
            }
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const bool in = c0 + 64 * k < n4;
                    const double p0 = (double)w[k].x * v[t][k].x, p1 = (double)w[k].y * v[t][k].y;
                    const double p2 = (double)w[k].z * v[t][k].z, p3 = (double)w[k].w * v[t][k].w;
                    acc[t] += in ? (p0 + p1) + (p2 + p3) : 0.0;
                    mag[t] += in ? (fabs(p0) + fabs(p1)) + (fabs(p2) + fabs(p3)) : 0.0;
                }
        }
#pragma unroll
        for (int t = 0; t < NT; ++t)
            for (int off = 32; off > 0; off >>= 1) {
                acc[t] += __shfl_xor(acc[t], off, 64);
                mag[t] += __shfl_xor(mag[t], off, 64);
            }
    } else {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int tt = t0 + t < batch ? t0 + t : batch - 1;
            moe_router_row(type, rp, H, bs, bpb, X + (unsigned long long)tt * ldx, acc[t], mag[t]);
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (t0 + t >= batch) break;
            logits[(unsigned long long)(t0 + t) * E + e] = acc[t];
            mags[(unsigned long long)(t0 + t) * E + e] = mag[t];
        }
    }
}

// The reference's fp64 router logit of one row, computed by one wave in the
// reference's column order (pyrite/kernels/native.c:527-553).
__device__ double moe_ref_row(int type, const uint8_t* rp, int H, int bs, int bpb, const float* x) {
    const int lane = threadIdx.x & 63;
    double s = 0.0;
    for (int base = 0; base < H; base += 64) {
        const int c = base + lane;
        double p = 0.0;
        if (c < H) {
            const int blk = c / bs;
            p = __dmul_rn(dq_elem<double>(type, rp + (unsigned long long)blk * bpb, c - blk * bs), (double)x[c]);
        }
        const int n = H - base < 64 ? H - base : 64;
        for (int k = 0; k < n; ++k) {
            const unsigned long long u = (unsigned long long)__double_as_longlong(p);
            const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)u, k);
            const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(u >> 32), k);
            s = __dadd_rn(s, __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo)));
        }
    }
    return s;
}

// The same logit computed by one thread, column after column: a rounded
// product, then a rounded add, per column.  Used when every row must be exact.
__device__ double moe_ref_row_seq(int type, const uint8_t* rp, int H, int bs, int bpb, const float* x) {
    double s = 0.0;
    for (int c = 0; c < H; ++c) {
        const int blk = c / bs;
        s = __dadd_rn(s, __dmul_rn(dq_elem<double>(type, rp + (unsigned long long)blk * bpb, c - blk * bs),
                                   (double)x[c]));
    }
    return s;
}

// ---------------------------------------------------------------- routing + plan

struct MoePlan {
    int* pair_tok;   // [max_pairs] token of each padded pair, -1 for padding
    int* pos;        // [batch * k] padded pair index of (token, slot)
    int* totals;     // [2]: padded pairs, chunks
    int* chunk_e;    // [chunks] expert of each chunk; chunk c holds padded pairs [c * MB, (c + 1) * MB)
    unsigned* amax;  // [padded pairs] zeroed with the plan (matrix-core experts), or null
};

struct MoeRouteArgs {
    int type;
    const uint8_t* W;
    unsigned long long row_bytes;
    int E, H, bs, bpb, k, MB;
    int norm_topk;
    double scale;
    double gamma;  // rounding budget per unit of sum |w x|
    const float* X;
    unsigned long long ldx;
    const double* logits;
    const double* mags;
    int* ids;          // [batch][k]
    double* wts;       // [batch][k]
    float* wts_out;    // [batch][k] or null
    int* ids_out;      // [batch][k] or null (caller's copy)
    int batch;
    unsigned int* arrive;
    MoePlan plan;
};

__device__ __forceinline__ bool rank_before(double la, int a, double lb, int b) {
    return la > lb || (la == lb && a < b);
}

// Routing of token t by a whole 256-thread workgroup: exact ranking, weights,
// and (last token's workgroup) the plan.  CO: the logits were written by other
// workgroups of the same launch and are read with device-coherent loads.
template <bool CO>
__device__ void moe_route_token(const MoeRouteArgs& a, const int t) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = a.E, k = a.k;
    __shared__ double s_l[kMoeMaxE];
    __shared__ double s_b[kMoeMaxE];
    __shared__ unsigned char s_mark[kMoeMaxE];
    __shared__ int s_top[kMoeMaxK + 1];
    __shared__ int s_marked[kMoeMaxE];
    __shared__ double s_red[4];
    __shared__ int s_poff[kMoeMaxE + 1];
    __shared__ int s_nmarked, s_last;
    const float* x = a.X + (unsigned long long)t * a.ldx;
    __shared__ int s_rank[kMoeMaxE];
    __shared__ double s_tl[kMoeMaxK + 1], s_tb[kMoeMaxK + 1];
    __shared__ double s_total;
    __shared__ double s_w[kMoeMaxK];

    // NaN logits rank last (as -inf), keeping the ranks a total order
    int nonfinite = 0;
    for (int e = tid; e < E; e += 256) {
        const unsigned long long o = (unsigned long long)t * E + e;
        const double l = CO ? ld_dev(a.logits + o) : a.logits[o];
        s_l[e] = isnan(l) ? -INFINITY : l;
        s_b[e] = a.gamma * (CO ? ld_dev(a.mags + o) : a.mags[o]);
        s_mark[e] = 0;
        nonfinite |= !isfinite(l) || !isfinite(s_b[e]);
    }
    if (tid == 0) s_nmarked = 0;
    nonfinite = __syncthreads_or(nonfinite);

    // rank of every expert in (-logit, e) order (a total order: ranks are
    // unique); the first n land in s_top.  Up to 128 experts, two threads
    // count each expert's rank over half of the others each.
    auto rank_top = [&](int n) {
        if (E <= 128) {  // block-uniform branch
            const int e = tid & 127, h = tid >> 7;
            const int j0 = h * ((E + 1) >> 1), j1 = h ? E : (E + 1) >> 1;
            int r = 0;
            if (e < E) {
                const double le = s_l[e];
#pragma unroll 8
                for (int j = j0; j < j1; ++j) r += rank_before(s_l[j], j, le, e);
                if (h == 0) s_rank[e] = r;
            }
            __syncthreads();
            if (e < E && h == 1) {
                r += s_rank[e];
                if (r < n) s_top[r] = e;
            }
        } else {
            for (int e = tid; e < E; e += 256) {
                const double le = s_l[e];
                int r = 0;
#pragma unroll 8
                for (int j = 0; j < E; ++j) r += rank_before(s_l[j], j, le, e);
                if (r < n) s_top[r] = e;
            }
        }
        __syncthreads();
    };

    // 1. tree-order top k+1; mark every row whose interval [l - B, l + B]
    //    meets the interval of one of them (their order is then uncertain;
    //    rows whose bounds are both zero are exact)
    const int kk = k + 1 <= E ? k + 1 : E;
    rank_top(kk);
    {
        // the top rows' logits and bounds gathered next to their ids, so the
        // scan below reads them without a dependent lookup
        if (tid < kk) {
            s_tl[tid] = s_l[s_top[tid]];
            s_tb[tid] = s_b[s_top[tid]];
        }
        __syncthreads();
        // up to 128 experts, two threads share each expert's top rows
        const bool two = E <= 128;
        const int e0 = two ? (tid & 127) : tid, q0 = two ? (tid >> 7) : 0, qs = two ? 2 : 1;
        for (int e = e0; e < E; e += two ? E : 256) {
            const double le = s_l[e], be = s_b[e];
            const bool fe = isfinite(le);
            for (int q = q0; q < kk; q += qs) {
                const int i = s_top[q];
                const double tl = s_tl[q], bb = s_tb[q] + be;
                if (i != e && ((bb > 0 && fabs(tl - le) <= bb * (1 + 0x1p-40)) || !fe || !isfinite(tl))) {
                    s_mark[e] = 1;
                    s_mark[i] = 1;
                }
            }
        }
    }
    __syncthreads();
    for (int e = tid; e < E; e += 256)
        if (s_mark[e]) s_marked[atomicAdd(&s_nmarked, 1)] = e;
    __syncthreads();
    // 2. recompute the marked rows exactly (one wave each), then rank again
    const int nm = s_nmarked;
    for (int q = wave; q < nm; q += 4) {
        const int e = s_marked[q];
        const double v = moe_ref_row(a.type, a.W + (unsigned long long)e * a.row_bytes, a.H, a.bs, a.bpb, x);
        if (lane == 0) { s_l[e] = isnan(v) ? -INFINITY : v; s_b[e] = 0.0; }
    }
    __syncthreads();
    if (nm > 0) rank_top(kk);

    // 3. The reference ranks by (-p, e) with p = exp(l - peak) / total
    //    (pyrite/tensor_ops.py:513-521: exp is the host libm's, total is
    //    summed left to right), not by (-l, e).  The top k+1 positions above
    //    are the exact (-l, e) order.  Where each of the first k positions
    //    leads the next by more than the rounding of l - peak, exp and the
    //    division can take away (the margin below, for an exp within 1 ulp),
    //    p strictly decreases along them and every other row has p no larger
    //    than position k's, so the (-p, e) order of the first k is this one.
    //    Otherwise (logits within about 2^-48 of each other, or a probability
    //    near the subnormal range), every row is recomputed exactly and the
    //    probabilities are formed as the reference forms them.  Non-finite
    //    logits keep the (-l, e) order, NaN last.
    // one thread per pair (i, i + 1), i < k, i + 1 < kk
    bool slow;
    {
        const int np = kk - 1 < k ? kk - 1 : k;
        int bad = 0;
        if (!nonfinite && tid < np) {
            const double l0 = s_l[s_top[0]], b0 = s_b[s_top[0]];
            const int ea = s_top[tid], eb = s_top[tid + 1];
            const double la = s_l[ea], lb = s_l[eb], ba = s_b[ea], bb = s_b[eb];
            if (!(ba == 0.0 && bb == 0.0 && la == lb)) {  // equal exact logits: equal p, index order
                const double gap = (la - lb) - (ba + bb);
                const double margin = 0x1p-48 * (1.0 + fabs(la - l0) + fabs(lb - l0) + b0 + ba + bb);
                bad = !(gap > margin) || lb - l0 < -700.0;
            }
        }
        slow = __syncthreads_or(bad);  // block-uniform
    }
    if (slow) {
        // every row as the reference computes it (pyrite/kernels/native.c:527-553)
        for (int e = tid; e < E; e += 256) {
            if (s_b[e] != 0.0) {
                s_l[e] = moe_ref_row_seq(a.type, a.W + (unsigned long long)e * a.row_bytes, a.H, a.bs, a.bpb, x);
                s_b[e] = 0.0;
            }
        }
        __syncthreads();
        // position 0 holds the exact first maximum
        const double peak = s_l[s_top[0]];
        for (int e = tid; e < E; e += 256) s_b[e] = libm_exp(s_l[e] - peak);
        __syncthreads();
        if (tid == 0) {
            double tot = 0.0;
            for (int e = 0; e < E; ++e) tot += s_b[e];
            s_total = tot;
        }
        __syncthreads();
        // the peak's term is exp(0) = 1, so the total is at least 1
        for (int e = tid; e < E; e += 256) s_l[e] = s_b[e] / s_total;
        __syncthreads();
        rank_top(k);  // by (-p, e) now
    }

    // 4. the chosen probabilities: exact in the slow case; otherwise the
    //    device's exp (within an ulp of the host's) and a tree total, which
    //    move the weights by fp64 rounding only
    const double peak = s_l[s_top[0]];
    if (!slow && a.norm_topk && !nonfinite) {
        // renormalised weights: p_s / (sum of the k chosen p) = e_s / (sum
        // of the k chosen e) with e = exp(l - peak), so the softmax total
        // cancels and only the chosen terms are formed (the same fp64
        // rounding-level difference as the tree total below)
        if (tid < k) s_w[tid] = exp(s_l[s_top[tid]] - peak);
    } else if (!slow) {
        double tot = 0.0;
        for (int e = tid; e < E; e += 256) {
            const double v = exp(s_l[e] - peak);
            s_b[e] = v;  // the bounds are no longer needed
            tot += v;
        }
        for (int off = 32; off > 0; off >>= 1) tot += __shfl_xor(tot, off, 64);
        if (lane == 0) s_red[wave] = tot;
        __syncthreads();
        const double total = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
        if (tid < k) s_w[tid] = total <= 0.0 ? 1.0 / (double)E : s_b[s_top[tid]] / total;
    } else if (tid < k) {
        s_w[tid] = s_l[s_top[tid]];
    }
    __syncthreads();
    // slot q's weight: renormalised by the sum of the k probabilities taken
    // in rank order (each slot's thread forms the same sum), then scaled
    if (tid < k) {
        const int q = tid;
        double tk = 0.0;
        if (a.norm_topk)
            for (int j = 0; j < k; ++j) tk += s_w[j];
        double w = s_w[q];
        if (a.norm_topk && tk > 0) w = w / tk;
        if (a.scale != 1.0) w = w * a.scale;
        const unsigned long long o = (unsigned long long)t * k + q;
        st_dev(a.ids + o, s_top[q]);
        a.wts[o] = w;
        if (a.ids_out) a.ids_out[o] = s_top[q];
        if (a.wts_out) a.wts_out[o] = (float)w;
    }
    if (a.batch > 1) {
        drain_dev();  // this token's ids have completed before its arrival
        __syncthreads();
    }
    // a single token's workgroup is the last by definition (and keeps its ids in LDS)
    if (tid == 0) s_last = a.batch == 1 ? 1 : (arrive_dev(a.arrive) == (unsigned)a.batch - 1);
    __syncthreads();
    if (!s_last) return;

    // 4. plan (last workgroup): bucket the (token, slot) pairs by expert,
    //    padded to chunks of MB.  The order inside a bucket does not matter:
    //    each pair's results are computed independently of its chunk mates.
    const MoePlan& p = a.plan;
    if (a.batch == 1 && a.MB == 1) {
        // One token, one pair per chunk, pairs in slot order (pair q is slot
        // q, so the combine reads them without the position table).  The k
        // experts are distinct, so no bucket holds two pairs.
        if (tid < k) {
            p.pair_tok[tid] = 0;
            p.pos[tid] = tid;
            p.chunk_e[tid] = s_top[tid];
        }
        if (tid == 0) {
            p.totals[0] = k;
            p.totals[1] = k;
        }
        return;  // a single token never counted an arrival
    }
    int* s_cnt = s_marked;  // reuse: E ints
    for (int e = tid; e < E; e += 256) s_cnt[e] = 0;
    // every token's ids, read once (device-coherent loads) into LDS
    constexpr int kIdsLds = 4096;
    __shared__ int s_ids[kIdsLds];
    const int npairs = a.batch * k;
    const bool ids_in_lds = npairs <= kIdsLds;
    auto id_of = [&](int q) { return ids_in_lds ? s_ids[q] : ld_dev(a.ids + q); };
    if (ids_in_lds) {
        if (a.batch == 1) {
            for (int q = tid; q < npairs; q += 256) s_ids[q] = s_top[q];
        } else {
            for (int q = tid; q < npairs; q += 256) s_ids[q] = ld_dev(a.ids + q);
        }
    }
    __syncthreads();
    for (int q = tid; q < npairs; q += 256) atomicAdd(&s_cnt[id_of(q)], 1);
    __syncthreads();
    // exclusive prefix sums over experts of padded pairs: each thread scans
    // 4 consecutive experts, then the 256 thread totals
    {
        const int e0 = tid * 4;
        int cp[4], sp = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = e0 + j;
            const int n = e < E ? s_cnt[e] : 0;
            cp[j] = sp;
            sp += (n + a.MB - 1) / a.MB * a.MB;
        }
        // inclusive scan across the wave
        int ip = sp;
        for (int off = 1; off < 64; off <<= 1) {
            const int up = __shfl_up(ip, off, 64);
            if (lane >= off) ip += up;
        }
        __shared__ int s_wp[4];
        if (lane == 63) s_wp[wave] = ip;
        __syncthreads();
        int bp = 0;
        for (int w2 = 0; w2 < wave; ++w2) bp += s_wp[w2];
        bp += ip - sp;  // exclusive prefix of this thread
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (e0 + j < E) s_poff[e0 + j] = bp + cp[j];
        if (tid == 255) {
            const int tp = bp + sp;  // a multiple of MB
            s_poff[E] = tp;
            p.totals[0] = tp;
            p.totals[1] = tp / a.MB;
        }
        __syncthreads();
        // padded pair offsets are multiples of MB, so expert e owns chunks
        // [poff[e] / MB, poff[e + 1] / MB)
        for (int e = tid; e < E; e += 256) {
            s_cnt[e] = s_poff[e];  // fill cursors
            for (int c = s_poff[e] / a.MB; c < s_poff[e + 1] / a.MB; ++c) p.chunk_e[c] = e;
        }
        __syncthreads();
    }
    for (int q = tid; q < npairs; q += 256) {
        const int slot = atomicAdd(&s_cnt[id_of(q)], 1);
        p.pair_tok[slot] = q / k;
        p.pos[q] = slot;
    }
    __syncthreads();
    for (int e = tid; e < E; e += 256)
        for (int q = s_cnt[e]; q < s_poff[e + 1]; ++q) p.pair_tok[q] = -1;
    if (p.amax)  // the gate/up launch folds each pair's largest |act| into it
        for (int q = tid; q < s_poff[E]; q += 256) p.amax[q] = 0u;
    if (tid == 0) st_dev(a.arrive, 0u);
}

__global__ __launch_bounds__(256) void moe_route_kernel(const MoeRouteArgs a) { moe_route_token<false>(a, blockIdx.x); }

// Router and routing in one launch (small batches): workgroup (x, t) computes
// the logits of experts 4x .. 4x + 3 (one per wave) for token t; the last of
// token t's workgroups to arrive routes the token.  tok_arrive[t] is zero
// before the launch and is left at zero.
__global__ __launch_bounds__(256) void moe_router_route_kernel(const MoeRouteArgs a, unsigned* tok_arrive) {
    const int t = blockIdx.y, wave = threadIdx.x >> 6;
    const int e = blockIdx.x * 4 + wave;
    if (e < a.E) {  // wave-uniform
        double acc, mag;
        moe_router_row(a.type, a.W + (unsigned long long)e * a.row_bytes, a.H, a.bs, a.bpb,
                       a.X + (unsigned long long)t * a.ldx, acc, mag);
        if ((threadIdx.x & 63) == 0) {
            st_dev(const_cast<double*>(a.logits) + (unsigned long long)t * a.E + e, acc);
            st_dev(const_cast<double*>(a.mags) + (unsigned long long)t * a.E + e, mag);
        }
    }
    drain_dev();  // this workgroup's logits have completed before its arrival
    __syncthreads();
    __shared__ int s_go;
    if (threadIdx.x == 0) s_go = arrive_dev(tok_arrive + t) == gridDim.x - 1;
    __syncthreads();
    if (!s_go) return;
    if (threadIdx.x == 0) st_dev(tok_arrive + t, 0u);
    moe_route_token<true>(a, t);
}

// ---------------------------------------------------------------- gather, swiglu, combine

__global__ __launch_bounds__(256) void moe_gather_kernel(const float* __restrict__ X, unsigned long long ldx, int H,
                                                         const int* __restrict__ pair_tok,
                                                         const int* __restrict__ totals, int max_pairs,
                                                         float* __restrict__ XG) {
    const int npad = totals[0];
    for (int q = blockIdx.x; q < npad && q < max_pairs; q += gridDim.x) {
        const int t = pair_tok[q];
        float* dst = XG + (unsigned long long)q * H;
        for (int c = threadIdx.x; c < H; c += 256) dst[c] = t >= 0 ? X[(unsigned long long)t * ldx + c] : 0.f;
    }
}

__global__ __launch_bounds__(256) void moe_swiglu_kernel(const float* __restrict__ G, const float* __restrict__ Uu,
                                                         int I, const int* __restrict__ totals, int max_pairs,
                                                         float* __restrict__ A) {
    const unsigned long long n = (unsigned long long)(totals[0] < max_pairs ? totals[0] : max_pairs) * I;
    for (unsigned long long i = (unsigned long long)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (unsigned long long)gridDim.x * 256) {
        A[i] = XSwiglu::act(G[i], Uu[i]);  // the same activation as the staged path
    }
}

__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ YD, int H, int k,
                                                          const int* __restrict__ pos, const double* __restrict__ wts,
                                                          float* __restrict__ out, unsigned long long ldo) {
    const int t = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= H) return;
    // every slot's weight, position and value are requested before the sum
    // (independent loads in flight together), then summed in slot order;
    // without a position table (pos null) slot s is pair t * k + s
    double w[kMoeMaxK];
    float y[kMoeMaxK];
#pragma unroll
    for (int s = 0; s < kMoeMaxK; ++s)
        if (s < k) {
            const unsigned long long q = (unsigned long long)t * k + s;
            w[s] = wts[q];
            y[s] = YD[(unsigned long long)(pos ? pos[q] : q) * H + i];
        }
    double acc = 0.0;
#pragma unroll
    for (int s = 0; s < kMoeMaxK; ++s)
        if (s < k && w[s] != 0.0) acc += w[s] * (double)y[s];
    out[(unsigned long long)t * ldo + i] = (float)acc;
}

// ---------------------------------------------------------------- expert matvec

struct MoeMat {
    const uint8_t* W;           // stacked [E][rows][row_bytes]
    unsigned long long slice;   // bytes per expert
    unsigned long long row_bytes;
    const float* X;             // [padded pairs][cols] (XGather: the caller's [batch][ldx] tokens)
    const float* X2;            // XSwiglu: up rows [padded pairs][cols]
    float* Y;                   // [padded pairs][rows]
    int rows, cols, lpr_log2;
};

struct MoeMvArgs {
    MoeMat m[2];
    int nm;
    int tile;                   // rows per item
    const int* chunk_e;         // [chunks] expert of each chunk (its pairs start at chunk * MB)
    const int* totals;          // [1]: chunks
    int E;
    const int* pair_tok;        // XGather: token of each padded pair
    unsigned long long ldx_tokens;
};

// Item i -> matrix (i / per_matrix), chunk, row tile; chunk -> expert by
// binary search over the chunk offsets.
template <int T, int MB, bool AL, bool XL, class XS>
__global__ __launch_bounds__(kMvThreads) void moe_mv_kernel(const MoeMvArgs a) {
    extern __shared__ float smem[];
    const int chunks = a.totals[1];
    int tiles[2];
    long long per_m[2], total = 0;
    for (int j = 0; j < a.nm; ++j) {
        tiles[j] = (a.m[j].rows + a.tile - 1) / a.tile;
        per_m[j] = (long long)chunks * tiles[j];
        total += per_m[j];
    }
    for (long long it = blockIdx.x; it < total; it += gridDim.x) {
        int j = 0;
        long long r = it;
        if (a.nm > 1 && r >= per_m[0]) { r -= per_m[0]; j = 1; }
        const MoeMat& m = a.m[j];
        const int chunk = (int)(r / tiles[j]);
        const int tile = (int)(r - (long long)chunk * tiles[j]);
        const int e = a.chunk_e[chunk];
        const int pair0 = chunk * MB;
        const int row0 = tile * a.tile;
        MvDesc d;
        d.W = m.W + (unsigned long long)e * m.slice + (unsigned long long)row0 * m.row_bytes;
        d.row_bytes = m.row_bytes;
        if constexpr (std::is_same<XS, XGather>::value) {
            d.X = m.X;  // the caller's tokens, gathered through pair_tok
            d.ldx = a.ldx_tokens;
            d.xrow = a.pair_tok + pair0;
        } else {
            d.X = m.X + (unsigned long long)pair0 * m.cols;
            d.ldx = m.cols;
            d.xrow = nullptr;
        }
        d.X2 = std::is_same<XS, XSwiglu>::value ? m.X2 + (unsigned long long)pair0 * m.cols : nullptr;
        d.Y = m.Y + (unsigned long long)pair0 * m.rows + row0;
        d.ldy = m.rows;
        d.rows = m.rows - row0 < a.tile ? m.rows - row0 : a.tile;
        d.cols = m.cols;
        d.lpr_log2 = m.lpr_log2;
        d.wg_begin = 0;
        d.wg_count = 1;
        d.pad = 0;
        d.Bnd = nullptr;
        __syncthreads();  // the previous item's waves are done with LDS
        NoObs ob;
        mv_body<T, MB, 1, AL, XL, false, XS>(d, 0, smem, ob);
    }
}

// ---------------------------------------------------------------- workspace + launch

struct MoeWorkspace {
    size_t bytes = 0;
    void* base = nullptr;
    void* arrive = nullptr;  // arrival counter (zeroed once; every launch leaves it at zero)
    size_t arrive_cap = 0;
};

static thread_local const char* g_moe_err = nullptr;
const char* moe_last_error() { return g_moe_err; }

// Per-device workspace, grown on demand (never during stream capture; a
// replaced block stays allocated for graphs captured before the growth).
static int moe_workspace(size_t bytes, hipStream_t stream, MoeWorkspace** out) {
    static MoeWorkspace ws[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return -4;
    MoeWorkspace& w = ws[dev];
    hipError_t e = hipSuccess;
    if (!w.arrive) e = workspace_grow(&w.arrive, &w.arrive_cap, 256, true, stream);
    if (e == hipSuccess && w.bytes < bytes) e = workspace_grow(&w.base, &w.bytes, bytes, false, stream);
    if (e == hipErrorStreamCaptureUnsupported) {
        g_moe_err = "MoE workspace must grow, which is not allowed during stream capture; run once before capturing";
        return -4;
    }
    if (e != hipSuccess) return -4;
    *out = &w;
    return 0;
}

// carve aligned pieces out of the workspace
struct Carver {
    char* p;
    size_t used = 0;
    template <typename U>
    U* take(size_t n) {
        used = (used + 255) & ~size_t(255);
        U* r = reinterpret_cast<U*>(p ? p + used : nullptr);
        used += n * sizeof(U);
        return r;
    }
};

template <int T, int MB, bool AL, bool XL, class XS>
static hipError_t moe_mv_launch_x(const MoeMvArgs& a, size_t lds, hipStream_t s) {
    const DevInfo& di = dev_info();
    static const int per_cu = [] {
        int v = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, moe_mv_kernel<T, MB, AL, XL, XS>, kMvThreads, 0) != hipSuccess ||
            v < 1)
            v = 1;
        return v;
    }();
    long long pc = per_cu;
    if (lds > 0 && (long long)(di.lds_per_cu / lds) < pc) pc = (long long)(di.lds_per_cu / lds);
    if (pc < 1) pc = 1;
    hipLaunchKernelGGL((moe_mv_kernel<T, MB, AL, XL, XS>), dim3((unsigned)(pc * di.cus)), dim3(kMvThreads), lds, s, a);
    return hipGetLastError();
}

// mode 0: activations already gathered / activated (XDirect); 1: gather the
// caller's tokens (XGather); 2: SwiGLU of the gate and up rows (XSwiglu).
// Modes 1 and 2 need the activations staged in LDS (moe_fused_ok).
template <int T, int MB>
static hipError_t moe_mv_launch_t(MoeMvArgs a, bool al, int mode, hipStream_t s) {
    int max_cols = 0;
    for (int j = 0; j < a.nm; ++j) {
        a.m[j].lpr_log2 = plan_lpr(units_per_row<T>(a.m[j].cols));
        max_cols = a.m[j].cols > max_cols ? a.m[j].cols : max_cols;
    }
    constexpr bool AQ = Geo<T>::bpb % 4 == 0;
    if constexpr (Geo<T>::bs > 1) {
        if (use_xl<T, MB, false>(max_cols)) {
            const size_t lds = lds_bytes<T, MB, false>(max_cols, true);
            if (mode == 1)
                return al && AQ ? moe_mv_launch_x<T, MB, AQ, true, XGather>(a, lds, s)
                                : moe_mv_launch_x<T, MB, false, true, XGather>(a, lds, s);
            if (mode == 2)
                return al && AQ ? moe_mv_launch_x<T, MB, AQ, true, XSwiglu>(a, lds, s)
                                : moe_mv_launch_x<T, MB, false, true, XSwiglu>(a, lds, s);
            return al && AQ ? moe_mv_launch_x<T, MB, AQ, true, XDirect>(a, lds, s)
                            : moe_mv_launch_x<T, MB, false, true, XDirect>(a, lds, s);
        }
    }
    if (mode != 0) return hipErrorInvalidValue;
    const size_t lds = lds_bytes<T, MB, false>(max_cols, false);
    return al && AQ ? moe_mv_launch_x<T, MB, AQ, false, XDirect>(a, lds, s)
                    : moe_mv_launch_x<T, MB, false, false, XDirect>(a, lds, s);
}

static hipError_t moe_mv_launch(int type, int MB, const MoeMvArgs& a, bool al, int mode, hipStream_t s) {
#define PYRITE_CASE(T)                                                 \
    case T:                                                          \
        switch (MB) {                                                \
        case 1: return moe_mv_launch_t<T, 1>(a, al, mode, s);        \
        case 2: return moe_mv_launch_t<T, 2>(a, al, mode, s);        \
        case 4: return moe_mv_launch_t<T, 4>(a, al, mode, s);        \
        default: return moe_mv_launch_t<T, 8>(a, al, mode, s);       \
        }
    switch (type) {
        PYRITE_FOR_EACH_TYPE(PYRITE_CASE)
    default: return hipErrorInvalidValue;
    }
#undef PYRITE_CASE
}

// Whether the fused gather / SwiGLU staging applies: quantized types whose
// staged activations fit the LDS budget.
static bool moe_fused_ok(int type, int MB, size_t cols) {
    const TypeGeo g = type_geo(type);
    if (g.bs == 1) return false;
    const int padi = (type == T_Q6_K || type == T_Q2_K || type == T_Q3_K) ? 128
                     : (type == T_Q4_K || type == T_Q5_K || type == T_IQ4_XS) ? 64 : 32;
    const size_t n16r = ((size_t)MB * (cols / 16) + 3) & ~size_t(3);
    const size_t bytes = n16r * 4 + (size_t)MB * (cols + cols / padi * 4) * 4;
    return bytes <= 65536;
}

// ---------------------------------------------------------------- MFMA experts
// Batches of 32 tokens and more: chunks of kMoeMxTok tokens per expert, and
// per chunk the expert's rows multiplied on the matrix cores
// (v_mfma_f32_16x16x32_f16 with the exact fp16 fragments of mx_traits.h; A
// row 2t + p = fp16 hi (p = 0) / lo (p = 1) part of token t, each token
// scaled by the power of two 2^-e_t that brings its largest finite |x| into
// [2^14, 2^15), the results multiplied back by 2^e_t).
//   moe_gu_kernel     items (chunk, row part): gathers the chunk's tokens as
//                     A fragments in LDS (moe_stage_frags, in the gate/up
//                     format's K-slot map), multiplies the part's gate and
//                     up rows, writes silu(gate) * up and folds the pair's
//                     largest finite |act| (zeroed with the routing plan)
//   moe_dn_kernel     items (chunk, row part): down rows against the chunk's
//                     activations (staged as fragments from act)
// A workgroup takes a contiguous range of items (consecutive items share a
// chunk); its 4 waves walk the part in 128-row tiles (two 16-row MFMA tiles
// per wave) with kMoeMxPF (gate/up) or kMoeDnPF (down) blocks of weights in
// flight per wave.
constexpr int kMoeMxTok = 8;
constexpr int kMoeMxRows = 128;
constexpr int kMoeMxMaxCols = 3072;  // activation fragments of a chunk: cols * 32 bytes of LDS
constexpr int kMoeMxPF = 3;          // blocks per wave in flight (gate/up: its LDS allows two workgroups per CU)
constexpr int kMoeDnPF = 2;          // down: two blocks keep it at 147 VGPRs, three workgroups per CU
                                     // (three blocks: 181 VGPRs, two; 64 tokens: 75 against 78.5 us)
constexpr int kMoeMxMaxPart = 512;   // rows per part at most (results buffered in LDS)

struct MoeMxArgs {
    const uint8_t* W[2];        // stacked [E][rows][row_bytes] (gate, up) or (down)
    unsigned long long slice;   // bytes per expert
    unsigned long long row_bytes;
    int rows, cols;
    int parts, part_rows;       // row parts per chunk; rows per part (a multiple of kMoeMxRows)
    const float* X;             // the caller's tokens [batch][ldx] (moe_gu_kernel)
    unsigned long long ldx;
    const int* pair_tok;        // token of each padded pair, -1 for padding
    int kmode;                  // K-slot map of the gate/up format (mx_kcol)
    const float* act;           // [pairs][cols] silu(gate) * up (moe_dn_kernel)
    unsigned* amax;             // [pairs] largest finite |act| (ordered uint bits)
    float* Y;                   // moe_gu_kernel: act [pairs][rows]; moe_dn_kernel: [pairs][rows]
    const int* chunk_e;         // expert of each chunk (its pairs start at chunk * kMoeMxTok)
    const int* totals;
    int E;
};

// silu(g) * u (pyrite/tensor_ops.py:509-510: v / (1 + exp(-v)) for v > -60, else 0) in fp32
__device__ __forceinline__ float moe_act(float g, float u) {
    return g > -60.f ? g / (1.f + expf(-g)) * u : 0.f;
}

// One workgroup per chunk: the gathered tokens' fragments, exponents, and the
// chunk's act maxima cleared for moe_gu_kernel.
// A chunk's tokens as A fragments in LDS (frag[(step * 4 + group) * 16 +
// 2 t + part], the K-slot map kmode) and each token's exponent (tok_e): the
// largest finite |x| of token t, then x * 2^-e_t split into fp16 hi and lo
// parts.  Padding pairs are zeros.  The whole workgroup calls it; it ends
// with a barrier.
__device__ void moe_stage_frags(const MoeMxArgs& a, int pair0, uint4* frag, int* tok_e, unsigned* tok_max,
                                int* tok_id) {
    const int tid = threadIdx.x;
    if (tid < kMoeMxTok) {
        tok_max[tid] = 0u;
        tok_id[tid] = a.pair_tok[pair0 + tid];
    }
    __syncthreads();
    // item idx = (step st, K-slot group gg, token t): 8 columns of token t;
    // each thread takes items tid + 256 j, 8 at a time, every load of a batch
    // issued before any is used
    constexpr int kB = 8;
    const int steps = a.cols >> 5, count = steps * 4 * kMoeMxTok;
    auto load_batch = [&](int base, float (&v)[kB][8]) {
        float4 q[kB][2];
#pragma unroll
        for (int j = 0; j < kB; ++j) {
            const int idx = base + tid + 256 * j;
            const int t = idx % kMoeMxTok, gg = (idx / kMoeMxTok) & 3, st = idx / (4 * kMoeMxTok);
            const int tok = idx < count ? tok_id[t] : -1;
            // padding pairs and items past the end read token 0's first columns (not used)
            const float* p = a.X + (tok < 0 ? 0ull : (unsigned long long)tok * a.ldx + mx_kcol(a.kmode, st, gg));
            q[j][0] = ld_x4(p);
            q[j][1] = ld_x4(p + 4);
        }
#pragma unroll
        for (int j = 0; j < kB; ++j) {
            const int idx = base + tid + 256 * j;
            const bool use = idx < count && tok_id[idx % kMoeMxTok] >= 0;
            const float4 x0 = q[j][0], x1 = q[j][1];
            const float w[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) v[j][i] = use ? w[i] : 0.f;
        }
    };
    for (int base = 0; base < count; base += 256 * kB) {
        float v[kB][8];
        load_batch(base, v);
#pragma unroll
        for (int j = 0; j < kB; ++j) {
            const float mx = finite_max8(v[j]);
            if (mx > 0.f) atomicMax(&tok_max[(base + tid + 256 * j) % kMoeMxTok], __float_as_uint(mx));
        }
    }
    __syncthreads();
    for (int base = 0; base < count; base += 256 * kB) {
        float v[kB][8];
        load_batch(base, v);
#pragma unroll
        for (int j = 0; j < kB; ++j) {
            const int idx = base + tid + 256 * j;
            if (idx >= count) continue;
            const int t = idx % kMoeMxTok, gg = (idx / kMoeMxTok) & 3, st = idx / (4 * kMoeMxTok);
            uint4 h, l;
            split8(v[j], norm_exp(__uint_as_float(tok_max[t])), h, l);
            frag[(st * 4 + gg) * 16 + 2 * t] = h;
            frag[(st * 4 + gg) * 16 + 2 * t + 1] = l;
        }
    }
    if (tid < kMoeMxTok) tok_e[tid] = norm_exp(__uint_as_float(tok_max[tid]));
    __syncthreads();
}

// The block sequence of one wave over a row part of one or two matrices that
// share the staged fragments: q runs over (tile, matrix, block); raw[p] holds
// block q0 + p.  acc[j] collects matrix j of the current tile; done(tile)
// is called after the last block of each tile.
template <int T, bool AL, int NM, int PF, class Done>
__device__ __forceinline__ void moe_mx_walk(const MoeMxArgs& a, int e, int row_lo, int row_hi, const uint4* frag,
                                            f4v (&acc)[NM][2], Done done) {
    using F = Mx<T>;
    // unaligned 256-column blocks (Q6_K rows: 210 bytes) as loads at the
    // spans' own byte addresses: about half the load instructions of dword
    // loads realigned in registers (the cache lines touched stay the same)
    constexpr bool UA = !AL && F::BS == 256;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, n = lane & 15;
    const int nblk = a.cols / F::BS;
    const int ntile = (row_hi - row_lo + kMoeMxRows - 1) / kMoeMxRows;
    const int per_tile = NM * nblk;
    const int nq = ntile * per_tile;
    auto load_q = [&](int q, typename F::Raw& r0, typename F::Raw& r1) {
        const int qq = q < nq ? q : nq - 1;
        const int tile = qq / per_tile, rem = qq - tile * per_tile;
        const int j = rem / nblk, b = rem - j * nblk;
        const uint8_t* Wm = a.W[j] + (unsigned long long)e * a.slice;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            long long r = (long long)row_lo + (long long)tile * kMoeMxRows + 32 * w + 16 * h + n;
            if (r >= a.rows) r = a.rows - 1;
            F::template load<AL, false, UA>(Wm + (unsigned long long)r * a.row_bytes + (size_t)b * F::BPB, g,
                                            h ? r1 : r0);
        }
    };
    typename F::Raw ra[PF], rb[PF];
#pragma unroll
    for (int p = 0; p < PF; ++p) {
        load_q(p, ra[p], rb[p]);
        asm volatile("" ::: "memory");
    }
    for (int q0 = 0; q0 < nq; q0 += PF) {
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const int q = q0 + p;
            if (q < nq) {
                const int tile = q / per_tile, rem = q - tile * per_tile;
                const int j = rem / nblk, b = rem - j * nblk;
                f4v D[2][F::NACC];
#pragma unroll
                for (int c = 0; c < F::NACC; ++c) D[0][c] = D[1][c] = f4v{0.f, 0.f, 0.f, 0.f};
                const uint4* fb = frag + (size_t)b * F::STEPS * 4 * 16;
                typename MxPreOf<F>::type pa, pb;
                mx_prep<F>(ra[p], g, pa);
                mx_prep<F>(rb[p], g, pb);
#pragma unroll
                for (int st = 0; st < F::STEPS; ++st) {
                    const uint4 av = fb[(st * 4 + g) * 16 + n];
                    const uint32_t aw[4] = {av.x, av.y, av.z, av.w};
                    const h8v A = __builtin_bit_cast(h8v, aw);
                    uint32_t ba[F::NACC][4], bb[F::NACC][4];
                    mx_frag<F>(ra[p], pa, st, g, ba);
                    mx_frag<F>(rb[p], pb, st, g, bb);
#pragma unroll
                    for (int c = 0; c < F::NACC; ++c) {
                        D[0][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(h8v, ba[c]), D[0][c], 0, 0, 0);
                        D[1][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(h8v, bb[c]), D[1][c], 0, 0, 0);
                    }
                }
                // j is wave-uniform: select the accumulator pair without dynamic indexing
#pragma unroll
                for (int jj = 0; jj < NM; ++jj) {
                    if (jj == j) {
                        F::epi(ra[p], D[0], acc[jj][0]);
                        F::epi(rb[p], D[1], acc[jj][1]);
                    }
                }
                if (rem == per_tile - 1) done(tile);
            }
            load_q(q + PF, ra[p], rb[p]);
            // keep the refills in slot order: loads complete in order, so a
            // slot refilled after a later one would make its wait cover both
            asm volatile("" ::: "memory");
        }
    }
}

// Contiguous item range of this workgroup over `total` items.
__device__ __forceinline__ void moe_item_range(long long total, long long& it0, long long& it1) {
    const long long per = (total + gridDim.x - 1) / gridDim.x;
    it0 = (long long)blockIdx.x * per;
    it1 = it0 + per < total ? it0 + per : total;
}

// Results of a part wait in LDS ([tile row][token], after the fragments)
// and are stored after the walk: global stores inside the walk would share
// the load counter and cut the weight pipeline short.
template <int T, bool AL>
__global__ __launch_bounds__(256, 2) void moe_gu_kernel(const MoeMxArgs a) {
    extern __shared__ float smem[];
    uint4* frag = reinterpret_cast<uint4*>(smem);
    float* res = smem + (size_t)a.cols * 8;  // [part_rows][kMoeMxTok]
    __shared__ int tok_e[kMoeMxTok];
    __shared__ unsigned tok_max[kMoeMxTok];
    __shared__ int tok_id[kMoeMxTok];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, n = lane & 15;
    long long it0, it1;
    moe_item_range((long long)a.totals[1] * a.parts, it0, it1);
    int staged = -1;
    for (long long it = it0; it < it1; ++it) {
        const int chunk = (int)(it / a.parts), part = (int)(it - (long long)chunk * a.parts);
        const int e = a.chunk_e[chunk];
        const int pair0 = chunk * kMoeMxTok;
        __syncthreads();  // the previous item's waves are done with the fragments and results
        if (chunk != staged) {
            moe_stage_frags(a, pair0, frag, tok_e, tok_max, tok_id);
            staged = chunk;
        }
        const int row_lo = part * a.part_rows;
        const int row_hi = row_lo + a.part_rows < a.rows ? row_lo + a.part_rows : a.rows;
        const int te0 = tok_e[2 * g], te1 = tok_e[2 * g + 1];
        f4v acc[2][2];
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[j][0] = acc[j][1] = f4v{0.f, 0.f, 0.f, 0.f};
        moe_mx_walk<T, AL, 2, kMoeMxPF>(a, e, row_lo, row_hi, frag, acc, [&](int tile) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int lr = tile * kMoeMxRows + 32 * w + 16 * h + n;  // row within the part
                const float g0 = __builtin_amdgcn_ldexpf(acc[0][h][0] + acc[0][h][1], te0);
                const float g1 = __builtin_amdgcn_ldexpf(acc[0][h][2] + acc[0][h][3], te1);
                const float u0 = __builtin_amdgcn_ldexpf(acc[1][h][0] + acc[1][h][1], te0);
                const float u1 = __builtin_amdgcn_ldexpf(acc[1][h][2] + acc[1][h][3], te1);
                res[lr * kMoeMxTok + 2 * g] = moe_act(g0, u0);
                res[lr * kMoeMxTok + 2 * g + 1] = moe_act(g1, u1);
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[j][h] = f4v{0.f, 0.f, 0.f, 0.f};
            }
        });
        __syncthreads();
        // store the part's act rows and fold their largest finite |act| per token
        const int nr = row_hi - row_lo;
        const int t = tid & (kMoeMxTok - 1);
        unsigned mx = 0u;
        for (int i = tid; i < nr * kMoeMxTok; i += 256) {  // i % kMoeMxTok == t
            const int lr = i / kMoeMxTok;
            const float v = res[i];
            a.Y[(unsigned long long)(pair0 + t) * a.rows + row_lo + lr] = v;
            const float f = fabsf(v);
            if (f <= 3.402823466e38f) mx = max(mx, __float_as_uint(f));
        }
        if (mx) atomicMax(&a.amax[pair0 + t], mx);
    }
}

template <int T, bool AL>
__global__ __launch_bounds__(256, 3) void moe_dn_kernel(const MoeMxArgs a) {
    extern __shared__ float smem[];
    uint4* frag = reinterpret_cast<uint4*>(smem);
    float* res = smem + (size_t)a.cols * 8;  // [part_rows][kMoeMxTok]
    __shared__ int tok_e[kMoeMxTok];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, n = lane & 15;
    const int steps = a.cols >> 5;
    long long it0, it1;
    moe_item_range((long long)a.totals[1] * a.parts, it0, it1);
    int staged = -1;
    for (long long it = it0; it < it1; ++it) {
        const int chunk = (int)(it / a.parts), part = (int)(it - (long long)chunk * a.parts);
        const int e = a.chunk_e[chunk];
        const int pair0 = chunk * kMoeMxTok;
        __syncthreads();  // the previous item's waves are done with the fragments and results
        if (chunk != staged) {
            const int count = steps * 4 * kMoeMxTok;
            for (int idx = tid; idx < count; idx += 256) {
                const int t = idx % kMoeMxTok, gg = (idx / kMoeMxTok) & 3, st = idx / (4 * kMoeMxTok);
                const float* p = a.act + (unsigned long long)(pair0 + t) * a.cols + mx_col<Mx<T>>(st, gg);
                const float4 x0 = ld_x4(p), x1 = ld_x4(p + 4);
                const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                uint4 h, l;
                split8(v, norm_exp(__uint_as_float(a.amax[pair0 + t])), h, l);
                frag[(st * 4 + gg) * 16 + 2 * t] = h;
                frag[(st * 4 + gg) * 16 + 2 * t + 1] = l;
            }
            if (tid < kMoeMxTok) tok_e[tid] = norm_exp(__uint_as_float(a.amax[pair0 + tid]));
            __syncthreads();
            staged = chunk;
        }
        const int row_lo = part * a.part_rows;
        const int row_hi = row_lo + a.part_rows < a.rows ? row_lo + a.part_rows : a.rows;
        const int te0 = tok_e[2 * g], te1 = tok_e[2 * g + 1];
        f4v acc[1][2];
        acc[0][0] = acc[0][1] = f4v{0.f, 0.f, 0.f, 0.f};
        moe_mx_walk<T, AL, 1, kMoeDnPF>(a, e, row_lo, row_hi, frag, acc, [&](int tile) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int lr = tile * kMoeMxRows + 32 * w + 16 * h + n;
                res[lr * kMoeMxTok + 2 * g] = __builtin_amdgcn_ldexpf(acc[0][h][0] + acc[0][h][1], te0);
                res[lr * kMoeMxTok + 2 * g + 1] = __builtin_amdgcn_ldexpf(acc[0][h][2] + acc[0][h][3], te1);
                acc[0][h] = f4v{0.f, 0.f, 0.f, 0.f};
            }
        });
        __syncthreads();
        const int nr = row_hi - row_lo;
        for (int i = tid; i < nr * kMoeMxTok; i += 256) {
            const int lr = i / kMoeMxTok, t = i - lr * kMoeMxTok;
            a.Y[(unsigned long long)(pair0 + t) * a.rows + row_lo + lr] = res[i];
        }
    }
}

// gate/up (gu) or down launch of one block format; grid workgroups.
template <int T, bool AL>
static hipError_t moe_mx_launch_t(const MoeMxArgs& a, bool gu, int grid, hipStream_t s) {
    const size_t lds = (size_t)a.cols * 32 + (size_t)a.part_rows * kMoeMxTok * 4;
    const void* fn = gu ? reinterpret_cast<const void*>(&moe_gu_kernel<T, AL>)
                        : reinterpret_cast<const void*>(&moe_dn_kernel<T, AL>);
    static const hipError_t attr_gu = hipFuncSetAttribute(reinterpret_cast<const void*>(&moe_gu_kernel<T, AL>),
                                                          hipFuncAttributeMaxDynamicSharedMemorySize,
                                                          kMoeMxMaxCols * 32 + kMoeMxMaxPart * kMoeMxTok * 4);
    static const hipError_t attr_dn = hipFuncSetAttribute(reinterpret_cast<const void*>(&moe_dn_kernel<T, AL>),
                                                          hipFuncAttributeMaxDynamicSharedMemorySize,
                                                          kMoeMxMaxCols * 32 + kMoeMxMaxPart * kMoeMxTok * 4);
    if (attr_gu != hipSuccess) return attr_gu;
    if (attr_dn != hipSuccess) return attr_dn;
    (void)fn;
    if (gu)
        hipLaunchKernelGGL((moe_gu_kernel<T, AL>), dim3((unsigned)grid), dim3(256), lds, s, a);
    else
        hipLaunchKernelGGL((moe_dn_kernel<T, AL>), dim3((unsigned)grid), dim3(256), lds, s, a);
    return hipGetLastError();
}

// K-slot map of a block format's MFMA fragments (mx_kcol)
static int moe_kmode(int type) {
#define PYRITE_CASE(T) \
    case T: return MxKMode<Mx<T>>::value;
    switch (type) {
        PYRITE_CASE(T_Q4_0) PYRITE_CASE(T_Q4_1) PYRITE_CASE(T_Q5_0) PYRITE_CASE(T_Q5_1)
        PYRITE_CASE(T_Q8_0) PYRITE_CASE(T_Q8_1) PYRITE_CASE(T_Q2_K) PYRITE_CASE(T_Q3_K)
        PYRITE_CASE(T_Q4_K) PYRITE_CASE(T_Q5_K) PYRITE_CASE(T_Q6_K) PYRITE_CASE(T_IQ4_NL)
        PYRITE_CASE(T_IQ4_XS)
    default: return 0;
    }
#undef PYRITE_CASE
}

static hipError_t moe_mx_launch(int type, const MoeMxArgs& a, bool gu, bool al, int grid, hipStream_t s) {
#define PYRITE_CASE(T)                                                                                     \
    case T:                                                                                              \
        return (al && Geo<T>::bpb % 4 == 0) ? moe_mx_launch_t<T, (Geo<T>::bpb % 4 == 0)>(a, gu, grid, s) \
                                            : moe_mx_launch_t<T, false>(a, gu, grid, s);
    switch (type) {
        PYRITE_CASE(T_Q4_0) PYRITE_CASE(T_Q4_1) PYRITE_CASE(T_Q5_0) PYRITE_CASE(T_Q5_1)
        PYRITE_CASE(T_Q8_0) PYRITE_CASE(T_Q8_1) PYRITE_CASE(T_Q2_K) PYRITE_CASE(T_Q3_K)
        PYRITE_CASE(T_Q4_K) PYRITE_CASE(T_Q5_K) PYRITE_CASE(T_Q6_K) PYRITE_CASE(T_IQ4_NL)
        PYRITE_CASE(T_IQ4_XS)
    default: return hipErrorInvalidValue;
    }
#undef PYRITE_CASE
}

int moe_ffn_launch(const MoeLayer& L, const float* X, size_t ldx, float* out, size_t ldo, int* ids_out,
                   float* wts_out, size_t batch, hipStream_t stream) {
    g_moe_err = nullptr;
    const TypeGeo gr = type_geo(L.router_type), gg = type_geo(L.gate_type), gu = type_geo(L.up_type),
                  gd = type_geo(L.down_type);
    if (!gr.valid || !gg.valid || !gu.valid || !gd.valid) return -1;
    const size_t E = L.n_experts, H = L.hidden, I = L.inter, K = L.k;
    if (E == 0 || H == 0 || I == 0 || K == 0 || K > E || E > (size_t)kMoeMaxE || K > (size_t)kMoeMaxK) return -2;
    if (batch == 0 || batch > 4096 || H > 65536 || I > 65536) return -2;
    if (H % gr.bs || H % gg.bs || H % gu.bs || I % gd.bs) return -2;
    const size_t rr = H / gr.bs * gr.bpb, gs = I * (H / gg.bs * gg.bpb), us = I * (H / gu.bs * gu.bpb),
                 ds = H * (I / gd.bs * gd.bpb);
    if (!L.router || !L.gate || !L.up || !L.down || !X || !out) return -3;
    if (L.router_len != E * rr || L.gate_len != E * gs || L.up_len != E * us || L.down_len != E * ds) return -3;
    if (ldx < H || ldo < H || (reinterpret_cast<uintptr_t>(X) & 3u)) return -3;
    // From 32 tokens on (about 2 per expert and more), the block formats run
    // their experts on the matrix cores in chunks of kMoeMxTok tokens;
    // otherwise the VALU expert kernels (measured faster at 8 tokens).
    const bool x16 = ((reinterpret_cast<uintptr_t>(X) & 15u) == 0) && (ldx % 4 == 0);
    const bool mfma = batch >= 32 && x16 && L.gate_type == L.up_type && mx_type_supported(L.gate_type) &&
                      mx_type_supported(L.down_type) && H <= (size_t)kMoeMxMaxCols && I <= (size_t)kMoeMxMaxCols;
    // chunk width: tokens per expert chunk (weights are read once per chunk)
    const int MB = mfma ? kMoeMxTok : batch == 1 ? 1 : batch <= 16 ? 2 : 4;
    const size_t max_pairs = batch * K + E * (size_t)(MB - 1);

    Carver c{nullptr};
    const size_t max_chunks = mfma ? max_pairs / kMoeMxTok : 0;
    unsigned* amax = nullptr;
    auto layout = [&](Carver& cv, double** logits, double** mags, int** ids, double** wts, MoePlan* p, float** xg,
                      float** g, float** u, float** act, float** yd) {
        amax = cv.take<unsigned>(mfma ? max_pairs : 0);
        *logits = cv.take<double>(batch * E);
        *mags = cv.take<double>(batch * E);
        *ids = cv.take<int>(batch * K);
        *wts = cv.take<double>(batch * K);
        p->pair_tok = cv.take<int>(max_pairs);
        p->pos = cv.take<int>(batch * K);
        p->totals = cv.take<int>(2);
        p->chunk_e = cv.take<int>(max_pairs);
        *xg = cv.take<float>(max_pairs * H);
        *g = cv.take<float>(max_pairs * I);
        *u = cv.take<float>(max_pairs * I);
        *act = cv.take<float>(max_pairs * I);
        *yd = cv.take<float>(max_pairs * H);
    };
    double *logits, *mags, *wts;
    int* ids;
    MoePlan plan;
    float *xg, *g, *u, *act, *yd;
    layout(c, &logits, &mags, &ids, &wts, &plan, &xg, &g, &u, &act, &yd);
    MoeWorkspace* ws = nullptr;
    if (const int rc = moe_workspace(c.used + 256, stream, &ws)) return rc;
    Carver cw{static_cast<char*>(ws->base)};
    layout(cw, &logits, &mags, &ids, &wts, &plan, &xg, &g, &u, &act, &yd);

    // 1. router logits, 2. route + plan (one launch for small batches)
    MoeRouteArgs ra;
    ra.type = L.router_type;
    ra.W = static_cast<const uint8_t*>(L.router);
    ra.row_bytes = rr;
    ra.E = (int)E;
    ra.H = (int)H;
    ra.bs = gr.bs;
    ra.bpb = gr.bpb;
    ra.k = (int)K;
    ra.MB = MB;
    ra.norm_topk = L.norm_topk_prob;
    ra.scale = L.scale;
    {
        // tree sums of <= H/64 + 6 adds per lane path, the reference's sequential sum of H terms
        const double u64 = 1.0 / 9007199254740992.0;
        const double d1 = (double)H / 64 + 8, d2 = (double)H;
        ra.gamma = (d1 * u64 / (1 - d1 * u64) + d2 * u64 / (1 - d2 * u64)) * (1 + 1.0 / 1024);
    }
    ra.X = X;
    ra.ldx = ldx;
    ra.logits = logits;
    ra.mags = mags;
    ra.ids = ids;
    ra.wts = wts;
    ra.wts_out = wts_out;
    ra.ids_out = ids_out;
    ra.batch = (int)batch;
    ra.arrive = static_cast<unsigned int*>(ws->arrive);
    plan.amax = mfma ? amax : nullptr;  // zeroed by the plan only for the matrix-core experts
    ra.plan = plan;
    if (batch <= kMoeFusedRouteBatch) {
        // counters 1 .. batch of the zeroed arrival block (0 is the token counter)
        hipLaunchKernelGGL(moe_router_route_kernel, dim3((unsigned)((E + 3) / 4), (unsigned)batch), dim3(256), 0,
                           stream, ra, static_cast<unsigned int*>(ws->arrive) + 1);
    } else {
        hipLaunchKernelGGL(moe_router_kernel, dim3((unsigned)((E + 3) / 4), (unsigned)((batch + kMoeRouterTok - 1) / kMoeRouterTok)),
                           dim3(256), 0, stream, L.router_type, static_cast<const uint8_t*>(L.router),
                           (unsigned long long)rr, (int)E, (int)H, gr.bs, gr.bpb, X, (unsigned long long)ldx,
                           (int)batch, logits, mags);
        if (hipGetLastError() != hipSuccess) return -4;
        hipLaunchKernelGGL(moe_route_kernel, dim3((unsigned)batch), dim3(256), 0, stream, ra);
    }
    if (hipGetLastError() != hipSuccess) return -4;
    if (mfma) {
        // 3. fragments of each chunk's tokens; 4. gate and up with silu(gate) * up;
        // 5. down; 6. combine.  Contiguous item ranges over at least twice
        // the CUs (item_grid), row parts so that about one item per workgroup
        // exists at the likely chunk count (one per distinct expert; measured
        // on MI355X, fewer and larger items beat two or more per workgroup).
        const int grid = 2 * dev_info().cus;
        const size_t est_chunks = E < batch * K ? E : batch * K;
        MoeMxArgs xa;
        xa.chunk_e = plan.chunk_e;
        xa.totals = plan.totals;
        xa.E = (int)E;
        xa.X = X;
        xa.ldx = ldx;
        xa.pair_tok = plan.pair_tok;
        xa.kmode = moe_kmode(L.gate_type);
        xa.amax = amax;
        auto set_parts = [&](size_t rows) {
            size_t parts = ((size_t)grid + est_chunks - 1) / est_chunks;
            size_t pr = (rows + parts - 1) / parts;
            pr = (pr + kMoeMxRows - 1) / kMoeMxRows * kMoeMxRows;
            if (pr > (size_t)kMoeMxMaxPart) pr = kMoeMxMaxPart;
            xa.part_rows = (int)pr;
            xa.parts = (int)((rows + pr - 1) / pr);
        };
        // One workgroup per item wherever the plan's largest chunk count
        // allows it: with the grid at 2 x CUs, a few chunks more than
        // estimated gave every workgroup two items (down at 64 tokens: 129
        // chunks, 516 items on 512 workgroups, 145 us instead of 80).
        // Workgroups past the actual items return at once.
        auto item_grid = [&]() {
            const size_t most = max_chunks * (size_t)xa.parts, cap = 4 * (size_t)dev_info().cus;
            const size_t g2 = most < cap ? most : cap;
            return (int)(g2 > (size_t)grid ? g2 : (size_t)grid);
        };
        xa.W[0] = static_cast<const uint8_t*>(L.gate);
        xa.W[1] = static_cast<const uint8_t*>(L.up);
        xa.slice = gs;
        xa.row_bytes = H / gg.bs * gg.bpb;
        xa.rows = (int)I;
        xa.cols = (int)H;
        xa.act = nullptr;
        xa.Y = act;
        set_parts(I);
        const bool al_gu2 = ((reinterpret_cast<uintptr_t>(L.gate) | reinterpret_cast<uintptr_t>(L.up)) & 3u) == 0;
        if (moe_mx_launch(L.gate_type, xa, true, al_gu2, item_grid(), stream) != hipSuccess) return -4;
        xa.W[0] = xa.W[1] = static_cast<const uint8_t*>(L.down);
        xa.slice = ds;
        xa.row_bytes = I / gd.bs * gd.bpb;
        xa.rows = (int)H;
        xa.cols = (int)I;
        xa.act = act;
        xa.Y = yd;
        set_parts(H);
        if (moe_mx_launch(L.down_type, xa, false, (reinterpret_cast<uintptr_t>(L.down) & 3u) == 0, item_grid(),
                          stream) != hipSuccess)
            return -4;
        hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((H + 255) / 256), (unsigned)batch), dim3(256), 0,
                           stream, yd, (int)H, (int)K, plan.pos, wts, out, (unsigned long long)ldo);
        return hipGetLastError() == hipSuccess ? 0 : -4;
    }
    // 3. gather (unless the gate/up launch gathers while staging)
    const bool fuse_in = x16 && moe_fused_ok(L.gate_type, MB, H) && moe_fused_ok(L.up_type, MB, H);
    const bool fuse_act = moe_fused_ok(L.down_type, MB, I);
    if (!fuse_in) {
        const unsigned gblocks = (unsigned)(max_pairs < 4096 ? max_pairs : 4096);
        hipLaunchKernelGGL(moe_gather_kernel, dim3(gblocks), dim3(256), 0, stream, X, (unsigned long long)ldx,
                           (int)H, plan.pair_tok, plan.totals, (int)max_pairs, xg);
        if (hipGetLastError() != hipSuccess) return -4;
    }
    // 4. gate and up
    auto tile_for = [&](size_t rows) {
        // aim for ~512 items per launch at the worst-case chunk count: each
        // item stages its chunk's activations, so larger items amortise that
        // (measured on MI355X: 512 beats 256-2048 at batch 1 and 8)
        const size_t chunks = (batch * K + MB - 1) / MB;
        size_t t = 16;
        while (t < 128 && chunks * ((rows + t - 1) / t) > 512) t *= 2;
        return (int)t;
    };
    const bool al_gu = ((reinterpret_cast<uintptr_t>(L.gate) | reinterpret_cast<uintptr_t>(L.up)) & 3u) == 0;
    MoeMvArgs ma;
    ma.chunk_e = plan.chunk_e;
    ma.totals = plan.totals;
    ma.E = (int)E;
    ma.pair_tok = plan.pair_tok;
    ma.ldx_tokens = ldx;
    auto mat = [&](const void* W, size_t slice, const TypeGeo& tg, const float* Xs, const float* X2s, float* Ys,
                   size_t rows, size_t cols) {
        MoeMat m;
        m.W = static_cast<const uint8_t*>(W);
        m.slice = slice;
        m.row_bytes = cols / tg.bs * tg.bpb;
        m.X = Xs;
        m.X2 = X2s;
        m.Y = Ys;
        m.rows = (int)rows;
        m.cols = (int)cols;
        m.lpr_log2 = 0;
        return m;
    };
    const float* xin = fuse_in ? X : xg;
    const int mode_in = fuse_in ? 1 : 0;
    ma.tile = tile_for(I);
    if (L.gate_type == L.up_type) {
        ma.nm = 2;
        ma.m[0] = mat(L.gate, gs, gg, xin, nullptr, g, I, H);
        ma.m[1] = mat(L.up, us, gu, xin, nullptr, u, I, H);
        if (moe_mv_launch(L.gate_type, MB, ma, al_gu, mode_in, stream) != hipSuccess) return -4;
    } else {
        ma.nm = 1;
        ma.m[0] = mat(L.gate, gs, gg, xin, nullptr, g, I, H);
        if (moe_mv_launch(L.gate_type, MB, ma, al_gu, mode_in, stream) != hipSuccess) return -4;
        ma.m[0] = mat(L.up, us, gu, xin, nullptr, u, I, H);
        if (moe_mv_launch(L.up_type, MB, ma, al_gu, mode_in, stream) != hipSuccess) return -4;
    }
    // 5. SwiGLU (unless the down launch applies it while staging)
    if (!fuse_act) {
        hipLaunchKernelGGL(moe_swiglu_kernel, dim3(1024), dim3(256), 0, stream, g, u, (int)I, plan.totals,
                           (int)max_pairs, act);
        if (hipGetLastError() != hipSuccess) return -4;
    }
    const bool al_dn = (reinterpret_cast<uintptr_t>(L.down) & 3u) == 0;
    // 6. down
    ma.nm = 1;
    ma.tile = tile_for(H);
    ma.m[0] = fuse_act ? mat(L.down, ds, gd, g, u, yd, H, I) : mat(L.down, ds, gd, act, nullptr, yd, H, I);
    if (moe_mv_launch(L.down_type, MB, ma, al_dn, fuse_act ? 2 : 0, stream) != hipSuccess)
        return -4;
    // 7. combine (one token: pairs in slot order)
    hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((H + 255) / 256), (unsigned)batch), dim3(256), 0, stream,
                       yd, (int)H, (int)K, batch == 1 && MB == 1 ? nullptr : plan.pos, wts, out,
                       (unsigned long long)ldo);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace pyrite
