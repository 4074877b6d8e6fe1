// MFMA dequant-matvec for the GGML block formats (batch 1..8), gfx950.
// Fragment construction and block formats: mx_traits.h.
//
// Schedule: a workgroup (4 waves) owns a 32-row tile (two 16-row MFMA column
// tiles sharing the A fragment); its waves split the row's blocks round-robin
// and the 4 partial results are summed in LDS in a fixed order, so results are
// deterministic.  Workgroups loop over tiles.  The A fragments of the whole
// row (or of a K chunk when they exceed the LDS budget) are built once per
// workgroup in LDS, compacted to the token-parts in use (MB = 2 * tokens).
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "dispatch.h"
#include "mx_traits.h"

namespace pyrite {

// ---------------------------------------------------------------- kernel

struct MxDesc {
    const uint8_t* W;
    unsigned long long row_bytes;
    const float* X;
    unsigned long long ldx;
    float* Y;
    unsigned long long ldy;
    float* part;          // split-K partial sums [ksplit][tiles][32 rows][8 tokens]
    unsigned* counters;   // per-tile arrival counters; zero between launches
    int rows;
    int cols;
    int batch;            // activation vectors (<= 8)
    int ksplit;           // K parts (workgroup tasks per 32-row tile)
    int kpart_steps;      // 32-column steps per K part (a multiple of the block's steps)
    int tiles;            // ceil(rows / 32)
    int task_begin;       // first task of this matrix; tasks = ksplit * tiles
    int pad;
};

constexpr int kMxMaxGroup = 16;
struct MxGroup {
    int n;
    int total_tasks;
    MxDesc d[kMxMaxGroup];
};

constexpr int kRedBytes = 4 * 2 * 64 * 4 * 4;  // [wave][row tile][lane][4] floats
constexpr int kPF = 2;                          // blocks per wave loaded ahead of their use

// Barrier for LDS hand-offs only: waits for this wave's LDS traffic, not for
// its outstanding global loads (which may be blocks prefetched for later).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Largest finite |x| per token over steps [s0, s1) into tok_max (ordered
// uint bits of a non-negative float; tok_max starts at zero).
template <int MB>
__device__ __forceinline__ void x_max(const MxDesc& d, int s0, int s1, int tid, unsigned* tok_max) {
    constexpr int NT = MB / 2;
    const int count = (s1 - s0) * 4 * NT;
    for (int idx = tid; idx < count; idx += 256) {
        const int s = s0 + idx / (4 * NT), rem = idx % (4 * NT);
        const int gg = rem / NT, t = rem % NT;
        if (t >= d.batch) continue;
        const float* xp = d.X + t * d.ldx + 32 * s + 8 * gg;
        const float4 a = ld_x4(xp), b = ld_x4(xp + 4);
        const float xs[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        const float mx = finite_max8(xs);
        if (mx > 0.f) atomicMax(&tok_max[t], __float_as_uint(mx));
    }
}

// A fragments of steps [s0, s1) into LDS, laid out [step][group][MB] x 16 bytes
// (8 halves: hi or lo parts of x[t][32 s + 8 group + i] * 2^-e_t, row 2t + p),
// e_t the token's normalising exponent from tok_max.
template <int MB>
__device__ __forceinline__ void stage_x(const MxDesc& d, int s0, int s1, int tid, const unsigned* tok_max,
                                        uint4* frag) {
    constexpr int NT = MB / 2;
    const int count = (s1 - s0) * 4 * NT;
    for (int idx = tid; idx < count; idx += 256) {
        const int s = idx / (4 * NT), rem = idx % (4 * NT);
        const int gg = rem / NT, t = rem % NT;
        uint4 hi = make_uint4(0u, 0u, 0u, 0u), lo = hi;
        if (t < d.batch) {
            const float* xp = d.X + t * d.ldx + 32 * (s0 + s) + 8 * gg;
            const float4 a = ld_x4(xp), b = ld_x4(xp + 4);
            const float xs[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            split8(xs, norm_exp(__uint_as_float(tok_max[t])), hi, lo);
        }
        uint4* f = frag + (s * 4 + gg) * MB + 2 * t;
        f[0] = hi;
        f[1] = lo;
    }
}

// One block of two 16-row column tiles: B fragments, MFMAs, block epilogue.
template <int T, int MB>
__device__ __forceinline__ void mx_block(const typename Mx<T>::Raw& ra, const typename Mx<T>::Raw& rb,
                                         const uint4* fblk, int g, int n, f4v (&acc)[2]) {
    using F = Mx<T>;
    f4v Da[F::NACC], Db[F::NACC];
#pragma unroll
    for (int p = 0; p < F::NACC; ++p) {
        Da[p] = f4v{0.f, 0.f, 0.f, 0.f};
        Db[p] = f4v{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int st = 0; st < F::STEPS; ++st) {
        uint4 av = make_uint4(0u, 0u, 0u, 0u);
        if (n < MB) av = fblk[(st * 4 + g) * MB + n];
        const uint32_t aw[4] = {av.x, av.y, av.z, av.w};
        const h8v a = __builtin_bit_cast(h8v, aw);
        uint32_t ba[F::NACC][4], bb[F::NACC][4];
        F::frag(ra, st, g, ba);
        F::frag(rb, st, g, bb);
#pragma unroll
        for (int p = 0; p < F::NACC; ++p) {
            Da[p] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(h8v, ba[p]), Da[p], 0, 0, 0);
            Db[p] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(h8v, bb[p]), Db[p], 0, 0, 0);
        }
    }
    F::epi(ra, Da, acc[0]);
    F::epi(rb, Db, acc[1]);
}

template <int T, int MB, bool AL>
__global__ __launch_bounds__(256) void mx_kernel(const MxGroup grp) {
    using F = Mx<T>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    float* red = reinterpret_cast<float*>(smem);
    uint4* frag = reinterpret_cast<uint4*>(smem + kRedBytes);
    __shared__ unsigned tok_max[8];
    __shared__ int last_flag;

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, n = lane & 15;
    int staged_mi = -1, staged_kp = -1;

    for (int task = blockIdx.x; task < grp.total_tasks; task += gridDim.x) {
        int mi = 0;
        while (mi + 1 < grp.n && task >= grp.d[mi + 1].task_begin) ++mi;
        const MxDesc& d = grp.d[mi];
        const int local = task - d.task_begin;
        const int kp = local / d.tiles, tile = local - kp * d.tiles;
        const int rows = d.rows;
        const int nblk = d.cols / F::BS;
        const int kps = d.kpart_steps;
        const int s0 = kp * kps;
        const int s1 = (s0 + kps < (d.cols >> 5)) ? s0 + kps : (d.cols >> 5);
        const int kb0 = s0 / F::STEPS;
        const int kb1 = (s1 / F::STEPS < nblk) ? s1 / F::STEPS : nblk;

        const long long r0 = (long long)tile * 32 + n, r1 = r0 + 16;
        const uint8_t* rp0 = d.W + (r0 < rows ? r0 : rows - 1) * d.row_bytes;
        const uint8_t* rp1 = d.W + (r1 < rows ? r1 : rows - 1) * d.row_bytes;

        // first blocks of this wave, loaded before the (possible) staging.
        // Loads are unconditional (block index clamped to the part's last
        // block) so every path has the same loads in flight and the waits
        // before a decode cover only the older loads.
        typename F::Raw ra[kPF], rb[kPF];
        int blk = kb0 + w;
        auto load_blk = [&](int bq, typename F::Raw& a0, typename F::Raw& a1) {
            const int bc = bq < kb1 ? bq : kb1 - 1;
            F::template load<AL>(rp0 + (size_t)bc * F::BPB, g, a0);
            F::template load<AL>(rp1 + (size_t)bc * F::BPB, g, a1);
        };
        // short parts (one block per wave at most) skip the prefetch pipeline
        const bool piped = kb1 - kb0 > 4;
        load_blk(blk, ra[0], rb[0]);
        if (piped) {
#pragma unroll
            for (int p = 1; p < kPF; ++p) load_blk(blk + 4 * p, ra[p], rb[p]);
        }

        if (mi != staged_mi || kp != staged_kp) {
            // Each token is staged scaled by the power of two 2^-e that brings
            // its largest finite |x| into [2^14, 2^15) (see norm_exp); results
            // are multiplied back by 2^e (exact).
            lds_barrier();
            if (tid < 8) tok_max[tid] = 0u;
            lds_barrier();
            x_max<MB>(d, s0, s1, tid, tok_max);
            lds_barrier();
            stage_x<MB>(d, s0, s1, tid, tok_max, frag);
            lds_barrier();
            staged_mi = mi;
            staged_kp = kp;
        }

        f4v acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        // each slot is refilled right after its block is decoded, so the other
        // slots' loads stay in flight during every decode
        if (!piped) {
            if (blk < kb1) mx_block<T, MB>(ra[0], rb[0], frag + (blk * F::STEPS - s0) * 4 * MB, g, n, acc);
        } else while (blk < kb1) {
#pragma unroll
            for (int p = 0; p < kPF; ++p) {
                const int bq = blk + 4 * p;
                if (bq < kb1) mx_block<T, MB>(ra[p], rb[p], frag + (bq * F::STEPS - s0) * 4 * MB, g, n, acc);
                load_blk(bq + 4 * kPF, ra[p], rb[p]);
            }
            blk += 4 * kPF;
        }

        // Sum the 4 waves' partials in a fixed order.  Lane (n, g) of wave w
        // holds rows r0 / r1 and token-parts 4g..4g+3 = tokens 2g and 2g+1 (hi, lo).
        float* rw = red + (w * 2 * 64 + lane) * 4;
        *reinterpret_cast<f4v*>(rw) = acc[0];
        *reinterpret_cast<f4v*>(rw + 64 * 4) = acc[1];
        lds_barrier();
        const int rt = tid >> 7, t = (tid >> 4) & 7, nn = tid & 15;
        float sum;
        {
            const int src = ((t >> 1) << 4) | nn, j = (t & 1) * 2;
            sum = 0.f;
#pragma unroll
            for (int ww = 0; ww < 4; ++ww) {
                const float* q = red + ((ww * 2 + rt) * 64 + src) * 4;
                sum += q[j] + q[j + 1];
            }
            sum = __builtin_amdgcn_ldexpf(sum, norm_exp(__uint_as_float(tok_max[t])));
        }
        const int trow = rt * 16 + nn;
        const long long row = (long long)tile * 32 + trow;
        if (d.ksplit == 1) {
            if (t < d.batch && row < rows) d.Y[t * d.ldy + row] = sum;
        } else {
            // split K: publish this part; the last part to arrive sums all parts
            // in part order (deterministic) and writes y, then re-arms the
            // counter (device-coherent hand-off, see st_dev / arrive_dev).
            float* pt = d.part + ((size_t)kp * d.tiles + tile) * 256;
            st_dev(pt + trow * 8 + t, sum);
            drain_dev();
            __syncthreads();
            if (tid == 0) last_flag = arrive_dev(&d.counters[tile]) == (unsigned)(d.ksplit - 1);
            __syncthreads();
            if (last_flag) {
                float tot = 0.f;
                for (int k = 0; k < d.ksplit; ++k) tot += ld_dev(d.part + ((size_t)k * d.tiles + tile) * 256 + trow * 8 + t);
                if (t < d.batch && row < rows) d.Y[t * d.ldy + row] = tot;
                if (tid == 0) st_dev(&d.counters[tile], 0u);
            }
        }
        lds_barrier();
    }
}

// ---------------------------------------------------------------- launcher

constexpr long long kMxTargetWgs = 1024;
// bytes of A fragments per workgroup: with the reduction area and the small
// static arrays the workgroup stays within 64 KiB of LDS
constexpr int kMxLdsBudget = 65536 - kRedBytes - 512;

struct MxPlanOut {
    long long tasks;
    size_t part_floats;
    size_t counters;
    int max_kps;
};

template <int T, int MB>
static MxPlanOut mx_plan(MxGroup& grp) {
    using F = Mx<T>;
    MxPlanOut out{0, 0, 0, 0};
    int kc = kMxLdsBudget / (MB * 64);
    kc -= kc % F::STEPS;
    for (int i = 0; i < grp.n; ++i) {
        MxDesc& d = grp.d[i];
        const int nsteps = d.cols / 32, nblk = d.cols / F::BS;
        d.tiles = (d.rows + 31) / 32;
        // K parts: only as many as the LDS budget for the activations needs
        // (a matrix's parts depend on its own shape, never on its group)
        int ks = (nsteps + kc - 1) / kc;
        int bpp = (nblk + ks - 1) / ks;  // blocks per part
        ks = (nblk + bpp - 1) / bpp;
        d.ksplit = ks;
        d.kpart_steps = bpp * F::STEPS;
        d.task_begin = (int)out.tasks;
        out.tasks += (long long)ks * d.tiles;
        if (ks > 1) {
            out.part_floats += (size_t)ks * d.tiles * 256;
            out.counters += d.tiles;
        }
        if (d.kpart_steps > out.max_kps) out.max_kps = d.kpart_steps;
    }
    return out;
}

// Split-K workspace, one per device, grown on demand.  Counters are zeroed
// when allocated and every launch leaves them at zero.  Launches that split K
// on one device must be ordered on one stream (they share this buffer).
struct MxWorkspace {
    float* part = nullptr;
    size_t part_cap = 0;
    unsigned* counters = nullptr;
    size_t counter_cap = 0;
};
static MxWorkspace g_ws[64];

static hipError_t mx_workspace(size_t part_floats, size_t counters, float** part, unsigned** ctr,
                               hipStream_t stream) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= 64) return e != hipSuccess ? e : hipErrorInvalidDevice;
    MxWorkspace& w = g_ws[dev];
    if (part_floats > w.part_cap || counters > w.counter_cap) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
            return hipErrorStreamCaptureUnsupported;  // grow the workspace before capturing
        (void)hipStreamSynchronize(stream);
        if (part_floats > w.part_cap) {
            if (w.part) (void)hipFree(w.part);
            w.part = nullptr;
            w.part_cap = 0;
            const size_t want = part_floats + part_floats / 2;
            if ((e = hipMalloc(&w.part, want * sizeof(float))) != hipSuccess) return e;
            w.part_cap = want;
        }
        if (counters > w.counter_cap) {
            if (w.counters) (void)hipFree(w.counters);
            w.counters = nullptr;
            w.counter_cap = 0;
            const size_t want = counters + counters / 2 + 256;
            if ((e = hipMalloc(&w.counters, want * sizeof(unsigned))) != hipSuccess) return e;
            if ((e = hipMemset(w.counters, 0, want * sizeof(unsigned))) != hipSuccess) return e;
            w.counter_cap = want;
        }
    }
    *part = w.part;
    *ctr = w.counters;
    return hipSuccess;
}

template <int T, int MB, bool AL>
static hipError_t mx_launch_group(MxGroup& grp, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    const MxPlanOut plan = mx_plan<T, MB>(grp);
    grp.total_tasks = (int)plan.tasks;
    if (plan.part_floats) {
        float* part = nullptr;
        unsigned* ctr = nullptr;
        hipError_t e = mx_workspace(plan.part_floats, plan.counters, &part, &ctr, stream);
        if (e != hipSuccess) return e;
        size_t po = 0, co = 0;
        for (int i = 0; i < grp.n; ++i) {
            MxDesc& d = grp.d[i];
            if (d.ksplit > 1) {
                d.part = part + po;
                d.counters = ctr + co;
                po += (size_t)d.ksplit * d.tiles * 256;
                co += d.tiles;
            } else {
                d.part = nullptr;
                d.counters = nullptr;
            }
        }
    }
    const long long wgs = plan.tasks < kMxTargetWgs ? plan.tasks : kMxTargetWgs;
    const size_t lds = kRedBytes + (size_t)plan.max_kps * 4 * MB * 16;
    if (start || stop)
        hipExtLaunchKernelGGL((mx_kernel<T, MB, AL>), dim3((unsigned)wgs), dim3(256), (uint32_t)lds, stream, start,
                              stop, 0, grp);
    else
        hipLaunchKernelGGL((mx_kernel<T, MB, AL>), dim3((unsigned)wgs), dim3(256), lds, stream, grp);
    return hipGetLastError();
}

template <int T, bool AL>
static hipError_t mx_launch_type(int batch, MxGroup& grp, hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
    if constexpr (Geo<T>::bs > 1) {
        if (batch <= 1) return mx_launch_group<T, 2, AL>(grp, s, e0, e1);
        if (batch <= 2) return mx_launch_group<T, 4, AL>(grp, s, e0, e1);
        if (batch <= 4) return mx_launch_group<T, 8, AL>(grp, s, e0, e1);
        return mx_launch_group<T, 16, AL>(grp, s, e0, e1);
    }
    return hipErrorInvalidValue;
}

bool mx_type_supported(int type) {
    switch (type) {
    case T_Q4_0: case T_Q4_1: case T_Q5_0: case T_Q5_1: case T_Q8_0: case T_Q8_1: case T_Q2_K:
    case T_Q3_K: case T_Q4_K: case T_Q5_K: case T_Q6_K: case T_IQ4_NL: case T_IQ4_XS:
        return true;
    default:
        return false;
    }
}

// Launch the MFMA path for up to 8 activation vectors starting at vector
// `done` of each matrix; arguments already validated.
int mx_group_launch(int type, const MatvecArgs* mats, size_t n, size_t batch, size_t done, bool al,
                    hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    const TypeGeo geo = type_geo(type);
    for (size_t base = 0; base < n; base += kMxMaxGroup) {
        MxGroup grp;
        grp.n = (int)((n - base) < (size_t)kMxMaxGroup ? (n - base) : (size_t)kMxMaxGroup);
        for (int i = 0; i < grp.n; ++i) {
            const MatvecArgs& m = mats[base + i];
            MxDesc& d = grp.d[i];
            d.W = static_cast<const uint8_t*>(m.w);
            d.row_bytes = m.cols / geo.bs * geo.bpb;
            d.X = m.x + done * m.ldx;
            d.ldx = m.ldx;
            d.Y = m.y + done * m.ldy;
            d.ldy = m.ldy;
            d.rows = (int)m.rows;
            d.cols = (int)m.cols;
            d.batch = (int)batch;
            d.part = nullptr;
            d.counters = nullptr;
        }
        hipEvent_t e0 = base == 0 ? start : nullptr;
        hipEvent_t e1 = (base + kMxMaxGroup >= n) ? stop : nullptr;
        hipError_t e = hipSuccess;
#define PYRITE_MX_CASE(T)                                                                  \
    case T:                                                                              \
        e = al ? mx_launch_type<T, (Geo<T>::bpb % 4 == 0)>((int)batch, grp, stream, e0, e1) \
               : mx_launch_type<T, false>((int)batch, grp, stream, e0, e1);               \
        break;
        switch (type) {
            PYRITE_MX_CASE(T_Q4_0)
            PYRITE_MX_CASE(T_Q4_1)
            PYRITE_MX_CASE(T_Q5_0)
            PYRITE_MX_CASE(T_Q5_1)
            PYRITE_MX_CASE(T_Q8_0)
            PYRITE_MX_CASE(T_Q8_1)
            PYRITE_MX_CASE(T_Q2_K)
            PYRITE_MX_CASE(T_Q3_K)
            PYRITE_MX_CASE(T_Q4_K)
            PYRITE_MX_CASE(T_Q5_K)
            PYRITE_MX_CASE(T_Q6_K)
            PYRITE_MX_CASE(T_IQ4_NL)
            PYRITE_MX_CASE(T_IQ4_XS)
        default:
            return -1;
        }
#undef PYRITE_MX_CASE
        if (e != hipSuccess) return -4;
    }
    return 0;
}

}  // namespace pyrite
