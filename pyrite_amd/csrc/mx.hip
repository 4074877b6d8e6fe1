// MFMA dequant-matvec for the GGML block formats (batch 3 and up), gfx950.
// Fragment construction and block formats: mx_traits.h.
//
// Schedule: a workgroup (4 waves) owns a task = a 32-row tile of one matrix
// and a K part.  It first issues every load of the task at once: its first
// 8-token chunk's activations (unless already staged) and the tile's weight
// bytes of the part as 16-byte buffer loads (coalesced, bounds-checked by the
// buffer range so rows past the matrix read as zero), then parks the weights
// in LDS and converts the activations into fp16 hi/lo A fragments in LDS.
// Its waves then split the part's blocks round-robin, decode B fragments from
// LDS and run the MFMAs; the 4 partial results are summed in LDS in a fixed
// order, so results are deterministic.  Batches of more than 8 vectors run
// every further 8-token chunk against the same parked weights (the next
// chunk's activations loaded during the current chunk's MFMAs), so a launch
// reads each weight byte once whatever the batch.  K parts are sized so that a part's
// fragments and weights fit in LDS with two workgroups per CU; matrices with
// more parts are combined by the last part to arrive (split K).
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
    float* part;          // split-K partial sums [nchunk][ksplit][tiles][32 rows][8 tokens]
    unsigned* counters;   // per-tile arrival counters; zero between launches
    int rows;
    int cols;
    int batch;            // activation vectors
    int ksplit;           // K parts (workgroup tasks per 32-row tile)
    int kpart_steps;      // 32-column steps per K part (a multiple of the block's steps)
    int tiles;            // ceil(rows / 32)
    int task_begin;       // first task of this matrix; tasks = ksplit * tiles
    int nch;              // 16-byte chunks loaded per row and part
    int rs;               // LDS bytes per row of the staged weights
    int nchunk;           // 8-token chunks of the batch, all multiplied against the parked weights
};

constexpr int kMxMaxGroup = 16;
struct MxGroup {
    int n;
    int total_tasks;
    int frag_bytes;       // LDS bytes reserved for A fragments (largest part of the group)
    int pad;
    MxDesc d[kMxMaxGroup];
};

constexpr int kRedBytes = 4 * 2 * 64 * 4 * 4;  // [wave][row tile][lane][4] floats
// LDS bytes for one part's A fragments and staged weights: with the
// reduction area and the static arrays two workgroups fit in a CU's 160 KiB
constexpr int kMxPartBudget = 71680;
// largest number of 16-byte weight loads per thread and part
constexpr int kMxMaxWLoads = 10;
constexpr unsigned kBufferWord3 = 0x00020000u;  // raw (untyped) buffer access on gfx9

// LDS row stride for a part of nbp blocks: the 16-byte chunks covering the
// row's bytes from a 16-byte boundary, an odd number of them so that the 16
// rows a wave decodes together fall in different banks
template <int T> constexpr int mx_nch(int nbp) { return (15 + nbp * Mx<T>::BPB + 15) / 16; }
template <int T> constexpr int mx_rs(int nbp) { return 16 * (mx_nch<T>(nbp) | 1); }
template <int T, int MB> constexpr bool mx_part_fits(int nbp) {
    return nbp * Mx<T>::STEPS * MB * 64 + 32 * mx_rs<T>(nbp) + kMxLdsPad <= kMxPartBudget &&
           32 * mx_nch<T>(nbp) <= 256 * kMxMaxWLoads;
}
// largest part (in blocks) of this format at this fragment height
template <int T, int MB> constexpr int mx_max_blocks() {
    int nb = 1;
    while (mx_part_fits<T, MB>(nb + 1)) ++nb;
    return nb;
}
// activation items (8 values of one token) and weight loads per thread
template <int T, int MB> constexpr int mx_xitems() {
    return (mx_max_blocks<T, MB>() * Mx<T>::STEPS * 4 * (MB / 2) + 255) / 256;
}
template <int T, int MB> constexpr int mx_wloads() { return (32 * mx_nch<T>(mx_max_blocks<T, MB>()) + 255) / 256; }

// Barrier for LDS hand-offs only: waits for this wave's LDS traffic, not for
// its outstanding global loads (which may be blocks prefetched for later).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
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
    typename MxPreOf<F>::type pa, pb;
    mx_prep<F>(ra, g, pa);
    mx_prep<F>(rb, g, pb);
#pragma unroll
    for (int st = 0; st < F::STEPS; ++st) {
        uint4 av = make_uint4(0u, 0u, 0u, 0u);
        if (n < MB) av = fblk[(st * 4 + g) * MB + n];
        const uint32_t aw[4] = {av.x, av.y, av.z, av.w};
        const h8v a = __builtin_bit_cast(h8v, aw);
        uint32_t ba[F::NACC][4], bb[F::NACC][4];
        mx_frag<F>(ra, pa, st, g, ba);
        mx_frag<F>(rb, pb, st, g, bb);
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
__global__ __launch_bounds__(256, 2) void mx_kernel(const MxGroup grp) {
    using F = Mx<T>;
    constexpr int NT = MB / 2, XI = mx_xitems<T, MB>(), SPI = 256 / (4 * NT), WI = mx_wloads<T, MB>();
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    float* red = reinterpret_cast<float*>(smem);
    uint4* frag = reinterpret_cast<uint4*>(smem + kRedBytes);
    uint8_t* wlds = smem + kRedBytes + grp.frag_bytes;
    // largest finite |x| per token, double-buffered over stagings (ordered
    // uint bits of a non-negative float)
    __shared__ unsigned tok_max[2][8];
    __shared__ int last_flag;

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, n = lane & 15;
    // staging role: token xt, 8-column group xg of steps xs + SPI * k
    const int xt = tid % NT, xg = (tid / NT) % 4, xs = tid / (4 * NT);
    int staged_mi = -1, staged_kp = -1, tb = 1;
    if (tid < 8) tok_max[0][tid] = 0u;

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
        const int nch = d.nch, rs = d.rs;

        // 1. activations of the part's first token chunk, unless this
        // workgroup staged them last (one chunk only)
        const int nck = d.nchunk;
        const bool stage = nck > 1 || mi != staged_mi || kp != staged_kp;
        float xv[XI][8];
        auto load_x = [&](int c) {  // tokens NT c .. NT c + NT - 1
            const int tok = NT * c + xt;
            const bool tok_ok = tok < d.batch;
            const float* xp = d.X + (unsigned long long)(tok_ok ? tok : 0) * d.ldx;
#pragma unroll
            for (int k = 0; k < XI; ++k) {
                const int s = s0 + xs + SPI * k;
                if (tok_ok && s < s1) {
                    const float* q = xp + mx_col<F>(s, xg);
                    const float4 u = ld_x4(q), v = ld_x4(q + 4);
                    xv[k][0] = u.x; xv[k][1] = u.y; xv[k][2] = u.z; xv[k][3] = u.w;
                    xv[k][4] = v.x; xv[k][5] = v.y; xv[k][6] = v.z; xv[k][7] = v.w;
                } else {
#pragma unroll
                    for (int i = 0; i < 8; ++i) xv[k][i] = 0.f;
                }
            }
        };
        if (stage) load_x(0);

        // 2. the tile's weight bytes of the part: row r's chunk c is the 16
        // bytes at (its part start rounded down to 16) + 16 c.  The buffer
        // covers the tile's rows from and to a 16-byte boundary (never past
        // the page holding the matrix's last byte), so every chunk lies wholly
        // inside or wholly outside it, and outside reads as zero.
        const long long trow0 = (long long)tile * 32;
        const int trows = rows - trow0 < 32 ? (int)(rows - trow0) : 32;
        const uint8_t* tw = d.W + trow0 * d.row_bytes;
        const uint8_t* tbase = reinterpret_cast<const uint8_t*>(reinterpret_cast<uintptr_t>(tw) & ~(uintptr_t)15);
        const unsigned pre = (unsigned)(tw - tbase);
        const unsigned part0 = pre + (unsigned)kb0 * F::BPB;  // row 0's part start in the buffer
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t*>(tbase), (short)0, (int)((pre + (unsigned)trows * (unsigned)d.row_bytes + 15u) & ~15u),
            (int)kBufferWord3);
        uint4 wv[WI];
#pragma unroll
        for (int k = 0; k < WI; ++k) {
            const int c = tid + 256 * k;
            const int r = c / nch, col = c - r * nch;
            // chunks past the 32 rows get an offset beyond the buffer: zero, no traffic
            const unsigned off = r < 32 ? ((part0 + (unsigned)r * (unsigned)d.row_bytes) & ~15u) + 16u * col
                                        : 0xFFFFFFF0u;
            typedef unsigned u4v __attribute__((ext_vector_type(4)));
            const u4v v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)off, 0, 0);
            wv[k] = make_uint4(v.x, v.y, v.z, v.w);
        }

        lds_barrier();  // the previous task's fragments, weights and partials are consumed
        const uint8_t* p0 = wlds + n * rs + ((part0 + (unsigned)n * (unsigned)d.row_bytes) & 15u);
        const uint8_t* p1 = wlds + (n + 16) * rs + ((part0 + (unsigned)(n + 16) * (unsigned)d.row_bytes) & 15u);
        const int rt = tid >> 7, t = (tid >> 4) & 7, nn = tid & 15;
        const int trow = rt * 16 + nn;
        const long long row = (long long)tile * 32 + trow;
        // every token chunk against the weights parked once: the weights are
        // read from HBM once per launch whatever the batch
        for (int c = 0; c < nck; ++c) {
            // 3. build the A fragments (the first chunk's while the weight
            // loads are still in flight), then park the weights
            if (stage) {
                // Each token is staged scaled by the power of two 2^-e that brings
                // its largest finite |x| into [2^14, 2^15) (see norm_exp); results
                // are multiplied back by 2^e (exact).  A thread's items all belong
                // to token xt of the chunk.
                float mx = 0.f;
#pragma unroll
                for (int k = 0; k < XI; ++k) mx = fmaxf(mx, finite_max8(xv[k]));
                tb ^= 1;
                if (tid < 8) tok_max[tb ^ 1][tid] = 0u;
                if (mx > 0.f) atomicMax(&tok_max[tb][xt], __float_as_uint(mx));
                lds_barrier();
                const int e = norm_exp(__uint_as_float(tok_max[tb][xt]));
#pragma unroll
                for (int k = 0; k < XI; ++k) {
                    const int s = xs + SPI * k;
                    if (s0 + s < s1) {
                        uint4 hi, lo;
                        split8(xv[k], e, hi, lo);
                        uint4* f = frag + (s * 4 + xg) * MB + 2 * xt;
                        f[0] = hi;
                        f[1] = lo;
                    }
                }
            }
            // the next chunk's activations, in flight during this chunk's MFMAs
            if (c + 1 < nck) load_x(c + 1);
            if (c == 0) {
#pragma unroll
                for (int k = 0; k < WI; ++k) {
                    const int cc = tid + 256 * k;
                    const int r = cc / nch, col = cc - r * nch;
                    if (r < 32) *reinterpret_cast<uint4*>(wlds + r * rs + 16 * col) = wv[k];
                }
            }
            lds_barrier();

            // 4. this wave's blocks: rows n and n + 16 of the tile
            f4v acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
            for (int b = kb0 + w; b < kb1; b += 4) {
                typename F::Raw ra, rb;
                F::template load<AL, true>(p0 + (b - kb0) * F::BPB, g, ra);
                F::template load<AL, true>(p1 + (b - kb0) * F::BPB, g, rb);
                mx_block<T, MB>(ra, rb, frag + (b * F::STEPS - s0) * 4 * MB, g, n, acc);
            }

            // Sum the 4 waves' partials in a fixed order.  Lane (n, g) of wave w
            // holds rows r0 / r1 and token-parts 4g..4g+3 = tokens 2g and 2g+1 (hi, lo).
            float* rw = red + (w * 2 * 64 + lane) * 4;
            *reinterpret_cast<f4v*>(rw) = acc[0];
            *reinterpret_cast<f4v*>(rw + 64 * 4) = acc[1];
            lds_barrier();
            float sum;
            {
                const int src = ((t >> 1) << 4) | nn, j = (t & 1) * 2;
                sum = 0.f;
#pragma unroll
                for (int ww = 0; ww < 4; ++ww) {
                    const float* q = red + ((ww * 2 + rt) * 64 + src) * 4;
                    sum += q[j] + q[j + 1];
                }
                sum = __builtin_amdgcn_ldexpf(sum, norm_exp(__uint_as_float(tok_max[tb][t])));
            }
            const int tok = NT * c + t;
            if (d.ksplit == 1) {
                if (t < NT && tok < d.batch && row < rows) d.Y[tok * d.ldy + row] = sum;
            } else {
                st_dev(d.part + (((size_t)c * d.ksplit + kp) * d.tiles + tile) * 256 + trow * 8 + t, sum);
            }
            if (c + 1 < nck) lds_barrier();  // fragments and partials consumed before the next chunk
        }
        staged_mi = nck > 1 ? -1 : mi;
        staged_kp = kp;
        if (d.ksplit > 1) {
            // split K: every chunk of this part is published; the last part to
            // arrive sums all parts in part order (deterministic) and writes y,
            // then re-arms the counter (device-coherent hand-off, see st_dev /
            // arrive_dev)
            drain_dev();
            __syncthreads();
            if (tid == 0) last_flag = arrive_dev(&d.counters[tile]) == (unsigned)(d.ksplit - 1);
            __syncthreads();
            if (last_flag) {
                for (int c = 0; c < nck; ++c) {
                    float tot = 0.f;
                    for (int k = 0; k < d.ksplit; ++k)
                        tot += ld_dev(d.part + (((size_t)c * d.ksplit + k) * d.tiles + tile) * 256 + trow * 8 + t);
                    const int tok = NT * c + t;
                    if (t < NT && tok < d.batch && row < rows) d.Y[tok * d.ldy + row] = tot;
                }
                if (tid == 0) st_dev(&d.counters[tile], 0u);
            }
        }
        lds_barrier();
    }
}

// ---------------------------------------------------------------- launcher

constexpr long long kMxTargetWgs = 1024;

struct MxPlanOut {
    long long tasks;
    size_t part_floats;
    size_t counters;
    int max_kps;
    int max_wbytes;
};

template <int T, int MB>
static MxPlanOut mx_plan(MxGroup& grp) {
    using F = Mx<T>;
    MxPlanOut out{0, 0, 0, 0, 0};
    constexpr int kmax = mx_max_blocks<T, MB>();
    for (int i = 0; i < grp.n; ++i) {
        MxDesc& d = grp.d[i];
        const int nblk = d.cols / F::BS;
        d.tiles = (d.rows + 31) / 32;
        // K parts: only as many as the LDS budget needs, balanced (a
        // matrix's parts depend on its own shape, never on its group)
        const int ks = (nblk + kmax - 1) / kmax;
        const int bpp = (nblk + ks - 1) / ks;  // blocks per part
        d.ksplit = (nblk + bpp - 1) / bpp;
        d.kpart_steps = bpp * F::STEPS;
        d.nch = mx_nch<T>(bpp);
        d.rs = mx_rs<T>(bpp);
    }
    // Matrices split over more K parts take the lower task numbers, so their
    // workgroups start first: their last part also sums the parts, the
    // longest chain of the launch.  (Each descriptor carries its own
    // pointers; the order changes no result.)
    for (int i = 1; i < grp.n; ++i)
        for (int j = i; j > 0 && grp.d[j - 1].ksplit < grp.d[j].ksplit; --j) {
            const MxDesc t = grp.d[j];
            grp.d[j] = grp.d[j - 1];
            grp.d[j - 1] = t;
        }
    for (int i = 0; i < grp.n; ++i) {
        MxDesc& d = grp.d[i];
        d.task_begin = (int)out.tasks;
        out.tasks += (long long)d.ksplit * d.tiles;
        if (d.ksplit > 1) {
            out.part_floats += (size_t)d.nchunk * d.ksplit * d.tiles * 256;
            out.counters += d.tiles;
        }
        if (d.kpart_steps > out.max_kps) out.max_kps = d.kpart_steps;
        if (32 * d.rs > out.max_wbytes) out.max_wbytes = 32 * d.rs;
    }
    return out;
}

// Split-K workspace, one per device, grown on demand (never during stream
// capture; a replaced block stays allocated for graphs captured before).
// Counters are zeroed when allocated and every launch leaves them at zero.
// Launches that split K on one device must be ordered on one stream (they
// share this buffer).
struct MxWorkspace {
    void* part = nullptr;
    size_t part_cap = 0;  // bytes
    void* counters = nullptr;
    size_t counter_cap = 0;  // bytes
};
static MxWorkspace g_ws[64];

static hipError_t mx_workspace(size_t part_floats, size_t counters, float** part, unsigned** ctr,
                               hipStream_t stream) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= 64) return e != hipSuccess ? e : hipErrorInvalidDevice;
    MxWorkspace& w = g_ws[dev];
    const size_t pb = part_floats * sizeof(float), cb = (counters + 256) * sizeof(unsigned);
    if (pb > w.part_cap && (e = workspace_grow(&w.part, &w.part_cap, pb, false, stream)) != hipSuccess) return e;
    if (cb > w.counter_cap && (e = workspace_grow(&w.counters, &w.counter_cap, cb, true, stream)) != hipSuccess)
        return e;
    *part = static_cast<float*>(w.part);
    *ctr = static_cast<unsigned*>(w.counters);
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
                po += (size_t)d.nchunk * d.ksplit * d.tiles * 256;
                co += d.tiles;
            } else {
                d.part = nullptr;
                d.counters = nullptr;
            }
        }
    }
    const long long wgs = plan.tasks < kMxTargetWgs ? plan.tasks : kMxTargetWgs;
    grp.frag_bytes = plan.max_kps * 4 * MB * 16;
    const size_t lds = kRedBytes + (size_t)grp.frag_bytes + (size_t)plan.max_wbytes + kMxLdsPad;
    // more than 64 KiB of dynamic LDS: declare the kernel's largest need once
    static const hipError_t lds_ok = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&mx_kernel<T, MB, AL>), hipFuncAttributeMaxDynamicSharedMemorySize,
        kRedBytes + kMxPartBudget);
    if (lds_ok != hipSuccess) return lds_ok;
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

// Launch the MFMA path for the activation vectors from vector `done` of each
// matrix on (up to 8 per 8-token chunk, every chunk in the same launch, so
// each weight is read once); arguments already validated.
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
            d.nchunk = batch > 8 ? (int)((batch + 7) / 8) : 1;
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
