// Shared device helpers for the gfx950 GGML kernels.
//
// Weight bytes are GGUF block payloads uploaded verbatim into HBM.  Several
// block sizes (18, 22, 34, 110, 210 bytes) leave blocks only 2-byte aligned, so
// the loaders below read whole, dword-aligned words and realign them with
// v_alignbyte_b32.  Every dword a loader touches contains at least one byte of
// the requested span, so no load leaves the caller's buffer.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace pyrite {

// ---------------------------------------------------------------- type table
// Ids, block sizes and bytes per block of the 21 supported GGML types, in the
// order of the reference table (pyrite/kernels/native.c:451-473).
enum TypeId : int {
    T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 6, T_Q5_1 = 7, T_Q8_0 = 8,
    T_Q8_1 = 9, T_Q2_K = 10, T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14,
    T_IQ4_NL = 20, T_IQ4_XS = 23, T_I8 = 24, T_I16 = 25, T_I32 = 26, T_I64 = 27,
    T_F64 = 28, T_BF16 = 30,
};

template <int T> struct Geo;
#define PYRITE_GEO(T, BS, BPB) \
    template <> struct Geo<T> { static constexpr int bs = BS; static constexpr int bpb = BPB; };
PYRITE_GEO(T_F32, 1, 4)
PYRITE_GEO(T_F16, 1, 2)
PYRITE_GEO(T_Q4_0, 32, 18)
PYRITE_GEO(T_Q4_1, 32, 20)
PYRITE_GEO(T_Q5_0, 32, 22)
PYRITE_GEO(T_Q5_1, 32, 24)
PYRITE_GEO(T_Q8_0, 32, 34)
PYRITE_GEO(T_Q8_1, 32, 36)
PYRITE_GEO(T_Q2_K, 256, 84)
PYRITE_GEO(T_Q3_K, 256, 110)
PYRITE_GEO(T_Q4_K, 256, 144)
PYRITE_GEO(T_Q5_K, 256, 176)
PYRITE_GEO(T_Q6_K, 256, 210)
PYRITE_GEO(T_IQ4_NL, 32, 18)
PYRITE_GEO(T_IQ4_XS, 256, 136)
PYRITE_GEO(T_I8, 1, 1)
PYRITE_GEO(T_I16, 1, 2)
PYRITE_GEO(T_I32, 1, 4)
PYRITE_GEO(T_I64, 1, 8)
PYRITE_GEO(T_F64, 1, 8)
PYRITE_GEO(T_BF16, 1, 2)
#undef PYRITE_GEO

// ---------------------------------------------------------------- scalars
__device__ __forceinline__ float half_bits_to_float(uint32_t h16) {
    // v_cvt_f32_f16: exact for every binary16 input, subnormals included
    // (kernels run with f16 denormals enabled, the gfx9 default).
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(h16 & 0xFFFFu));
}

__device__ __forceinline__ double half_bits_to_double(uint32_t h16) {
    return (double)half_bits_to_float(h16);
}

__device__ __forceinline__ float bf16_bits_to_float(uint32_t b16) {
    return __uint_as_float((b16 & 0xFFFFu) << 16);
}

// ---------------------------------------------------------------- loads
__device__ __forceinline__ uint32_t ld_u32(const uint8_t* p) {
    return *reinterpret_cast<const uint32_t*>(p);
}

// Four dwords from a 4-byte-aligned address: one global_load_dwordx4.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
__device__ __forceinline__ void ld_a4x4(const uint8_t* p, uint32_t (&w)[4]) {
    u32x4_a4 v = *reinterpret_cast<const u32x4_a4*>(p);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
}

// Global loads at any byte address: gfx950 global loads accept unaligned
// addresses (the unaligned access mode ROCm runs the GPU in).
typedef uint32_t u32x4_a1 __attribute__((ext_vector_type(4), aligned(1)));
typedef uint32_t u32x2_a1 __attribute__((ext_vector_type(2), aligned(1)));
typedef uint32_t u32_a1 __attribute__((aligned(1)));
typedef uint16_t u16_a1 __attribute__((aligned(1)));

// N dwords holding bytes [p, p + NB) (NB <= 4N), p of any alignment when !AL.
// Aligned case: plain dword loads (merged into dwordx4 where possible).
// Unaligned case, UA: dwordx4 / dwordx2 / dword loads at the span's own byte
// addresses, then a 16- and an 8-bit load for a tail of 1-3 bytes, so every
// load lies inside the span; the bytes past NB in the last output word are 0.
// (Fewer instructions; measured faster for the 16-byte spans of the 210- and
// 110-byte super-blocks, slower for the whole-block spans of the 18- and
// 34-byte blocks, whose lanes' spans straddle 16-byte boundaries.)
// Unaligned case, !UA: dword-aligned loads whose addresses are clamped to the
// last dword that still overlaps the span, then v_alignbyte_b32 realigns them;
// the bytes past NB in the last output word are unspecified.
template <int NB, bool AL, bool UA = false>
__device__ __forceinline__ void ld_span(const uint8_t* p, uint32_t (&w)[(NB + 3) / 4]) {
    constexpr int N = (NB + 3) / 4;
    if constexpr (AL) {
#pragma unroll
        for (int k = 0; k < N; k += 4) {
            if (k + 4 <= N) {
                uint32_t t[4];
                ld_a4x4(p + 4 * k, t);
                w[k] = t[0]; w[k + 1] = t[1]; w[k + 2] = t[2]; w[k + 3] = t[3];
            } else {
#pragma unroll
                for (int j = k; j < N; ++j) w[j] = ld_u32(p + 4 * j);
            }
        }
    } else if constexpr (UA) {
        constexpr int K4 = NB / 16 * 4;                     // dwords from dwordx4 loads
        constexpr int K2 = (NB - 4 * K4) / 8 * 2;           // then from a dwordx2 load
        constexpr int K1 = (NB - 4 * K4 - 4 * K2) / 4;      // then from a dword load
        constexpr int REM = NB - 4 * (K4 + K2 + K1);        // tail bytes (0-3)
#pragma unroll
        for (int k = 0; k < K4; k += 4) {
            const u32x4_a1 v = *reinterpret_cast<const u32x4_a1*>(p + 4 * k);
            w[k] = v.x; w[k + 1] = v.y; w[k + 2] = v.z; w[k + 3] = v.w;
        }
        if constexpr (K2 > 0) {
            const u32x2_a1 v = *reinterpret_cast<const u32x2_a1*>(p + 4 * K4);
            w[K4] = v.x; w[K4 + 1] = v.y;
        }
        if constexpr (K1 > 0) w[K4 + K2] = *reinterpret_cast<const u32_a1*>(p + 4 * (K4 + K2));
        if constexpr (REM > 0) {
            constexpr int o = 4 * (K4 + K2 + K1);
            uint32_t t = 0;
            if constexpr (REM >= 2) t = *reinterpret_cast<const u16_a1*>(p + o);
            if constexpr (REM == 3) t |= (uint32_t)p[o + 2] << 16;
            if constexpr (REM == 1) t = p[o];
            w[N - 1] = t;
        }
    } else {
        // base = p rounded down to a dword (pointer arithmetic keeps the global
        // address space); dword k of the span window is safe to read unclamped
        // while 4k <= NB - 4, because the last dword overlapping the span starts
        // at ((s + NB - 1) & ~3) >= NB - 4.
        const uint32_t s = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 3u);
        const uint8_t* base = p - s;
        const uint32_t last = (s + NB - 1) & ~3u;
        // dwords [0, NX4) come from dwordx4 loads that lie wholly inside the window
        constexpr int NX4 = (NB >= 16) ? ((NB - 16) / 16 + 1) * 4 : 0;
        uint32_t t[N + 1];
#pragma unroll
        for (int k = 0; k < NX4; k += 4) {
            uint32_t v[4];
            ld_a4x4(base + 4 * k, v);
            t[k] = v[0]; t[k + 1] = v[1]; t[k + 2] = v[2]; t[k + 3] = v[3];
        }
#pragma unroll
        for (int k = NX4; k <= N; ++k) {
            if (4 * k + 4 <= NB) {
                t[k] = ld_u32(base + 4 * k);
            } else {
                const uint32_t off = (4u * k < last) ? 4u * k : last;
                t[k] = ld_u32(base + off);
            }
        }
#pragma unroll
        for (int k = 0; k < N; ++k) w[k] = __builtin_amdgcn_alignbyte(t[k + 1], t[k], s);
    }
}

// ---------------------------------------------------------------- x access
__device__ __forceinline__ float4 ld_x4(const float* p) {
    return *reinterpret_cast<const float4*>(p);
}

// Bit operations whose result the compiler cannot see through.  Code words are
// built with these so that the byte conversions below stay single
// v_cvt_f32_ubyte{0..3} instructions; with a visible mask the compiler turns
// each byte into v_bfe_u32 + v_cvt_f32_ubyte0 (two instructions per weight).
__device__ __forceinline__ uint32_t oand(uint32_t v, uint32_t m) {
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "s"(m), "v"(v));
    return r;
}
// (v & m) | c
__device__ __forceinline__ uint32_t oandor(uint32_t v, uint32_t m, uint32_t c) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(m), "v"(c));
    return r;
}
// (hi & mask) | (lo & ~mask)
__device__ __forceinline__ uint32_t obfi(uint32_t mask, uint32_t hi, uint32_t lo) {
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(mask), "v"(hi), "v"(lo));
    return r;
}

// sum_i ubyte_i(v) * x_i + acc  (v_cvt_f32_ubyte{0..3} + v_fmac)
__device__ __forceinline__ float dot_ub4(uint32_t v, float4 x, float acc) {
    acc = fmaf((float)(v & 0xFFu), x.x, acc);
    acc = fmaf((float)((v >> 8) & 0xFFu), x.y, acc);
    acc = fmaf((float)((v >> 16) & 0xFFu), x.z, acc);
    acc = fmaf((float)(v >> 24), x.w, acc);
    return acc;
}

// IQ4 codebook (kvalues_iq4nl, pyrite/kernels/native.c:347-349) biased by +128
// so every entry is an unsigned byte: 1 24 45 63 79 93 106 118 129 141 153 166
// 181 197 217 241.
constexpr uint32_t IQ4B_0 = 0x3F2D1801u, IQ4B_1 = 0x766A5D4Fu;
constexpr uint32_t IQ4B_2 = 0xA6998D81u, IQ4B_3 = 0xF1D9C5B5u;

// Look up four nibbles (one per byte, values 0..15) in the biased codebook.
__device__ __forceinline__ uint32_t iq4_lut4(uint32_t n) {
    const uint32_t sel = n & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(IQ4B_1, IQ4B_0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(IQ4B_3, IQ4B_2, sel);
    // selector 0x0C yields 0x00 and 0x0D yields 0xFF: a byte mask from bit 3
    const uint32_t msel = 0x0C0C0C0Cu | ((n >> 3) & 0x01010101u);
    const uint32_t mask = __builtin_amdgcn_perm(0u, 0u, msel);
    return obfi(mask, hi, lo);
}

// Spread the low 4 bits of v to bit 0 of each byte.
__device__ __forceinline__ uint32_t spread4(uint32_t v) {
    return ((v & 0xFu) * 0x00204081u) & 0x01010101u;
}

// ---------------------------------------------------------------- cross-workgroup hand-off
// A "last workgroup to arrive" step reads values that other workgroups of the
// same launch wrote.  An agent-scope fence would make them visible, but on
// gfx950 it writes back the whole L2 of the XCD (buffer_wbl2), which costs
// microseconds per call.  Instead the shared values are stored and loaded as
// agent-scope relaxed atomics (device-coherent accesses that do not leave
// stale copies in a per-XCD L2), and a workgroup increments the arrival
// counter only after its own stores have completed (s_waitcnt 0).  The reader
// runs only after observing the final count.  Nothing spins: a workgroup that
// is not last simply exits.
//
// Why this is enough (an argument about gfx950 hardware, not the C++ memory
// model, under which relaxed atomics alone would not order the stores before
// the reads):
//   1. an agent-scope atomic store or load is performed at the device-coherent
//      level (it does not stay in or read from one XCD's L2), so every
//      agent-scope access to an address sees one order of values;
//   2. s_waitcnt 0 returns only after the wave's earlier stores have been
//      acknowledged by that level, so they precede the counter increment,
//      which is itself performed there;
//   3. the deciding workgroup issues its loads only after the increment's
//      returned value (the final count) has arrived and been branched on, and
//      a wave issues memory instructions in program order, so each load is
//      performed after every contributor's stores.
// Callers: the split-K sum of the MFMA matvec (mx.hip), the LM-head argmax
// and fused head (lmhead.hip), the MoE router/routing hand-offs and plan
// (moe.hip).  The library builds for gfx950 only; another target would need
// this argument checked again.
template <typename V>
__device__ __forceinline__ void st_dev(V* p, V v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename V>
__device__ __forceinline__ V ld_dev(const V* p) {
    return __hip_atomic_load(const_cast<V*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// wait until this wave's earlier memory operations have completed
__device__ __forceinline__ void drain_dev() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// returns the counter's previous value; every wave that stored shared values
// must drain_dev() before the barrier that precedes this call
__device__ __forceinline__ unsigned arrive_dev(unsigned* counter) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Arrival of workgroup k of n at a two-level counter tree: fan sub-counters
// sub[0..fan) and a root; workgroup k arrives at sub[k % fan], the last of
// each sub-counter's members at the root.  True for exactly one workgroup, the
// last to arrive overall.  Leaves every sub-counter at zero; the root is left
// at its final count, for the caller to reset.  Device-scope atomics on one
// address are serialised (measured about 30 ns apart on MI355X), so n
// arrivals on a single counter take n times that; the tree cuts the chain to
// about n / fan + fan.  Same calling rules as arrive_dev.
__device__ __forceinline__ bool arrive_tree(unsigned* sub, unsigned* root, unsigned fan, unsigned k, unsigned n) {
    if (fan > n) fan = n;
    const unsigned j = k % fan;
    const unsigned members = (n - j + fan - 1) / fan;  // workgroups k' < n with k' % fan == j
    if (arrive_dev(sub + j) != members - 1) return false;
    st_dev(sub + j, 0u);
    return arrive_dev(root) == fan - 1;
}

// ---------------------------------------------------------------- lane sums
// GFX9 DPP controls: quad_perm [1,0,3,2] (lane ^ 1), quad_perm [2,3,0,1]
// (lane ^ 2), row_half_mirror (lane i <-> 7 - i inside 8), row_mirror
// (lane i <-> 15 - i inside 16).  Applied in this order each step pairs a lane
// with one from the other half of its aligned group, so after step k every
// lane holds the sum over its aligned group of 2^k lanes.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over each aligned group of 2^lg lanes (lg wave-uniform, 0..6) for every
// element of v; every lane of a group receives the group sum.
template <int R, int B>
__device__ __forceinline__ void group_sum(float (&v)[R][B], int lg) {
#define PYRITE_ALL(expr)                                      \
    _Pragma("unroll") for (int r = 0; r < R; ++r)             \
        _Pragma("unroll") for (int b = 0; b < B; ++b) expr;
    if (lg >= 1) PYRITE_ALL(v[r][b] += dpp_f<0xB1>(v[r][b]))
    if (lg >= 2) PYRITE_ALL(v[r][b] += dpp_f<0x4E>(v[r][b]))
    if (lg >= 3) PYRITE_ALL(v[r][b] += dpp_f<0x141>(v[r][b]))
    if (lg >= 4) PYRITE_ALL(v[r][b] += dpp_f<0x140>(v[r][b]))
    // ds_swizzle bit mode inside 32 lanes: and_mask 0x1F, xor_mask 0x10
    if (lg >= 5) PYRITE_ALL(v[r][b] += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v[r][b]), 0x401F)))
    if (lg >= 6) PYRITE_ALL(v[r][b] += __shfl_xor(v[r][b], 32, 64))
#undef PYRITE_ALL
}

}  // namespace pyrite
