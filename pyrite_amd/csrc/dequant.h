// Exact element-wise dequantization of GGML blocks on the device.
//
// dq_elem<T>(type, block, e) returns element e of one block.  With T = double
// every operation is the one the reference performs in double
// (pyrite/kernels/native.c:129-437); all products there are exact, so the
// result is bit-identical to the reference whatever the contraction mode.
// With T = float the same formulas give (float) of the reference double: each
// scale product is exact in binary32 (<= 24 significant bits) and the one
// remaining add/sub or final product rounds once, which equals rounding the
// double result (a double-precision intermediate rounds innocuously for a
// single binary32 operation).
#pragma once

#include "common.h"

namespace pyrite {

__device__ __forceinline__ uint32_t b8(const uint8_t* p) { return p[0]; }
__device__ __forceinline__ uint32_t b16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }
__device__ __forceinline__ uint32_t b32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

__constant__ static const int kIQ4[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                          1,    13,   25,  38,  53,  69,  89,  113};

template <typename T>
__device__ __forceinline__ T half_as(uint32_t h) {
    return (T)half_bits_to_float(h);
}

// Q4_K/Q5_K 6-bit (scale, min) pair j (pyrite/kernels/native.c:52-60)
__device__ __forceinline__ void k4_pair(const uint8_t* s, int j, int& sc, int& mn) {
    if (j < 4) {
        sc = s[j] & 63;
        mn = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

template <typename T>
__device__ T dq_elem(int type, const uint8_t* b, int e) {
    switch (type) {
    case T_F32: return (T)__uint_as_float(b32(b));
    case T_F16: return half_as<T>(b16(b));
    case T_BF16: return (T)bf16_bits_to_float(b16(b));
    case T_F64: {
        unsigned long long u = (unsigned long long)b32(b) | ((unsigned long long)b32(b + 4) << 32);
        return (T)__longlong_as_double((long long)u);
    }
    case T_I8: return (T)(int)(int8_t)b8(b);
    case T_I16: return (T)(int)(int16_t)b16(b);
    case T_I32: return (T)(int32_t)b32(b);
    case T_I64: {
        unsigned long long u = (unsigned long long)b32(b) | ((unsigned long long)b32(b + 4) << 32);
        return (T)(double)(long long)u;  // through double, as the reference does
    }
    case T_Q4_0: {
        const int i = e & 15;
        const int q = (e < 16) ? (b[2 + i] & 15) : (b[2 + i] >> 4);
        return half_as<T>(b16(b)) * (T)(q - 8);
    }
    case T_Q4_1: {
        const int i = e & 15;
        const int q = (e < 16) ? (b[4 + i] & 15) : (b[4 + i] >> 4);
        return half_as<T>(b16(b)) * (T)q + half_as<T>(b16(b + 2));
    }
    case T_Q5_0: {
        const int i = e & 15;
        const uint32_t qh = b32(b + 2);
        const int q = (e < 16) ? ((b[6 + i] & 15) | (int)(((qh >> i) & 1u) << 4))
                               : ((b[6 + i] >> 4) | (int)(((qh >> (i + 16)) & 1u) << 4));
        return half_as<T>(b16(b)) * ((T)q - (T)16.0);
    }
    case T_Q5_1: {
        const int i = e & 15;
        const uint32_t qh = b32(b + 4);
        const int q = (e < 16) ? ((b[8 + i] & 15) | (int)(((qh >> i) & 1u) << 4))
                               : ((b[8 + i] >> 4) | (int)(((qh >> (i + 16)) & 1u) << 4));
        return half_as<T>(b16(b)) * (T)q + half_as<T>(b16(b + 2));
    }
    case T_Q8_0: return half_as<T>(b16(b)) * (T)(int)(int8_t)b[2 + e];
    case T_Q8_1: return half_as<T>(b16(b)) * (T)(int)(int8_t)b[4 + e];
    case T_IQ4_NL: {
        const int i = e & 15;
        const int n = (e < 16) ? (b[2 + i] & 15) : (b[2 + i] >> 4);
        return half_as<T>(b16(b)) * (T)kIQ4[n];
    }
    case T_IQ4_XS: {
        const int ib = e >> 5, j = e & 15;
        const int ls = ((b[4 + ib / 2] >> (4 * (ib & 1))) & 15) | (int)(((b16(b + 2) >> (2 * ib)) & 3u) << 4);
        const T dl = half_as<T>(b16(b)) * ((T)ls - (T)32.0);
        const uint8_t q = b[8 + 16 * ib + j];
        const int n = ((e & 31) < 16) ? (q & 15) : (q >> 4);
        return dl * (T)kIQ4[n];
    }
    case T_Q2_K: {
        const int h = e >> 7, g = (e >> 5) & 3, r = (e >> 4) & 1, l = e & 15;
        const uint32_t sc = b[8 * h + 2 * g + r];
        const int q = (b[16 + 32 * h + 16 * r + l] >> (2 * g)) & 3;
        const T dl = half_as<T>(b16(b + 80)) * (T)(int)(sc & 15);
        const T ml = half_as<T>(b16(b + 82)) * (T)(int)(sc >> 4);
        return dl * (T)q - ml;
    }
    case T_Q3_K: {
        const int h = e >> 7, g = (e >> 5) & 3, r = (e >> 4) & 1, l = e & 15;
        const int j = 8 * h + 2 * g + r;
        const uint8_t* s = b + 96;
        const int low4 = (j < 8) ? (s[j] & 15) : (s[j - 8] >> 4);
        const int hi2 = (s[8 + (j & 3)] >> (2 * (j >> 2))) & 3;
        const int code = low4 | (hi2 << 4);
        const int lo = (b[32 + 32 * h + 16 * r + l] >> (2 * g)) & 3;
        const int hb = (b[16 * r + l] >> (4 * h + g)) & 1;
        const T dl = half_as<T>(b16(b + 108)) * ((T)code - (T)32.0);
        return dl * (T)(lo - (hb ? 0 : 4));
    }
    case T_Q4_K:
    case T_Q5_K: {
        const int c = e >> 6, half = (e >> 5) & 1, l = e & 31, j = 2 * c + half;
        int sc, mn;
        k4_pair(b + 4, j, sc, mn);
        const uint8_t* qs = b + (type == T_Q4_K ? 16 : 48);
        int q = half ? (qs[32 * c + l] >> 4) : (qs[32 * c + l] & 15);
        if (type == T_Q5_K && ((b[16 + l] >> j) & 1)) q += 16;
        const T d1 = half_as<T>(b16(b)) * (T)sc;
        const T m1 = half_as<T>(b16(b + 2)) * (T)mn;
        return d1 * (T)q - m1;
    }
    case T_Q6_K: {
        const int h = e >> 7, g = (e >> 5) & 3, l = e & 31;
        const uint8_t lq = b[64 * h + l + 32 * (g & 1)];
        const int low = (g & 2) ? (lq >> 4) : (lq & 15);
        const int high = (b[128 + 32 * h + l] >> (2 * g)) & 3;
        const int q = (low | (high << 4)) - 32;
        const int s = (int8_t)b[192 + 8 * h + 2 * g + l / 16];
        return half_as<T>(b16(b + 208)) * (T)s * (T)q;
    }
    default: return (T)0;
    }
}

}  // namespace pyrite
