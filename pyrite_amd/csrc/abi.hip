// C ABI of libpyrite_hip.so (declared in include/pyrite_hip.h).
//
// The drop-in entry points keep the reference's contract
// (pyrite/kernels/native.c:484-576): the same validation order and return
// codes, borrowed host buffers, no state visible to the caller.  They stage the
// call through per-thread device buffers on the per-thread default stream, so
// concurrent callers on different host threads do not share buffers or
// streams (the reference kernel is reentrant; so is this).
#include <hip/hip_runtime.h>

#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>
#include <vector>

#include "pyrite_hip.h"
#include "dispatch.h"

using namespace pyrite;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* what, hipError_t e = hipSuccess) {
    if (e != hipSuccess) {
        char buf[256];
        snprintf(buf, sizeof buf, "%s: %s", what, hipGetErrorString(e));
        g_last_error = buf;
    } else {
        g_last_error = what;
    }
    return code;
}

// Geometry check of pyrite/kernels/native.c:496-516.
int geometry(int type_id, size_t rows, size_t cols, size_t* row_bytes, size_t* expected) {
    const TypeGeo g = type_geo(type_id);
    if (!g.valid) return -1;
    if (rows == 0 || cols == 0 || cols % (size_t)g.bs != 0 || cols / g.bs > SIZE_MAX / g.bpb) return -2;
    *row_bytes = (cols / g.bs) * g.bpb;
    if (*row_bytes > SIZE_MAX / rows) return -2;
    *expected = *row_bytes * rows;
    return 0;
}

// Per-thread staging buffers for the host-pointer entry points.  They are
// kept for the life of the thread (never freed during static destruction,
// when the HIP runtime may already be gone).
struct Staging {
    void* buf[3] = {nullptr, nullptr, nullptr};
    size_t cap[3] = {0, 0, 0};
    int device = -1;

    void* get(int i, size_t bytes, hipError_t* err) {
        int dev = 0;
        *err = hipGetDevice(&dev);
        if (*err != hipSuccess) return nullptr;
        if (dev != device) {  // buffers belong to one device; drop them on a switch
            for (int k = 0; k < 3; ++k) { buf[k] = nullptr; cap[k] = 0; }
            device = dev;
        }
        if (cap[i] < bytes) {
            if (buf[i]) (void)hipFree(buf[i]);
            buf[i] = nullptr;
            cap[i] = 0;
            size_t want = bytes < 4096 ? 4096 : bytes + bytes / 4;
            *err = hipMalloc(&buf[i], want);
            if (*err != hipSuccess) return nullptr;
            cap[i] = want;
        }
        return buf[i];
    }
};
thread_local Staging g_staging;

std::mutex g_grow_mutex;
std::vector<void*> g_retired;  // replaced workspace blocks, kept until the process ends

}  // namespace

hipError_t pyrite::workspace_grow(void** block, size_t* cap, size_t want, bool zero, hipStream_t stream) {
    std::lock_guard<std::mutex> lock(g_grow_mutex);
    if (*block && *cap >= want) return hipSuccess;  // another caller grew it meanwhile
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
        return hipErrorStreamCaptureUnsupported;
    size_t bytes = want > 2 * *cap ? want : 2 * *cap;
    bytes = (bytes + 255) & ~size_t(255);
    void* fresh = nullptr;
    hipError_t e = hipMalloc(&fresh, bytes);
    if (e != hipSuccess) return e;
    if (zero && (e = hipMemset(fresh, 0, bytes)) != hipSuccess) {
        (void)hipFree(fresh);
        return e;
    }
    if (*block) g_retired.push_back(*block);
    *block = fresh;
    *cap = bytes;
    return hipSuccess;
}

extern "C" {

const char* pyrite_hip_last_error(void) { return g_last_error.c_str(); }

int pyrite_native_types(int* ids, size_t capacity) {
    const size_t count = sizeof(kTypeIds) / sizeof(kTypeIds[0]);
    if (ids == NULL) return (int)count;
    const size_t n = count < capacity ? count : capacity;
    for (size_t i = 0; i < n; ++i) ids[i] = kTypeIds[i];
    return (int)n;
}

int pyrite_matvec(int type_id, const uint8_t* data, size_t data_len, const double* x, double* out, size_t rows,
                  size_t cols) {
    size_t row_bytes = 0, expected = 0;
    const int g = geometry(type_id, rows, cols, &row_bytes, &expected);
    if (g != 0 || data == NULL || x == NULL || out == NULL || data_len != expected)
        return g != 0 ? g : -3;
    hipError_t e;
    uint8_t* dw = static_cast<uint8_t*>(g_staging.get(0, data_len, &e));
    if (!dw) return fail(-4, "pyrite_matvec: weight staging", e);
    double* dx = static_cast<double*>(g_staging.get(1, cols * sizeof(double), &e));
    if (!dx) return fail(-4, "pyrite_matvec: x staging", e);
    double* dy = static_cast<double*>(g_staging.get(2, rows * sizeof(double), &e));
    if (!dy) return fail(-4, "pyrite_matvec: y staging", e);
    hipStream_t s = hipStreamPerThread;
    if ((e = hipMemcpyAsync(dw, data, data_len, hipMemcpyHostToDevice, s)) != hipSuccess ||
        (e = hipMemcpyAsync(dx, x, cols * sizeof(double), hipMemcpyHostToDevice, s)) != hipSuccess)
        return fail(-4, "pyrite_matvec: upload", e);
    const int rc = matvec64_launch(type_id, dw, data_len, rows, cols, dx, dy, s);
    if (rc != 0) return rc == -4 ? fail(-4, "pyrite_matvec: launch", hipGetLastError()) : rc;
    if ((e = hipMemcpyAsync(out, dy, rows * sizeof(double), hipMemcpyDeviceToHost, s)) != hipSuccess ||
        (e = hipStreamSynchronize(s)) != hipSuccess)
        return fail(-4, "pyrite_matvec: download", e);
    return 0;
}

int pyrite_dequantize_rows(int type_id, const uint8_t* data, size_t data_len, double* out, size_t rows,
                           size_t cols) {
    size_t row_bytes = 0, expected = 0;
    const int g = geometry(type_id, rows, cols, &row_bytes, &expected);
    if (g != 0 || data == NULL || out == NULL || data_len != expected || cols > SIZE_MAX / rows)
        return g != 0 ? g : -3;
    if (rows * cols > SIZE_MAX / sizeof(double)) return -3;
    hipError_t e;
    uint8_t* dw = static_cast<uint8_t*>(g_staging.get(0, data_len, &e));
    if (!dw) return fail(-4, "pyrite_dequantize_rows: weight staging", e);
    double* dout = static_cast<double*>(g_staging.get(2, rows * cols * sizeof(double), &e));
    if (!dout) return fail(-4, "pyrite_dequantize_rows: output staging", e);
    hipStream_t s = hipStreamPerThread;
    if ((e = hipMemcpyAsync(dw, data, data_len, hipMemcpyHostToDevice, s)) != hipSuccess)
        return fail(-4, "pyrite_dequantize_rows: upload", e);
    const int rc = dequant_launch(type_id, dw, data_len, rows, cols, dout, 1, s);
    if (rc != 0) return rc == -4 ? fail(-4, "pyrite_dequantize_rows: launch", hipGetLastError()) : rc;
    if ((e = hipMemcpyAsync(out, dout, rows * cols * sizeof(double), hipMemcpyDeviceToHost, s)) != hipSuccess ||
        (e = hipStreamSynchronize(s)) != hipSuccess)
        return fail(-4, "pyrite_dequantize_rows: download", e);
    return 0;
}

int pyrite_dev_matvec(int type_id, const void* w, size_t w_len, size_t rows, size_t cols, const float* x,
                      size_t ldx, float* y, size_t ldy, size_t batch, void* stream) {
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : hipStreamPerThread;
    const int rc = matvec_launch(type_id, static_cast<const uint8_t*>(w), w_len, rows, cols, x, ldx, y, ldy,
                                 batch, s);
    if (rc == -4) return fail(-4, "pyrite_dev_matvec: launch", hipGetLastError());
    return rc;
}

int pyrite_dev_matvec_grouped(int type_id, const pyrite_matvec_desc* descs, size_t n, size_t batch,
                              void* stream) {
    static_assert(sizeof(pyrite_matvec_desc) == sizeof(MatvecArgs), "descriptor layout");
    if (descs == NULL) return -3;
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : hipStreamPerThread;
    const int rc = matvec_group_launch(type_id, reinterpret_cast<const MatvecArgs*>(descs), n, batch, s);
    if (rc == -4) return fail(-4, "pyrite_dev_matvec_grouped: launch", hipGetLastError());
    return rc;
}

int pyrite_dev_matvec_grouped_timed(int type_id, const pyrite_matvec_desc* descs, size_t n, size_t batch,
                                    void* stream, void* start_event, void* stop_event) {
    if (descs == NULL) return -3;
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : hipStreamPerThread;
    const int rc = matvec_group_launch(type_id, reinterpret_cast<const MatvecArgs*>(descs), n, batch, s,
                                       static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event));
    if (rc == -4) return fail(-4, "pyrite_dev_matvec_grouped_timed: launch", hipGetLastError());
    return rc;
}

int pyrite_dev_dequantize(int type_id, const void* w, size_t w_len, size_t rows, size_t cols, void* out,
                          int out_f64, void* stream) {
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : hipStreamPerThread;
    const int rc = dequant_launch(type_id, static_cast<const uint8_t*>(w), w_len, rows, cols, out, out_f64, s);
    if (rc == -4) return fail(-4, "pyrite_dev_dequantize: launch", hipGetLastError());
    return rc;
}

int pyrite_dev_lm_head_argmax(int type_id, const void* w, size_t w_len, size_t rows, size_t cols, const float* x,
                              size_t ldx, float* logits, size_t ldl, int32_t* ids, size_t batch, void* stream) {
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : hipStreamPerThread;
    const int rc = lm_head_launch(type_id, static_cast<const uint8_t*>(w), w_len, rows, cols, x, ldx, logits, ldl,
                                  reinterpret_cast<int*>(ids), batch, s);
    if (rc == -4) {
        if (const char* m = lm_last_error()) return fail(-4, m);
        return fail(-4, "pyrite_dev_lm_head_argmax: launch", hipGetLastError());
    }
    return rc;
}

int pyrite_dev_lm_head_argmax_noalloc(int type_id, const void* w, size_t w_len, size_t rows, size_t cols,
                                      const float* x, size_t ldx, float* logits, size_t ldl, int32_t* ids,
                                      size_t batch, void* stream) {
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : hipStreamPerThread;
    const int rc = lm_head_noalloc_launch(type_id, static_cast<const uint8_t*>(w), w_len, rows, cols, x, ldx,
                                          logits, ldl, reinterpret_cast<int*>(ids), batch, s);
    if (rc != 0) {
        if (const char* m = lm_last_error()) return fail(rc, m);
        if (rc == -4) return fail(-4, "pyrite_dev_lm_head_argmax_noalloc: launch", hipGetLastError());
    }
    return rc;
}

int pyrite_dev_moe_ffn(const pyrite_moe_layer* layer, const float* x, size_t ldx, float* out, size_t ldo,
                       int32_t* ids, float* weights, size_t batch, void* stream) {
    static_assert(sizeof(pyrite_moe_layer) == sizeof(MoeLayer), "MoE layer layout");
    if (layer == NULL) return -3;
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : hipStreamPerThread;
    const int rc = moe_ffn_launch(*reinterpret_cast<const MoeLayer*>(layer), x, ldx, out, ldo,
                                  reinterpret_cast<int*>(ids), weights, batch, s);
    if (rc == -4) {
        if (const char* m = moe_last_error()) return fail(-4, m);
        return fail(-4, "pyrite_dev_moe_ffn: launch", hipGetLastError());
    }
    return rc;
}

int pyrite_dev_add_rms_norm(const float* h, size_t ldh, const float* delta, size_t ldd, const float* weight,
                            size_t n, double eps, float* h_out, size_t ldo, float* normed, size_t ldn, size_t batch,
                            void* stream) {
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : hipStreamPerThread;
    const int rc = add_rms_norm_launch(h, ldh, delta, ldd, weight, n, eps, h_out, ldo, normed, ldn, batch, s);
    if (rc == -4) return fail(-4, "pyrite_dev_add_rms_norm: launch", hipGetLastError());
    return rc;
}

int pyrite_dev_matvec_swiglu(int type_id, const void* w, size_t w_len, size_t rows, size_t cols, const float* gate,
                             const float* up, size_t ldx, float* y, size_t ldy, size_t batch, void* stream) {
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : hipStreamPerThread;
    const int rc = matvec_swiglu_launch(type_id, static_cast<const uint8_t*>(w), w_len, rows, cols, gate, up, ldx, y,
                                        ldy, batch, s);
    if (rc == -4) return fail(-4, "pyrite_dev_matvec_swiglu: launch", hipGetLastError());
    return rc;
}

int pyrite_dev_attention_decode(const pyrite_attention_layer* layer, const float* q, const float* k,
                                const float* v, size_t position, size_t slot, size_t n_ctx, float* out,
                                void* stream) {
    if (!layer) return -3;
    static_assert(sizeof(pyrite_attention_layer) == sizeof(AttnLayer), "attention layer layout");
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : hipStreamPerThread;
    AttnLayer L;
    memcpy(&L, layer, sizeof L);
    if (L.rotary_dim == 0) L.rotary_dim = L.head_dim;  // the reference's `rotary_dim or head_dim`
    const int rc = attention_decode_launch(L, q, k, v, position, slot, n_ctx, out, s);
    if (rc != 0) {
        if (const char* m = attn_last_error()) return fail(rc, m);
        if (rc == -4) return fail(-4, "pyrite_dev_attention_decode: launch", hipGetLastError());
    }
    return rc;
}

int pyrite_dev_rms_norm(const float* x, size_t ldx, const float* weight, size_t n, double eps, float* y, size_t ldy,
                        size_t batch, void* stream) {
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : hipStreamPerThread;
    const int rc = rms_norm_launch(x, ldx, weight, n, eps, y, ldy, batch, s);
    if (rc == -4) return fail(-4, "pyrite_dev_rms_norm: launch", hipGetLastError());
    return rc;
}

}  // extern "C"
