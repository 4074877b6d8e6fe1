// Host-side type geometry and launchers shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace pyrite {

struct TypeGeo {
    bool valid;
    int bs;   // elements per block
    int bpb;  // bytes per block
};

// The 21 GGML types of the reference table, in table order
// (pyrite/kernels/native.c:451-473).
constexpr int kTypeIds[21] = {0, 1, 2, 3, 6, 7, 8, 9, 10, 11, 12, 13, 14, 20, 23, 24, 25, 26, 27, 28, 30};

inline TypeGeo type_geo(int id) {
    switch (id) {
    case 0: return {true, 1, 4};
    case 1: return {true, 1, 2};
    case 2: return {true, 32, 18};
    case 3: return {true, 32, 20};
    case 6: return {true, 32, 22};
    case 7: return {true, 32, 24};
    case 8: return {true, 32, 34};
    case 9: return {true, 32, 36};
    case 10: return {true, 256, 84};
    case 11: return {true, 256, 110};
    case 12: return {true, 256, 144};
    case 13: return {true, 256, 176};
    case 14: return {true, 256, 210};
    case 20: return {true, 32, 18};
    case 23: return {true, 256, 136};
    case 24: return {true, 1, 1};
    case 25: return {true, 1, 2};
    case 26: return {true, 1, 4};
    case 27: return {true, 1, 8};
    case 28: return {true, 1, 8};
    case 30: return {true, 1, 2};
    default: return {false, 0, 0};
    }
}

#define PYRITE_FOR_EACH_TYPE(X)                                                                     \
    X(0) X(1) X(2) X(3) X(6) X(7) X(8) X(9) X(10) X(11) X(12) X(13) X(14) X(20) X(23) X(24) X(25) \
    X(26) X(27) X(28) X(30)

// One matrix of a grouped matvec (same layout as pyrite_matvec_desc).
struct MatvecArgs {
    const void* w;
    size_t w_len;
    size_t rows;
    size_t cols;
    const float* x;
    size_t ldx;
    float* y;
    size_t ldy;
};

// matvec.hip: several same-type matrices in one launch (16 per launch).
// start/stop (optional) are recorded by the first / last launch itself.
int matvec_group_launch(int type, const MatvecArgs* mats, size_t n, size_t batch, hipStream_t stream,
                        hipEvent_t start = nullptr, hipEvent_t stop = nullptr);

// mx.hip: MFMA path for the quantized block formats, up to 8 vectors starting
// at vector `done` of each matrix (arguments already validated).
bool mx_type_supported(int type);
int mx_group_launch(int type, const MatvecArgs* mats, size_t n, size_t batch, size_t done, bool al,
                    hipStream_t stream, hipEvent_t start, hipEvent_t stop);

// mg.hip: MFMA dequant-GEMM for large batches (arguments already validated);
// consecutive matrices with the same activations share a launch.
long long mg_workgroups(int type, const MatvecArgs* mats, size_t n, size_t batch, int* kblocks);
int mg_group_launch(int type, const MatvecArgs* mats, size_t n, size_t batch, bool al, hipStream_t stream,
                    hipEvent_t start, hipEvent_t stop);

// matvec.hip: Y[b][r] = sum_c W[r][c] X[b][c] in fp32, any batch (chunked by 8).
// Returns 0, -1 (type), -2 (geometry), -3 (pointer/length/alignment), -4 (launch).
int matvec_launch(int type, const uint8_t* W, size_t w_len, size_t rows, size_t cols, const float* X, size_t ldx,
                  float* Y, size_t ldy, size_t batch, hipStream_t stream);

// dequant.hip: fp64 matvec over exact fp64 weights (the host drop-in path).
int matvec64_launch(int type, const uint8_t* W, size_t w_len, size_t rows, size_t cols, const double* X,
                    double* Y, hipStream_t stream);

// lmhead.hip: fp32 logits of every row plus ids[b] = first index of the
// maximum of the reference's fp64 logits, for b < batch.
int lm_head_launch(int type, const uint8_t* W, size_t w_len, size_t rows, size_t cols, const float* X, size_t ldx,
                   float* logits, size_t ldl, int* ids, size_t batch, hipStream_t stream);
// The same over a fixed device scratch array (no allocation): batch <= 8 and
// (batch - 1) * ldl + rows <= 1894336.
int lm_head_noalloc_launch(int type, const uint8_t* W, size_t w_len, size_t rows, size_t cols, const float* X,
                           size_t ldx, float* logits, size_t ldl, int* ids, size_t batch, hipStream_t stream);
const char* lm_last_error();

// moe.hip: one Qwen3-MoE FFN layer (router, top-k, experts, combine) for
// batch tokens; layout identical to pyrite_moe_layer of include/pyrite_hip.h.
struct MoeLayer {
    int router_type;
    const void* router;
    size_t router_len;
    int gate_type;
    const void* gate;
    size_t gate_len;
    int up_type;
    const void* up;
    size_t up_len;
    int down_type;
    const void* down;
    size_t down_len;
    size_t n_experts;
    size_t hidden;
    size_t inter;
    size_t k;
    int norm_topk_prob;
    double scale;
};
int moe_ffn_launch(const MoeLayer& L, const float* X, size_t ldx, float* out, size_t ldo, int* ids_out,
                   float* wts_out, size_t batch, hipStream_t stream);
const char* moe_last_error();

// norm.hip: RMSNorm of batch vectors of n floats (Wt may be null: weight 1).
int rms_norm_launch(const float* X, size_t ldx, const float* Wt, size_t n, double eps, float* Y, size_t ldy,
                    size_t batch, hipStream_t stream);

// layer.hip: residual add + RMSNorm (Hout may alias H), the SwiGLU-staged
// down projection, and single-token attention over an fp32 KV cache.
int add_rms_norm_launch(const float* H, size_t ldh, const float* D, size_t ldd, const float* Wt, size_t n,
                        double eps, float* Hout, size_t ldo, float* N, size_t ldn, size_t batch,
                        hipStream_t stream);
int matvec_swiglu_launch(int type, const uint8_t* W, size_t w_len, size_t rows, size_t cols, const float* G,
                         const float* U, size_t ldx, float* Y, size_t ldy, size_t batch, hipStream_t stream);
// layout identical to pyrite_attention_layer of include/pyrite_hip.h
struct AttnLayer {
    size_t n_heads;
    size_t n_kv_heads;
    size_t head_dim;
    size_t value_dim;
    size_t rotary_dim;
    double rope_theta;
    double eps;
    const float* q_norm;
    const float* k_norm;
    float* k_cache;
    float* v_cache;
    size_t capacity;
};
int attention_decode_launch(const AttnLayer& L, const float* q, const float* k, const float* v, size_t position,
                            size_t slot, size_t n_ctx, float* out, hipStream_t stream);
const char* attn_last_error();

// abi.hip: grow a per-device workspace block to at least `want` bytes
// (geometrically: at least twice the old capacity), zero-filled when `zero`.
// The replaced block is never freed: a HIP graph captured before the growth
// keeps its address, so it stays allocated (and unused by later eager calls)
// until the process ends; the retired blocks of one workspace add up to less
// than its live block.  Growth is refused while `stream` is capturing
// (hipErrorStreamCaptureUnsupported).  Serialised by a process-wide mutex.
hipError_t workspace_grow(void** block, size_t* cap, size_t want, bool zero, hipStream_t stream);

// dequant.hip: exact dequantization into fp32 (out_f64 == 0) or fp64.
int dequant_launch(int type, const uint8_t* W, size_t w_len, size_t rows, size_t cols, void* out, int out_f64,
                   hipStream_t stream);

}  // namespace pyrite
