/*
 * libpyrite_hip.so -- MI355X (gfx950) GGML dequantize x matvec, C ABI.
 *
 * Part 1 is a drop-in for the reference's native kernel library: the same three
 * symbols, signatures, argument meaning and return codes as
 * pyrite/kernels/native.c, so pyrite/kernels/native.py can load this library
 * instead of compiling native.c (one extra branch in its _load_library).
 *
 * Part 2 is device-resident: weights are GGUF block bytes uploaded verbatim
 * into HBM, activations and outputs are fp32 device buffers, and work is
 * queued on a caller-supplied HIP stream (NULL = the per-thread default
 * stream).  These replace the per-call host round trips at the reference's
 * dispatch sites (pyrite/executor.py:481-594, 757-793, 852-875).
 * The MFMA matvec's split-K partials and counters, the LM head's candidate
 * lists and the MoE layer's plan and activations live in per-device
 * workspaces shared by every call on that device: such calls must not
 * overlap (keep them on one stream, or order the streams), and the first
 * call that grows a workspace must not race with another call.
 *
 * Return codes (pyrite/kernels/native.c:496-525, 562-566):
 *    0  success
 *   -1  unknown GGML type id
 *   -2  bad geometry: rows == 0, cols == 0, cols not a multiple of the block
 *       size, size overflow, or a shape the device kernels do not support
 *   -3  NULL pointer, data_len != rows * row_bytes, or a misaligned buffer
 *   -4  HIP runtime error (message from pyrite_hip_last_error())
 * Types: F32 F16 Q4_0 Q4_1 Q5_0 Q5_1 Q8_0 Q8_1 Q2_K Q3_K Q4_K Q5_K Q6_K
 *        IQ4_NL IQ4_XS I8 I16 I32 I64 F64 BF16 (ids 0 1 2 3 6 7 8 9 10 11 12
 *        13 14 20 23 24 25 26 27 28 30), reported in that order.
 */
#ifndef PYRITE_HIP_H
#define PYRITE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------ 1. drop-in */

/* Replaces pyrite_native_types (pyrite/kernels/native.c:484-494): ids == NULL
 * returns the count (21); otherwise copies min(count, capacity) ids in table
 * order and returns how many were written. */
int pyrite_native_types(int *ids, size_t capacity);

/* Replaces pyrite_matvec (pyrite/kernels/native.c:518-555).  data: host bytes
 * of rows x row_bytes GGUF blocks (borrowed for the call); x: host double[cols];
 * out: host double[rows].  Runs on the GPU in fp64 over the exact fp64
 * weights, so out differs from the reference only by fp64 summation order. */
int pyrite_matvec(int type_id, const uint8_t *data, size_t data_len,
                  const double *x, double *out, size_t rows, size_t cols);

/* Replaces pyrite_dequantize_rows (pyrite/kernels/native.c:557-576).  out is
 * host double[rows * cols], row-major; values are bit-identical to the
 * reference (computed in fp64 on the GPU). */
int pyrite_dequantize_rows(int type_id, const uint8_t *data, size_t data_len,
                           double *out, size_t rows, size_t cols);

/* ------------------------------------------------------------ 2. device-resident */

/* Last error message of the calling thread ("" if none). */
const char *pyrite_hip_last_error(void);

/* y[b * ldy + r] = sum_c dequant(w)[r][c] * x[b * ldx + c] for b < batch.
 * w: device bytes (rows x row_bytes, any alignment); x, y: device fp32.
 * Quantized types need x 16-byte aligned and ldx % 4 == 0.  Replaces the
 * native matvec calls of pyrite/executor.py:481-509 and 545-594 (there with
 * batch 1 and fp64 host buffers). */
int pyrite_dev_matvec(int type_id, const void *w, size_t w_len, size_t rows, size_t cols,
                      const float *x, size_t ldx, float *y, size_t ldy, size_t batch,
                      void *stream);

/* One matrix of a grouped matvec: y[b * ldy + r] = sum_c dequant(w)[r][c] * x[b * ldx + c]. */
typedef struct pyrite_matvec_desc {
    const void *w;
    size_t w_len;
    size_t rows;
    size_t cols;
    const float *x;
    size_t ldx;
    float *y;
    size_t ldy;
} pyrite_matvec_desc;

/* n same-type matrices (for example a layer's q/k/v, or gate/up) in one
 * launch per 16 matrices; same rules as pyrite_dev_matvec for each.  Replaces
 * the per-tensor loop of pyrite/executor.py:689-697 and 672-683. */
int pyrite_dev_matvec_grouped(int type_id, const pyrite_matvec_desc *descs, size_t n,
                              size_t batch, void *stream);

/* As pyrite_dev_matvec_grouped, with HIP events (hipEvent_t, may be NULL)
 * recorded by the first launch at its start and by the last at its end, so
 * they time the kernels themselves rather than host submission. */
int pyrite_dev_matvec_grouped_timed(int type_id, const pyrite_matvec_desc *descs, size_t n,
                                    size_t batch, void *stream, void *start_event,
                                    void *stop_event);

/* Exact dequantization into device memory: fp32 when out_f64 == 0 (equal to
 * (float) of the reference double) or fp64 (bit-identical).  Replaces
 * pyrite_dequantize_rows at pyrite/executor.py:470-475 (embedding rows). */
int pyrite_dev_dequantize(int type_id, const void *w, size_t w_len, size_t rows, size_t cols,
                          void *out, int out_f64, void *stream);

/* LM head with greedy selection.  logits[b * ldl + r] = fp32 dot product of
 * row r with x[b] (as pyrite_dev_matvec), and ids[b] = the first index of the
 * maximum of the reference's fp64 logits for the same x (fp32 values widened
 * to double), i.e. what pyrite/executor.py:852-875 followed by
 * Sampler.greedy (pyrite/sampler.py:12-15) returns.  The id is exact: rows
 * whose fp32 logit, widened by a rigorous rounding-error bound, could still
 * be the maximum are recomputed on the device in the reference's own fp64
 * order.  cols <= 65536.  Uses a per-device workspace grown on first use
 * (call once outside stream capture before capturing). */
int pyrite_dev_lm_head_argmax(int type_id, const void *w, size_t w_len, size_t rows, size_t cols,
                              const float *x, size_t ldx, float *logits, size_t ldl, int32_t *ids,
                              size_t batch, void *stream);

/* pyrite_dev_lm_head_argmax without any allocation, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  Same
 * arguments, results and codes as pyrite_dev_lm_head_argmax; its workspace is
 * a fixed 8 MiB device array in the library (one per GPU, kept until the
 * process ends) instead of memory allocated on first use.  Limits: batch <= 8
 * and (batch - 1) * ldl + rows <= 1894336 (e.g. 8 vectors of a 151936-row
 * vocabulary), else -2.  Every call on one GPU shares the array: calls that
 * overlap on one GPU (different streams, or host threads) race. */
int pyrite_dev_lm_head_argmax_noalloc(int type_id, const void *w, size_t w_len, size_t rows, size_t cols,
                                      const float *x, size_t ldx, float *logits, size_t ldl, int32_t *ids,
                                      size_t batch, void *stream);

/* One Qwen3-MoE FFN layer.  Tensors are GGUF bytes in device memory: the
 * router [n_experts][hidden] (ffn_gate_inp), and the stacked expert tensors
 * gate and up [n_experts][inter][hidden] and down [n_experts][hidden][inter]
 * (expert e = contiguous byte slice e, pyrite/qwen3_moe.py:364-398). */
typedef struct pyrite_moe_layer {
    int router_type;
    const void *router;
    size_t router_len;
    int gate_type;
    const void *gate;
    size_t gate_len;
    int up_type;
    const void *up;
    size_t up_len;
    int down_type;
    const void *down;
    size_t down_len;
    size_t n_experts;
    size_t hidden;
    size_t inter;
    size_t k;              /* experts per token (num_experts_per_tok) */
    int norm_topk_prob;    /* renormalise the k weights when their sum is positive */
    double scale;          /* expert_weights_scale */
} pyrite_moe_layer;

/* out[b * ldo + i] = the layer's output for token x[b] (pyrite/executor.py:757-793
 * with _expert, :672-683): router logits, softmax, experts ranked by (-p, e),
 * top k, weights (renormalised / scaled), SwiGLU experts, weighted sum in rank
 * order.  ids[b * k + s] (device int32, may be NULL) receives the chosen
 * experts in rank order, identical to the reference's; weights (device fp32,
 * may be NULL) their weights.  The expert ids stay on the device and drive
 * the expert kernels directly.  n_experts <= 1024, k <= 32, batch <= 4096.
 * Uses a per-device workspace grown on first use (call once outside stream
 * capture before capturing). */
int pyrite_dev_moe_ffn(const pyrite_moe_layer *layer, const float *x, size_t ldx, float *out, size_t ldo,
                       int32_t *ids, float *weights, size_t batch, void *stream);

/* RMSNorm: y[b][i] = x[b][i] * (1 / sqrt(sum_j x[b][j]^2 / n + eps)) * weight[i]
 * (weight NULL = 1), computed in fp64 and rounded to fp32.  Replaces
 * pyrite/tensor_ops.py:502-506 and pyrite/executor.py:621-624. */
int pyrite_dev_rms_norm(const float *x, size_t ldx, const float *weight, size_t n, double eps, float *y,
                        size_t ldy, size_t batch, void *stream);

/* ------------------------------------------------------------ 3. layer operations */

/* Residual add and RMSNorm in one pass: h_out[b] = h[b] + delta[b] (fp32), and
 * normed[b] = rms_norm(h_out[b]) * weight (weight NULL = 1; fp64 inside, one
 * rounding).  h_out may alias h.  Replaces the residual adds of
 * pyrite/executor.py:795-811 (pyrite/dense.py:497-513) together with the
 * rms_norm that follows each (the FFN norm, or the next layer's attention
 * norm). */
int pyrite_dev_add_rms_norm(const float *h, size_t ldh, const float *delta, size_t ldd, const float *weight,
                            size_t n, double eps, float *h_out, size_t ldo, float *normed, size_t ldn,
                            size_t batch, void *stream);

/* The dense FFN's down projection with its activation fused in:
 * y[b * ldy + r] = sum_c dequant(w)[r][c] * silu(gate[b * ldx + c]) * up[b * ldx + c],
 * silu(v) = v / (1 + exp(-v)) for v > -60, else 0 (pyrite/tensor_ops.py:509-510),
 * formed in fp32 while the matvec stages its input.  Block formats only (-1
 * for plain types); gate and up 16-byte aligned, ldx % 4 == 0; the staged
 * activations must fit 144 KiB of LDS, which holds at least 31040 columns
 * per vector when one vector is staged and 15520 when two are (more for the
 * 256-element formats), else -2.  Replaces the act and ffn_down steps of
 * pyrite/dense.py:473-495. */
int pyrite_dev_matvec_swiglu(int type_id, const void *w, size_t w_len, size_t rows, size_t cols,
                             const float *gate, const float *up, size_t ldx, float *y, size_t ldy, size_t batch,
                             void *stream);

/* One layer's attention geometry and its KV cache (device fp32 arrays). */
typedef struct pyrite_attention_layer {
    size_t n_heads;        /* query heads (num_attention_heads) */
    size_t n_kv_heads;     /* key/value heads; n_heads / n_kv_heads <= 16 */
    size_t head_dim;       /* query/key width per head: even, <= 256 */
    size_t value_dim;      /* value width per head: <= 256 */
    size_t rotary_dim;     /* leading values of a head that RoPE rotates: even, <= head_dim; 0 = head_dim */
    double rope_theta;
    double eps;            /* RMSNorm epsilon of the QK-norm */
    const float *q_norm;   /* [head_dim] QK-norm weights (attn_q_norm), or NULL: no query norm */
    const float *k_norm;   /* [head_dim] (attn_k_norm), or NULL */
    float *k_cache;        /* [capacity][n_kv_heads * head_dim], 8-byte aligned */
    float *v_cache;        /* [capacity][n_kv_heads * value_dim] */
    size_t capacity;       /* cache slots */
} pyrite_attention_layer;

/* Single-token attention (pyrite/executor.py:685-755 with _rope, :627-646):
 * q [n_heads * head_dim], k [n_kv_heads * head_dim], v [n_kv_heads * value_dim]
 * are this token's projections.  Each query and key head gets its QK-norm
 * (when given) and NEOX RoPE at `position`; the key (rounded to fp32, as the
 * reference's LayerKV stores it) and the value are written to cache slot
 * `slot`; then every query head h attends, with scale 1 / sqrt(head_dim), to
 * slots [0, n_ctx) of kv head h / (n_heads / n_kv_heads), and
 * out [n_heads * value_dim] receives the softmax-weighted values.  Requires
 * slot < n_ctx <= capacity.  The slots are a ring the caller manages: the
 * reference's oldest-first eviction at max_kv_tokens (LayerKV.truncate,
 * :130-134) is capacity = max_kv_tokens and slot = tokens seen % capacity
 * (the attended set is the same; its order only changes fp rounding).
 * Uses a per-device workspace grown on first use. */
int pyrite_dev_attention_decode(const pyrite_attention_layer *layer, const float *q, const float *k,
                                const float *v, size_t position, size_t slot, size_t n_ctx, float *out,
                                void *stream);

#ifdef __cplusplus
}
#endif

#endif /* PYRITE_HIP_H */
