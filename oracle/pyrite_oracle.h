/*
 * CPU oracle for the fused GGML dequantize x matvec hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library restates, in plain C with IEEE
 * double arithmetic, what the reference computes on this path so that the
 * HIP kernels can be checked against it.  Only tests/, the smoke check in
 * __graft_entry__.py and the cpu_baseline leg of bench.py may load it, and
 * only to compare against: the product library (pyrite_amd) never calls it and
 * has no CPU fallback.
 *
 * Every function names the reference file:line it follows.  Reference paths
 * are relative to the Raghav549/Pyrite checkout.
 */
#ifndef PYRITE_ORACLE_H
#define PYRITE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- type table (pyrite/kernels/native.c:444-482, pyrite/ggml_types.py:34-74) */
int oracle_native_types(int *ids, size_t capacity);
/* block elements / bytes per block for a type id; 0 on unknown id */
int oracle_type_geometry(int type_id, size_t *block_size, size_t *bytes_per_block);

/* ---- scalar helpers (pyrite/kernels/native.c:19-60) */
double oracle_half_to_double(uint16_t h);
/* IEEE double -> binary16, round-half-even, no clamping (struct '<e' semantics,
 * used by tests/k_quant.py:18-26).  Returns -1 in *overflow when the rounded
 * value does not fit (Python raises OverflowError there). */
uint16_t oracle_double_to_half(double v, int *overflow);

/* ---- per-block decode (pyrite/kernels/native.c:129-437) */
int oracle_decode_block(int type_id, const uint8_t *block, double *out);

/* ---- the C-ABI entry points restated (pyrite/kernels/native.c:484-576).
 * Same argument meaning, same accumulation order, same error codes. */
int oracle_matvec(int type_id, const uint8_t *data, size_t data_len,
                  const double *x, double *out, size_t rows, size_t cols);
int oracle_dequantize_rows(int type_id, const uint8_t *data, size_t data_len,
                           double *out, size_t rows, size_t cols);

/* ---- fixture quantizers.  Return bytes written, or a negative code:
 * -1 unknown type / no encoder, -2 n not a multiple of the block size,
 * -4 the reference encoder would raise (fp16 overflow, division by a zero step). */
long oracle_quantize(int type_id, const double *values, size_t n, uint8_t *out);

/* ---- synthetic inputs: splitmix64 -> Box-Muller (double) -> fp32 */
void oracle_fill_normal(uint64_t seed, double mean, double stddev, float *out, size_t n);

/* ---- routing / activation / sampling math (pyrite/tensor_ops.py:502-521,
 * pyrite/executor.py:757-793, pyrite/sampler.py:12-15) */
void oracle_softmax(const double *v, size_t n, double *out);
double oracle_silu(double v);
void oracle_rms_norm(const double *x, const double *w, size_t n, double eps, double *out);
long oracle_argmax_first(const double *v, size_t n);
/* pyrite/executor.py:627-646: NEOX RoPE of one head in place (the first
 * rotary_dim values; 0 = all n) */
void oracle_rope(double *v, size_t n, long position, double theta, size_t rotary_dim);
/* pyrite/executor.py:685-755 after the q/k/v projections, for one token:
 * per-head QK-norm (q_norm / k_norm may be NULL) and RoPE, the key and value
 * appended to an fp32 cache at index n_prev (caches hold n_prev earlier
 * tokens, oldest first: [n_prev + 1][n_kv * head_dim] and
 * [n_prev + 1][n_kv * value_dim]), then every head's softmax-weighted values
 * over all n_prev + 1 tokens into out [n_heads * value_dim].  -2 on a bad
 * shape. */
int oracle_attention(const double *q, const double *k, const double *v, size_t n_heads, size_t n_kv,
                     size_t head_dim, size_t value_dim, size_t rotary_dim, double theta, double eps,
                     const double *q_norm, const double *k_norm, long position, float *k_cache,
                     float *v_cache, size_t n_prev, double *out);
/* top-k routing: ids[k], weights[k]; probs[n] optional (may be NULL) */
int oracle_route(const double *logits, size_t n_experts, size_t k, int norm_topk_prob,
                 double expert_weights_scale, int *ids, double *weights, double *probs);

/* One Qwen3-MoE FFN for one token (pyrite/executor.py:672-683, 757-793).
 * Stacked tensors hold n_experts consecutive [rows x cols] slices
 * (pyrite/qwen3_moe.py:364-398): gate/up are [inter x hidden], down is
 * [hidden x inter]; the router is [n_experts x hidden]. */
int oracle_moe_ffn(const uint8_t *router, size_t router_len, int router_type,
                   const uint8_t *gate, size_t gate_len, int gate_type,
                   const uint8_t *up, size_t up_len, int up_type,
                   const uint8_t *down, size_t down_len, int down_type,
                   size_t n_experts, size_t hidden, size_t inter, size_t k,
                   int norm_topk_prob, double expert_weights_scale,
                   const double *x, double *out, int *ids, double *weights,
                   double *router_logits);

#ifdef __cplusplus
}
#endif

#endif
