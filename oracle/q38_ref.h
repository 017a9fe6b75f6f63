/*
 * q38_ref.h -- CPU restatement of the reference engine's attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the oracle that the HIP
 * kernels are compared against, and the CPU baseline that bench.py times
 * beside them.  Nothing in the product library links, loads or calls it.
 *
 * Every function restates one function of the reference crate
 * (StepfenShawn/qwen3.8_27b_in_rust, src/model/ops.rs) in plain C with the
 * same operation order: fmaf() wherever the reference calls mul_add, a
 * separate multiply and add where it has `*` and `+`, f64 accumulation in
 * the two norms, the iterative f32 RoPE angle and sequential sums.  The
 * file is compiled with -ffp-contract=off so that the compiler adds no
 * fused operations of its own (rustc never contracts).
 *
 * Shapes are the crate's compile-time constants (src/model/mod.rs:13-24).
 */
#ifndef Q38_REF_H
#define Q38_REF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q38R_LINEAR_QK_HEADS 16
#define Q38R_LINEAR_V_HEADS 48
#define Q38R_LINEAR_HEAD_DIM 128
#define Q38R_LINEAR_QK_DIM 2048
#define Q38R_LINEAR_V_DIM 6144
#define Q38R_LINEAR_QKV_DIM 10240
#define Q38R_ATTN_HEADS 24
#define Q38R_ATTN_KV_HEADS 4
#define Q38R_ATTN_HEAD_DIM 256
#define Q38R_ATTN_Q_DIM 6144
#define Q38R_ATTN_QG_DIM 12288
#define Q38R_ATTN_KV_DIM 1024
#define Q38R_RMS_EPS 1e-6f

/* ---- elementwise primitives: ops.rs:476-610 ---- */
float q38r_rms_scale(const float *values, int length);                 /* ops.rs:476-483 */
void q38r_rmsnorm_inplace(float *values, const float *weight, int n);  /* ops.rs:493-498 */
float q38r_sigmoid(float x);                                           /* ops.rs:501-503 */
float q38r_silu(float x);                                              /* ops.rs:506-508 */
float q38r_softplus(float x);                                          /* ops.rs:511-516 */
void q38r_l2norm(float *values, int length);                           /* ops.rs:562-571 */
float q38r_dot_128(const float *left, const float *right);             /* ops.rs:573-579 */
float q38r_mad_dot_128(float *output, const float *input, float scale,
                       const float *right);                            /* ops.rs:584-591 */
float q38r_rope_theta_scale(void);                                     /* ops.rs:596 */
void q38r_rope(float *values, int heads, uint32_t position);          /* ops.rs:595-610 */

/*
 * Attention heads (ops.rs:868-938): `run_head` for all 24 query heads over
 * positions 0..positions-1 of one layer's cache.  Row p of head j starts at
 * key_rows + p*row_stride + j*256 (the crate's cache has row_stride 1024).
 * gate may be NULL, which skips the sigmoid gate of ops.rs:914-917.
 * scores is scratch of 24*positions floats.  n_threads > 1 splits the heads
 * across threads as rayon does (ops.rs:919-938); the result does not depend
 * on the thread count.
 */
void q38r_attn_heads(const float *q, const float *gate, const float *key_rows,
                     const float *value_rows, size_t row_stride, int positions,
                     float *scores, float *out, int n_threads);

/*
 * full_core (ops.rs:813-940), whole: q/gate split, q and k RMSNorm, RoPE,
 * KV append at current_position of the layer's slot (layer/4), attention and
 * the output gate.  Caches are [17][context_length][1024].  Returns 0, or -1
 * when the cache row is out of bounds (ops.rs:858-864).
 */
int q38r_full_core(const float *q_norm, const float *k_norm, const float *q_and_gate,
                   float *key, const float *value, float *q, float *gate, float *scores,
                   float *attention, float *key_cache, float *value_cache,
                   size_t cache_len_floats, size_t context_length, uint32_t current_position,
                   int layer, int n_threads);

/*
 * Gated-DeltaNet heads (ops.rs:689-733): decay, delta-rule update and
 * readout for all 48 value heads.  beta is post-sigmoid, g is the log-decay
 * (the reference's alpha after ops.rs:686; the decay is exp(g)).
 * state is [48][128][128], q and k [16][128], v and out [48][128].
 */
void q38r_gdn_heads(float *state, const float *q, const float *k, const float *v,
                    const float *beta, const float *g, float *out, int n_threads);

/*
 * linear_core (ops.rs:648-742), whole: conv1d (k=4) with state shift, SiLU,
 * per-head L2 norm of q and k, beta/decay gates, the recurrence, then the
 * gated RMSNorm.  conv_w is [10240][4], dt/a are [48], norm_w is [128].
 * qkv [10240], beta and alpha [48] are overwritten as in the reference.
 */
void q38r_linear_core(const float *conv_w, const float *dt, const float *a,
                      const float *norm_w, float *conv_state, float *delta_state,
                      float *qkv, const float *z, float *beta, float *alpha,
                      float *attention, int n_threads);

/* ---- weight projections: src/kernel/quant.rs, src/kernel/tensor.rs ---- */
#define Q38R_Q8K_BLOCK 256
#define Q38R_GGML_F32 0
#define Q38R_GGML_F16 1
#define Q38R_GGML_Q8_0 8
#define Q38R_GGML_Q2_K 10
#define Q38R_GGML_Q3_K 11
#define Q38R_GGML_IQ4_NL 20
#define Q38R_GGML_Q4_K 12
#define Q38R_GGML_Q5_K 13
#define Q38R_GGML_Q6_K 14
#define Q38R_GGML_IQ4_XS 23
#define Q38R_GGML_IQ2_XXS 16
#define Q38R_GGML_IQ2_XS 17
#define Q38R_GGML_IQ3_XXS 18
#define Q38R_GGML_IQ1_S 19
#define Q38R_GGML_IQ3_S 21
#define Q38R_GGML_IQ2_S 22
#define Q38R_GGML_IQ1_M 29
#define Q38R_GGML_BF16 30

float q38r_f16_to_f32(uint16_t value);                                   /* quant.rs:22-47 */
/* quantize_block, quant.rs:55-95: one 256-value block. */
void q38r_quantize_block(const float *values, float *scale, int8_t *quants, int16_t *sums);
/* quantize_q8_k, quant.rs:97-128, for n_tokens rows of `width` floats,
 * written planar: quants int8 [T][W] | sums int16 [T][W/256][16] |
 * scales f32 [T][W/256].  Returns -1 when width is not a multiple of 256. */
int q38r_quantize_q8_k(const float *input, int n_tokens, int width, void *planar);
/* Bytes of one 256-weight block of a K-quant type (0 if unsupported). */
int q38r_quant_block_bytes(int ggml_type);
/* dot_q2/q3/q4/q5/q6_k_q8_k_scalar (tensor.rs:301-457), dot_iq4_nl_q8_k and
 * dot_iq4_xs_q8_k (iq.rs:355-405): one weight row against token `token` of
 * a planar Q8_K buffer of n_tokens rows. */
float q38r_dot_q8_k(int ggml_type, const uint8_t *row, const void *planar, int n_tokens, int width, int token);
/* tensor_gemv_q8_k / tensor_gemm_q8_k (tensor.rs:1131-1173, :1217-1270):
 * out[t*rows + row] for every row and token; rows split over threads. */
int q38r_gemv_q8_k(int ggml_type, int rows, int width, const void *weights, const void *planar, int n_tokens,
                   float *out, int n_threads);

/* The f32-input path (tensor_gemv_f32 / tensor_gemm_f32, tensor.rs:1095-1129,
 * :1175-1215) for F32, F16, BF16 and Q8_0 weights: bytes and weights of one
 * block (0 if unsupported), one row dot (dot_*_scalar, tensor.rs:79-117),
 * and out[t*rows + row] for n_tokens f32 input rows [T][width]. */
int q38r_f32_block(int ggml_type, int *block_elems);
float q38r_dot_f32_row(int ggml_type, const uint8_t *row, const float *input, int n);
int q38r_gemv_f32(int ggml_type, int rows, int width, const void *weights, const float *input, int n_tokens,
                  float *out, int n_threads);

/* Layer slot maps, ops.rs:38-47. */
int q38r_is_full_attention(int layer);
int q38r_recurrent_index(int layer);

/* Thread count the CPU baseline would use: sched_getaffinity of this process. */
int q38r_available_cores(void);

#ifdef __cplusplus
}
#endif
#endif
