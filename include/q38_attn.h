/*
 * q38_attn.h -- C ABI of the MI355X (gfx950) attention path of the
 * Qwen3.8-27B hybrid: full-attention GQA decode/prefill over a paged KV cache
 * and the Gated-DeltaNet recurrence.
 *
 * Reference: StepfenShawn/qwen3.8_27b_in_rust.  The path there is two private
 * functions of the model layer, full_core (src/model/ops.rs:813-940) and
 * linear_core (src/model/ops.rs:648-742), called per token from
 * full_attention / linear_attention (ops.rs:942, :744) and, token by token,
 * from the prefill loops (ops.rs:1153-1172, :1084-1099).  Their state lives
 * in Q38Model (src/model/mod.rs:155-158): key_cache / value_cache
 * [17][ctx][1024], conv_state [48][10240*3], delta_state [48][48*128*128].
 *
 * Conventions (mirroring the reference's Result<_, i32> with Err(-1)):
 *  - every function returns 0 on success and -1 on failure; q38_last_error()
 *    then gives the reason (thread-local, valid until the next failing call).
 *    Arguments are checked on the host before anything is changed: a call
 *    that fails its checks launches nothing and leaves the KV cache (pages,
 *    page tables, sequences) as it was;
 *  - pointers named d_* are device pointers; all other pointers are host
 *    memory that is read during the call and never retained;
 *  - work is stream-ordered on the context's stream; results are visible to
 *    the host after q38_sync() or q38_download();
 *  - a context and everything created from it is used from one host thread
 *    at a time (the reference has one caller thread; its parallelism is
 *    internal, as here);
 *  - shapes are the model's compile-time constants (src/model/mod.rs:13-24):
 *    attention 24 query heads, 4 kv heads, head_dim 256 (query head h reads
 *    kv head h/6); DeltaNet 16 q/k heads, 48 value heads, head_dim 128 (value
 *    head vh reads q/k head vh%16).
 */
#ifndef Q38_ATTN_H
#define Q38_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct q38_ctx q38_ctx;
typedef struct q38_kv q38_kv;

/* ------------------------------------------------------------ errors, context */

/* Text of the last failure on this thread ("" if none). */
const char *q38_last_error(void);

/* Number of HIP devices visible to this process (0 without a GPU). */
int q38_device_count(int *count);

/* Open device `device`, create the context's stream and load the gfx950 code
 * objects from module_dir (NULL: the directory holding this library).
 * Replaces the host-side setup the reference does in Q38Model::bind
 * (ops.rs:1450-1501) for the path's buffers. */
int q38_ctx_create(q38_ctx **out, int device, const char *module_dir);
int q38_ctx_destroy(q38_ctx *ctx);
/* The hipStream_t all work of this context is ordered on. */
void *q38_ctx_stream(q38_ctx *ctx);
int q38_sync(q38_ctx *ctx);
/* Compute units, peak engine clock (kHz), LDS bytes per workgroup, and the
 * device name (name_len bytes, NUL-terminated). */
int q38_device_info(q38_ctx *ctx, int *cu_count, int *clock_khz, int *lds_bytes, char *name,
                    size_t name_len);

/* Device buffers for callers that have no allocator of their own. */
int q38_alloc(q38_ctx *ctx, size_t bytes, void **d_ptr);
int q38_free(q38_ctx *ctx, void *d_ptr);
int q38_upload(q38_ctx *ctx, void *d_dst, const void *src, size_t bytes);
int q38_download(q38_ctx *ctx, void *dst, const void *d_src, size_t bytes);
int q38_zero(q38_ctx *ctx, void *d_dst, size_t bytes);

/* Context tokens one decode workgroup streams (a multiple of 16, the page
 * size, in 16..4096), or 0 (the default) to choose per launch: one workgroup per CU
 * for one sequence, at most 1024 tokens for batches.  A tuning setting with
 * no counterpart in the reference (whose rayon split is per head, ops.rs:919-938);
 * results do not depend on it beyond f32 rounding. */
int q38_set_decode_split(q38_ctx *ctx, int tokens);

/* ------------------------------------------------------------- paged KV cache */

/*
 * Device-resident paged replacement of Q38Model.key_cache / value_cache
 * (src/model/mod.rs:157-158, sized at ops.rs:1464).  n_slots full-attention
 * layer slots (the reference has 17: layers 3, 7, ..., 63 and the MTP layer
 * 64, slot = layer/4, ops.rs:858).  Each slot holds max_pages pages of 16
 * tokens; a page is [4 kv heads][16 tokens][256] f32 for K and the same for
 * V (128 KiB per page and slot).  Sequences map logical pages to physical
 * pages through a page table of max_tokens_per_seq/16 entries; one page id
 * serves the same positions in every slot.
 */
int q38_kv_create(q38_ctx *ctx, int n_slots, int max_pages, int max_seqs, int max_tokens_per_seq,
                  q38_kv **out);
int q38_kv_destroy(q38_kv *kv);
/* Pages not held by any sequence. */
int q38_kv_free_pages(q38_kv *kv, int *n_free);

/* A new empty sequence (capacity 0). */
int q38_seq_create(q38_kv *kv, int *seq);
/* Release the sequence and its pages. */
int q38_seq_free(q38_kv *kv, int seq);
/* Back to position 0 with no pages (Q38ModelOps::reset, ops.rs:1691-1699:
 * positions are rewritten before they are read again, so no page is
 * cleared). */
int q38_seq_reset(q38_kv *kv, int seq);
/* Positional rollback: keep positions < n_tokens, release whole pages past
 * them (the reference rolls the KV cache back by position only,
 * restore_target_state ops.rs:1642-1647). */
int q38_seq_truncate(q38_kv *kv, int seq, int n_tokens);
/* Make positions < n_tokens addressable, taking pages from the pool. */
int q38_seq_reserve(q38_kv *kv, int seq, int n_tokens);
/* Map the sequence's logical pages 0..n_pages-1 to the given physical pages
 * (taken out of the pool; they must be free).  For callers that place pages
 * themselves, e.g. a randomly permuted page table. */
int q38_seq_set_pages(q38_kv *kv, int seq, int n_pages, const int32_t *page_ids);
/* Positions currently addressable (a multiple of 16). */
int q38_seq_capacity(q38_kv *kv, int seq, int *n_tokens);

/* Store token rows [n_tokens][1024] (4 kv heads x 256) of K and V at
 * positions pos0.. of the sequence in layer `layer`'s slot (the append of
 * ops.rs:858-866, for many tokens).  Reserves pages as needed. */
int q38_kv_write(q38_kv *kv, int layer, int seq, int pos0, int n_tokens, const float *d_k,
                 const float *d_v);
/* Prefill's key/value block images (bf16 hi/lo copies of each 32-position
 * block, laid out as the prefill kernel's tiles) are kept per (sequence,
 * layer) between q38_attn_prefill calls, so a call converts only blocks it
 * has not converted before: a prompt prefilled in pieces, or a few tokens
 * verified after a long context, no longer re-converts the whole prefix.
 * Every write at position p (appends, q38_kv_write, prefill) and every
 * truncate, reset, free or q38_seq_set_pages drops the images from p's
 * block on.  They take 74,752 bytes per block and kv head (~9.3 KB per
 * token and layer).  enable = 0 frees them and converts every call whole;
 * results are the same bit for bit.  On by default.  No counterpart in the
 * reference (its prefill reads the f32 cache directly, ops.rs:1153-1172). */
int q38_kv_set_prefill_cache(q38_kv *kv, int enable);

/* Gather positions pos0..pos0+n_tokens-1 back into rows [n_tokens][1024]. */
int q38_kv_read(q38_kv *kv, int layer, int seq, int pos0, int n_tokens, float *d_k, float *d_v);

/* --------------------------------------------------------- full attention */

/*
 * Attention core of full_core (ops.rs:858-938) for n_seq sequences, one
 * decode token each, in layer `layer` (a full-attention layer: (layer+1)%4 ==
 * 0, or 64).  For sequence b: if d_k_new is not NULL its row b
 * ([1024] = 4 kv heads x 256, post-norm and post-RoPE) and d_v_new's row b
 * are first stored at positions[b] (ops.rs:858-866); then every query head
 * attends over positions 0..positions[b] (ops.rs:879-913) and, if d_gate is
 * not NULL, is multiplied by sigmoid(gate) (ops.rs:914-917).
 * d_q, d_gate, d_out: [n_seq][24][256] (q post-norm, post-RoPE).
 * Sequence ids must be distinct.  Fails (-1) when positions[b] + 1 exceeds
 * the sequence's context limit (the check of ops.rs:860-864 and :1702).
 */
int q38_attn_decode(q38_kv *kv, int layer, int n_seq, const int32_t *seq_ids,
                    const int32_t *positions, const float *d_q, const float *d_k_new,
                    const float *d_v_new, const float *d_gate, float *d_out);

/*
 * full_core whole (ops.rs:813-940), n_seq sequences, one token each:
 * d_q_and_gate [n_seq][24][512] (per head: 256 q then 256 gate, the layout
 * of ops.rs:832-837), d_key / d_value [n_seq][1024] raw projections,
 * d_q_norm / d_k_norm [256].  q and k get RMSNorm (eps 1e-6) and RoPE at
 * positions[b]; the new k/v are appended; d_out [n_seq][24][256] receives
 * the gated attention output.
 */
int q38_full_core(q38_kv *kv, int layer, int n_seq, const int32_t *seq_ids,
                  const int32_t *positions, const float *d_q_norm, const float *d_k_norm,
                  const float *d_q_and_gate, const float *d_key, const float *d_value,
                  float *d_out);

/*
 * q38_full_core with no device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate -- tight serving loops,
 * harnesses that forbid hipMalloc.  It is not for HIP stream capture: an
 * append that starts a new page uploads that page's id through a pinned
 * staging ring (a stream-ordered copy, and a stream synchronisation when the
 * ring wraps), and positions and page ids are launch arguments fixed at the
 * call; q38_decode_graph_* is the replayable form.  Arguments,
 * results and errors are those of q38_full_core; the split-K partials live
 * in a fixed per-device scratch array of Q38_NOALLOC_SCRATCH_BYTES instead
 * of the context's growable workspace, so a call whose partials need more
 * (n_seq sequences of P_b cached tokens: sum over b of ceil((P_b+1)/split)
 * splits x 24,768 bytes) fails with -1 before anything is changed.  The
 * scratch needs no clearing (every split writes its partials before the
 * merge reads them).  All calls on one GPU share that array: calls that
 * overlap on one GPU (other streams or contexts) race on it.  Pages for the
 * appended rows come from the pool as in q38_full_core, which allocates no
 * device memory either.
 */
#define Q38_NOALLOC_SCRATCH_BYTES (16u << 20)
int q38_full_core_noalloc(q38_kv *kv, int layer, int n_seq, const int32_t *seq_ids,
                          const int32_t *positions, const float *d_q_norm, const float *d_k_norm,
                          const float *d_q_and_gate, const float *d_key, const float *d_value,
                          float *d_out);


/* The q/k RMSNorm + RoPE prologue of full_core alone (ops.rs:832-856) for
 * n_tokens tokens at positions pos0, pos0+1, ...: writes d_q_out, d_gate_out
 * [n_tokens][24][256] and d_k_out [n_tokens][1024]. */
int q38_attn_pre(q38_ctx *ctx, int n_tokens, int pos0, const float *d_q_norm, const float *d_k_norm,
                 const float *d_q_and_gate, const float *d_key, float *d_q_out, float *d_gate_out,
                 float *d_k_out);

/*
 * Prefill of one sequence (batch_full_attention, ops.rs:1153-1172, which runs
 * full_core for tokens base_pos .. base_pos+n_tokens-1 in order): stores the
 * n_tokens rows of d_k / d_v ([n][1024], post-norm, post-RoPE) at base_pos..,
 * then token t attends causally over positions 0..base_pos+t.
 * d_q, d_gate (nullable), d_out: [n_tokens][24][256].
 */
int q38_attn_prefill(q38_kv *kv, int layer, int seq, int base_pos, int n_tokens, const float *d_q,
                     const float *d_k, const float *d_v, const float *d_gate, float *d_out);

/* ----------------------------------------------------------- Gated DeltaNet */

/*
 * Recurrence core of linear_core (ops.rs:689-733) for n_seq independent
 * states, one token each.  Sequence s: state d_state + s*state_stride floats,
 * [48][128][128] (row c of value head vh is S[vh][c][0..128]); d_q, d_k
 * [n_seq][16][128] (L2-normalised); d_v, d_out [n_seq][48][128]; d_beta
 * [n_seq][48] (post-sigmoid); d_g [n_seq][48] the log-decay (the
 * reference's alpha after ops.rs:686; the state is scaled by exp(g)).
 */
int q38_gdn_step(q38_ctx *ctx, int n_seq, float *d_state, int64_t state_stride, const float *d_q,
                 const float *d_k, const float *d_v, const float *d_beta, const float *d_g,
                 float *d_out);

/*
 * The same recurrence over n_tokens consecutive tokens of one state
 * (batch_linear_attention's token loop, ops.rs:1088-1099): d_q, d_k
 * [n_tokens][16][128], d_v and d_out [n_tokens][48][128], d_beta, d_g
 * [n_tokens][48].  The state ends as after n_tokens calls of q38_gdn_step.
 */
int q38_gdn_prefill(q38_ctx *ctx, float *d_state, int n_tokens, const float *d_q, const float *d_k,
                    const float *d_v, const float *d_beta, const float *d_g, float *d_out);

/* Per-layer DeltaNet weights of linear_core (bound at ops.rs:62-100). */
typedef struct {
    const float *d_conv_w; /* ssm_conv1d [10240][4] */
    const float *d_dt;     /* ssm_dt.bias [48] */
    const float *d_a;      /* ssm_a [48] */
    const float *d_norm;   /* ssm_norm [128] */
} q38_linear_weights;

/*
 * linear_core whole (ops.rs:648-742) for n_tokens consecutive tokens of each
 * of n_seq sequences (n_tokens > 1 is batch_linear_attention's loop,
 * ops.rs:1084-1099, with n_seq 1).  Sequence s: d_conv_state + s*30720
 * ([10240][3]), d_delta_state + s*786432 ([48][128][128]).  Per token
 * (index s*n_tokens + t): d_qkv [10240] raw projection, d_z [6144], d_beta,
 * d_alpha [48] raw; d_out [6144] receives rmsnorm(o) * silu(z).  With
 * n_tokens > 1, d_conv_state, d_qkv, d_z and d_out must be 16-byte aligned.
 */
int q38_linear_core(q38_ctx *ctx, int n_seq, int n_tokens, const q38_linear_weights *w,
                    float *d_conv_state, float *d_delta_state, const float *d_qkv,
                    const float *d_z, const float *d_beta, const float *d_alpha, float *d_out);

/* ---------------------------------------------------- replayed token graph */

/*
 * A token's work recorded once as a HIP graph and replayed per token.  The
 * reference runs, per token and layer, full_core (ops.rs:942-986 calling
 * :813-940) or linear_core (ops.rs:744-804 calling :648-742) with the
 * projections around them; a serving loop repeats the same launches every
 * token.  A graph is built in order from:
 *  - decode calls (q38_decode_graph_add_decode): the q38_attn_decode form
 *    (d_q_norm NULL: q post-norm and post-RoPE, optional append
 *    d_k_new/d_v_new, optional d_gate) or the q38_full_core form (d_q_norm
 *    and d_k_norm set: d_q holds q|gate rows, d_k_new/d_v_new the raw key
 *    and value, d_gate unused) of one full-attention layer, for the graph's
 *    n_seq (1..64) distinct sequences at the positions given at begin;
 *  - one-token linear_core calls (q38_decode_graph_add_linear_core, the
 *    arguments of q38_linear_core with n_tokens 1);
 *  - graphs of the caller's own work (q38_decode_graph_add_graph: a
 *    hipGraph_t, copied at the add), e.g. the projections and norms between
 *    the cores, captured from the caller's stream;
 * each step after the previous one.  Device buffers are fixed at the add.
 * Results equal those of the plain calls in the same order, bit for bit.
 *
 * begin: checks the sequences, records the positions; add_decode checks the
 * call at those positions and reserves the pages it appends to.  end:
 * instantiates (nothing is launched).  set_positions: waits for the
 * context's stream (a replay in flight reads the arguments it replaces),
 * checks every decode call at the new positions with nothing changed on
 * failure, reserves pages (their ids are uploaded on the stream, ahead of
 * the next replay) and rewrites every decode launch's arguments and grid;
 * the other steps do not depend on positions.  launch: one replay on the
 * context's stream at the positions last set.  The graph owns its split-K
 * workspace; no allocation, memset or host synchronisation is recorded in
 * it.  q38_decode_graph_create is begin + one add_decode per call + end.
 * Calls on one graph come from one thread.
 */
typedef struct q38_decode_graph q38_decode_graph;
typedef struct {
    int32_t layer;
    int32_t pad_;
    const float *d_q;
    const float *d_k_new;
    const float *d_v_new;
    const float *d_gate;
    const float *d_q_norm;
    const float *d_k_norm;
    float *d_out;
} q38_decode_call;
int q38_decode_graph_begin(q38_kv *kv, int n_seq, const int32_t *seq_ids, const int32_t *positions,
                           q38_decode_graph **out);
int q38_decode_graph_add_decode(q38_decode_graph *g, const q38_decode_call *call);
int q38_decode_graph_add_linear_core(q38_decode_graph *g, int n_seq, const q38_linear_weights *w,
                                     float *d_conv_state, float *d_delta_state, const float *d_qkv,
                                     const float *d_z, const float *d_beta, const float *d_alpha, float *d_out);
int q38_decode_graph_add_graph(q38_decode_graph *g, void *hip_graph);
int q38_decode_graph_end(q38_decode_graph *g);
int q38_decode_graph_create(q38_kv *kv, int n_seq, const int32_t *seq_ids, const int32_t *positions,
                            int n_calls, const q38_decode_call *calls, q38_decode_graph **out);
int q38_decode_graph_set_positions(q38_decode_graph *g, const int32_t *positions);
int q38_decode_graph_launch(q38_decode_graph *g);
int q38_decode_graph_destroy(q38_decode_graph *g);

/* ------------------------------------------------------- weight projections */

/*
 * The projections on either side of the attention path (project,
 * ops.rs:623-639): activations quantised to Q8_K once (quantize_input,
 * ops.rs:617-620) and shared by every projection of the layer, then one
 * K-quant x Q8_K dot per weight row.
 *
 * A device Q8_K buffer for n_tokens rows of `width` floats (width a multiple
 * of 256) is planar: int8 quants [n_tokens][width] | int16 sums of each 16
 * quants [n_tokens][width/256][16] | f32 scales [n_tokens][width/256];
 * q38_q8k_bytes gives its size.
 */
int q38_q8k_bytes(int n_tokens, int width, size_t *bytes);

/* quantize_q8_k (src/kernel/quant.rs:97-128, quantize_block :55-95) of
 * d_x [n_tokens][width]: per 256 values, the first value of largest
 * magnitude m sets scale m/-127 (stored as 1/(-127/m)), quants are
 * round-to-nearest-even of x * (-127/m) capped at 127; all-zero blocks give
 * zeros.  Bit-exact with the reference. */
int q38_quantize_q8_k(q38_ctx *ctx, int n_tokens, int width, const float *d_x, void *d_q8k);

/* tensor_gemv_q8_k / tensor_gemm_q8_k (src/kernel/tensor.rs:1131-1173,
 * :1217-1270) for every weight type the reference projects on this path:
 * Q2_K (ggml type 10), Q3_K (11), Q4_K (12), Q5_K (13), Q6_K (14), IQ2_XXS
 * (16), IQ2_XS (17), IQ3_XXS (18), IQ1_S (19), IQ4_NL (20), IQ3_S (21),
 * IQ2_S (22), IQ4_XS (23) and IQ1_M (29): d_weights [rows][width/256
 * blocks] in the GGUF block layout (84, 110, 144, 176, 210, 66, 74, 98, 50,
 * 8 x 18, 110, 82, 136, 56 bytes per 256 weights, 16-byte aligned base),
 * d_q8k from q38_quantize_q8_k, d_out [n_tokens][rows] (token-major, as the
 * reference's batched form writes it).  width is at most 49152.  Each
 * element equals the reference's scalar dot_q*_k_q8_k (tensor.rs:301-457)
 * or dot_iq*_q8_k (src/kernel/iq.rs:355-667) bit for bit.  From 8 tokens
 * on, where the matrix has rows for 64+ tiles of 32 rows x 32 tokens, the
 * integer dots run on the int8 matrix unit (IQ4_NL: from 32 tokens, 16 for
 * 8192+ rows); the result is the same bit for bit.  Other weight types
 * fail with -1 (the reference's f32 path below, or types outside this
 * path). */
int q38_gemv_q8_k(q38_ctx *ctx, int ggml_type, int rows, int width, const void *d_weights, const void *d_q8k,
                  int n_tokens, float *d_out);

/* Several projections of one layer that read the same quantised input
 * (project called in turn on one `quantized` buffer: q|gate, k and v in
 * full_attention, ops.rs:954-958; ffn gate and up, ops.rs:1600-1613): up
 * to 4 matrices of one type and width, matrix i with rows[i] rows at
 * d_weights[i], its output at d_out[i] [n_tokens][rows[i]], in one launch.
 * Each output equals q38_gemv_q8_k's for that matrix bit for bit, and the
 * matrices share launches: below 8 tokens every matrix streams through one
 * GEMV launch; from 8 on, a matrix whose 32-row x 32-token grid exceeds 5
 * workgroups per CU takes the 128 x 64 tiles, a launch of its own, and the
 * others share one split-block launch where their grids add up to 64
 * workgroups (the GEMV otherwise), so a matrix may take another form here
 * than alone (IQ4_NL: each matrix as in q38_gemv_q8_k). */
int q38_gemv_q8_k_multi(q38_ctx *ctx, int ggml_type, int n_mats, const int *rows, int width,
                        const void *const *d_weights, const void *d_q8k, int n_tokens, float *const *d_out);

/* quantize_input followed by project on each matrix of one input
 * (ops.rs:617-639, called so by full_attention ops.rs:954-958 and the FFN
 * ops.rs:1600-1613): the same as q38_quantize_q8_k(ctx, n_tokens, width,
 * d_x, d_q8k) and then q38_gemv_q8_k_multi(ctx, ggml_type, n_mats, rows,
 * width, d_weights, d_q8k, n_tokens, d_out), bit for bit, d_q8k (16-byte
 * aligned, q38_q8k_bytes) holding the quantised input afterwards; d_x
 * [n_tokens][width] f32, 16-byte aligned.  For one token (every matrix
 * then on the GEMV) it is one launch instead of two: each GEMV workgroup
 * quantises the input itself.  Fails with -1 as those two calls do. */
int q38_quantize_project_q8_k(q38_ctx *ctx, int ggml_type, int n_mats, const int *rows, int width,
                              const void *const *d_weights, const float *d_x, int n_tokens, void *d_q8k,
                              float *const *d_out);

/* tensor_gemv_f32 / tensor_gemm_f32 (src/kernel/tensor.rs:1095-1129,
 * :1175-1215): the projection path of weights project() does not quantise
 * for (ops.rs:632-637), with f32 activations d_x [n_tokens][width]:
 * F32 (ggml type 0), F16 (1), BF16 (30) or Q8_0 (8) weights d_weights
 * [rows][row bytes] in the GGUF layout, d_out [n_tokens][rows].  width a
 * multiple of 8 (Q8_0: of 64), d_weights 16-byte aligned (Q8_0: 4), d_x
 * 16-byte aligned.  Every product w * x enters the sum exactly (fused
 * multiply-adds, or products of exact bf16 parts), Q8_0's block scale d
 * applied to the block's sum of q * x (d * q is exact in f32, as the
 * reference forms it); the sums are reassociated (the reference's own x86
 * build reassociates them too), so each element lies within the rounding of
 * an f32 sum of the reference's scalar dot_*_scalar (tensor.rs:79-117).
 * Few tokens take a GEMV (Q8_0: the activations staged in LDS per 8 or 16
 * rows); from 4 tokens (Q8_0: 9) on, where width is a multiple of 64, the
 * bf16 matrix unit with x split exactly into three bf16 parts (F16 / F32
 * weights into two / three). */
int q38_gemv_f32(q38_ctx *ctx, int ggml_type, int rows, int width, const void *d_weights, const float *d_x,
                 int n_tokens, float *d_out);

#ifdef __cplusplus
}
#endif
#endif
