/*
 * Kernel argument blocks shared by the host launcher (g++) and the gfx950
 * code objects (hipcc --genco).  Plain C structs of pointers and 32-bit
 * integers so both compilers lay them out identically; each kernel takes its
 * block by value (it travels in the kernarg segment, so per-call metadata
 * such as sequence ids and positions needs no host-to-device copy).
 *
 * Shapes are the model's compile-time constants (reference
 * src/model/mod.rs:13-24).
 */
#ifndef Q38_KARGS_H
#define Q38_KARGS_H

#include <stdint.h>

#define Q38_ATTN_HEADS 24
#define Q38_ATTN_KV_HEADS 4
#define Q38_ATTN_GROUP 6 /* query heads per kv head: heads 6j..6j+5 read kv head j */
#define Q38_ATTN_HEAD_DIM 256
#define Q38_ATTN_Q_DIM 6144
#define Q38_ATTN_QG_DIM 12288
#define Q38_ATTN_KV_DIM 1024
#define Q38_PAGE_TOKENS 16
/* one page of one layer: [4 kv heads][16 tokens][256] floats, K and V pools apart */
#define Q38_PAGE_FLOATS (Q38_ATTN_KV_HEADS * Q38_PAGE_TOKENS * Q38_ATTN_HEAD_DIM)

#define Q38_LIN_QK_HEADS 16
#define Q38_LIN_V_HEADS 48
#define Q38_LIN_HEAD_DIM 128
#define Q38_LIN_QK_DIM 2048
#define Q38_LIN_V_DIM 6144
#define Q38_LIN_QKV_DIM 10240
#define Q38_LIN_STATE_FLOATS (Q38_LIN_V_HEADS * Q38_LIN_HEAD_DIM * Q38_LIN_HEAD_DIM)

#define Q38_MAX_BATCH 64 /* sequences per decode launch */
#define Q38_MAX_SPLITS 4096 /* splits of one sequence in one decode launch */
#define Q38_MAX_SPLIT_TOKENS 4096 /* context tokens one decode workgroup streams */
#define Q38_DECODE_WAVES 4 /* waves of a decode workgroup */
#define Q38_HEAD_PAGE_SPLITS 256 /* splits whose first page ids a decode launch can carry */

/* Split-K paged decode: grid (total_splits, 4 kv heads). */
typedef struct {
    float *kpool;              /* this layer's K pages: [max_pages][4][16][256] */
    float *vpool;              /* this layer's V pages */
    const int32_t *page_table; /* [max_seqs][pt_stride] physical page ids */
    const float *q;            /* [n_seq][24][256], post-norm, post-RoPE (fused pre step:
                                  raw [n_seq][24][512] q|gate rows) */
    const float *k_new;        /* [n_seq][1024] appended at pos[b] first, or NULL (fused pre
                                  step: the raw key, normed and rotated before the append) */
    const float *v_new;        /* [n_seq][1024] or NULL */
    const float *gate;         /* [n_seq][24][256] output gate logits, or NULL */
    float *out;                /* [n_seq][24][256] */
    float *part_o;             /* [total_splits][24][256] unnormalised partial outputs */
    float *part_ml;            /* [total_splits][24][2]  (running max in log2 units, sum) */
    const float *q_norm;       /* fused pre step: [256] q RMSNorm weight, else unused */
    const float *k_norm;       /* fused pre step: [256] k RMSNorm weight */
    float theta_scale;         /* fused pre step: RoPE 1e7^(-2/64) in f32 */
    int32_t gate_head_stride;  /* floats between heads' gates: 256, or 512 in q|gate rows */
    int32_t pt_stride;
    int32_t n_seq;
    int32_t split_tokens; /* multiple of Q38_PAGE_TOKENS */
    int32_t total_splits;
    int32_t seq[Q38_MAX_BATCH];
    int32_t pos[Q38_MAX_BATCH]; /* attend over positions 0..pos inclusive */
    int32_t split_base[Q38_MAX_BATCH + 1];
    int32_t head_pages[Q38_HEAD_PAGE_SPLITS][2]; /* physical ids of split g's first two pages (the
                                                    second repeats the first where the split has
                                                    one), when total_splits <= 256 */
} q38_decode_args;

/* Copy token rows between [n][1024] arrays and a sequence's pages.
 * grid (n_tokens, 2): y = 0 moves K, y = 1 moves V. */
typedef struct {
    float *kpool;
    float *vpool;
    const int32_t *page_table;
    float *k_rows; /* [n][1024] */
    float *v_rows;
    int32_t pt_stride;
    int32_t seq;
    int32_t pos0;
    int32_t n_tokens;
    int32_t to_pages; /* 1: rows -> pages (append), 0: pages -> rows (gather) */
    int32_t pad_;
} q38_kv_copy_args;

/* q/gate split, q and k RMSNorm, RoPE.  grid (n_tokens, 28): y < 24 is a
 * query head, y >= 24 a kv head. */
typedef struct {
    const float *q_and_gate; /* [n][24][512] head-interleaved q | gate */
    const float *key;        /* [n][4][256] raw */
    const float *q_norm;     /* [256] */
    const float *k_norm;     /* [256] */
    float *q_out;            /* [n][24][256] */
    float *gate_out;         /* [n][24][256] */
    float *k_out;            /* [n][4][256] */
    int32_t pos0;      /* token t is at position pos0 + t */
    int32_t n_tokens;
    float theta_scale; /* 1e7^(-2/64) in f32 */
    int32_t pad_;
} q38_attn_pre_args;

/* Gated-DeltaNet recurrence, one token of each of n_seq independent states
 * (q38_gdn_step_rows: grid (48 value heads x 8 row blocks, n_seq)). */
typedef struct {
    float *state;      /* seq s at state + s*state_stride: [48][128][128] */
    const float *q;    /* [s*q_stride + kh*128 ...] */
    const float *k;
    const float *v;    /* [s*v_stride + vh*128 ...] */
    const float *beta; /* [s*48 + vh], post-sigmoid */
    const float *g;    /* log-decay, same layout */
    float *out;        /* [s*6144 + vh*128 + c] */
    int64_t state_stride;
    int32_t q_stride; /* floats between consecutive sequences' q (and k) */
    int32_t v_stride;
    int32_t n_seq;
    int32_t pad_;
} q38_gdn_args;

/* linear_core whole for one token of each of n_seq sequences in one launch
 * (q38_gdn_decode: grid (48 value heads, n_seq), 512 threads). */
typedef struct {
    const float *qkv_raw;   /* [n_seq][10240] raw projection */
    const float *conv_w;    /* [10240][4] */
    float *conv_state;      /* seq s at + s*30720: [10240][3], shifted in place */
    float *state;           /* seq s at + s*786432: [48][128][128] */
    const float *z;         /* [n_seq][6144] gate of the gated RMSNorm */
    const float *beta_raw;  /* [n_seq][48] */
    const float *alpha_raw; /* [n_seq][48] */
    const float *dt;        /* [48] */
    const float *a;         /* [48] */
    const float *norm_w;    /* [128] */
    float *out;             /* [n_seq][6144] */
    int32_t *arrivals;      /* [n_seq][Q38_GDN_ARRIVALS] arrival counters (one per key head),
                               zero between calls */
} q38_gdn_decode_args;
#define Q38_GDN_ARRIVALS 16

/* Chunked Gated-DeltaNet prefill (chunk Q38_GDN_CHUNK tokens).  The prep
 * kernel (grid (48 value heads, n_chunks, n_seq)) writes one record per head
 * and chunk to `work`: a bf16 hi/lo image of the scan's operands laid out as
 * the scan's LDS, in three parts the scan fetches separately, each a
 * multiple of 4 KiB: W hi, W lo [64][136] + 2 KiB pad (36 KiB) | Q' hi, lo
 * [64][136], Bm hi, lo [64][72] (52 KiB) | K'^T hi, lo [128][72] (36 KiB) --
 * then U' f32 [64][128] and gamma_C; the
 * scan kernel (grid (48 x 4 row slabs, n_seq)) carries the state through the
 * chunks. */
#define Q38_GDN_CHUNK 64
#define Q38_GDN_WROW 136 /* bf16 per W / Q' image row: 128 + 16 B pad */
#define Q38_GDN_BROW 72  /* bf16 per Bm / K'^T image row: 64 + 16 B pad */
#define Q38_GDN_W_BYTES (36 * 1024)  /* W hi, lo + pad */
#define Q38_GDN_QB_BYTES (52 * 1024) /* Q' hi, lo, Bm hi, lo */
#define Q38_GDN_KT_BYTES (36 * 1024) /* K'^T hi, lo */
#define Q38_GDN_IMAGE_BYTES (Q38_GDN_W_BYTES + Q38_GDN_QB_BYTES + Q38_GDN_KT_BYTES)
#define Q38_GDN_RECORD_BYTES (Q38_GDN_IMAGE_BYTES + 64 * 128 * 4 + 256)
#define Q38_GDN_SCAN_WAVES 8 /* waves of a chunk-scan workgroup, two per SIMD */
typedef struct {
    float *state;      /* seq s at state + s*state_stride: [48][128][128] */
    const float *q;    /* token (s*T + t): q + (s*T + t)*q_stride + kh*128 */
    const float *k;
    const float *v;    /* v + (s*T + t)*v_stride + vh*128 */
    const float *beta; /* [(s*T + t)*48 + vh], post-sigmoid */
    const float *g;    /* log-decay, same layout */
    float *out;        /* [(s*T + t)*6144 + vh*128 + c], before the gated norm */
    void *work;        /* [n_seq][48][n_chunks] records of Q38_GDN_RECORD_BYTES */
    int64_t state_stride;
    int32_t q_stride;
    int32_t v_stride;
    int32_t n_tokens;
    int32_t n_chunks;  /* chunks of this launch: chunk0 .. chunk0 + n_chunks - 1 */
    int32_t chunk0;
    int32_t pad_;
} q38_gdn_chunk_args;
/* chunks per prep/scan launch pair: a stage's records (16 x 48 x 158 KB, ~121 MB
 * per sequence) stay in the last-level cache between the two launches */
#define Q38_GDN_STAGE_CHUNKS 16

/* Gated RMSNorm of ops.rs:735-740 on [n][48][128] recurrence outputs:
 * grid (n_tokens * n_seq * 3), 256 threads, 16 rows per workgroup; every
 * pointer 16-byte aligned. */
typedef struct {
    const float *o;    /* [(s*T + t)*6144 + vh*128 + c] */
    const float *z;    /* same layout */
    const float *norm_w; /* [128] */
    float *out;
} q38_gdn_post_args;

/* conv1d(k=4) with state shift, SiLU, per-head L2 norm of q and k, and the
 * beta / decay gates, for n_tokens consecutive tokens of n_seq sequences.
 * grid (11, ceil(n_tokens / Q38_GDN_PRE_TOKENS), n_seq), 256 threads: x < 10
 * is a 1024-channel group, x == 10 the gates, y a run of Q38_GDN_PRE_TOKENS
 * tokens.  qkv_raw, conv_state_in and conv_state_out 16-byte aligned. */
#define Q38_GDN_PRE_TOKENS 8
typedef struct {
    const float *qkv_raw;   /* [(s*T + t)*10240] */
    const float *conv_w;    /* [10240][4] */
    const float *conv_state_in;  /* seq s at + s*30720: [10240][3] */
    float *conv_state_out;       /* may equal conv_state_in when T == 1 */
    float *qkv_out;         /* [(s*T + t)*10240]: q | k | v after conv, SiLU, L2 */
    const float *beta_raw;  /* [(s*T + t)*48] */
    const float *alpha_raw;
    const float *dt;        /* [48] */
    const float *a;         /* [48] */
    float *beta_out;        /* sigmoid(beta) */
    float *g_out;           /* a * softplus(alpha + dt) */
    int32_t n_tokens;
    int32_t n_seq;
} q38_gdn_pre_args;

/* Causal prefill attention of one sequence on bf16 MFMA.  grid
 * (12 * n_qblocks), 4 waves: a workgroup serves Q38_PREFILL_QUERIES query
 * tokens of 2 of the 6 query heads of one kv head (3 head pairs per kv
 * head), one wave per 32 tokens x 1 head. */
#define Q38_PREFILL_KEYS 32    /* keys per K/V block */
#define Q38_PREFILL_QUERIES 64 /* query tokens per prefill workgroup */
#define Q38_PREFILL_HEAD_PAIRS 3
#define Q38_PREFILL_BINS 64     /* workgroups per kv head when the host places the jobs */
#define Q38_PREFILL_JOBS_MAX 4  /* jobs per such workgroup */
#define Q38_PREFILL_SPLITS_MAX (3 * 64) /* jobs split into pieces in one launch */
/* One placed job: head pair << 6 | query block (0xFFFF: none), its key
 * blocks [kb0, kb1), and the partial slot its piece writes (0xFFFF: the
 * whole job, normalised and stored).  Key-block indices are 32-bit: a
 * sequence may hold up to 16,777,216 tokens, 524,288 blocks of 32 keys. */
typedef struct {
    uint16_t code;
    uint16_t slot;
    int32_t kb0;
    int32_t kb1;
} q38_prefill_job;
/* A job split into n pieces written to partial slots slot0 .. slot0+n-1. */
typedef struct {
    uint16_t code;
    uint16_t slot0;
    uint16_t n;
    uint16_t pad_;
} q38_prefill_split;
#define Q38_PREFILL_KROW 264  /* bf16 per K row in a block image (256 + 16 B pad) */
#define Q38_PREFILL_VROW 40   /* bf16 per transposed V row (32 key slots + 16 B pad) */
/* One K/V block of one kv head split into bf16 hi/lo, laid out exactly as
 * the prefill kernel's LDS tile: K hi [32][264] | K lo | V^T hi [256][40] |
 * V^T lo, 74,752 bytes. */
#define Q38_PREFILL_IMAGE_BYTES (2 * Q38_PREFILL_KEYS * Q38_PREFILL_KROW * 2 + 2 * 256 * Q38_PREFILL_VROW * 2)
typedef struct {
    const float *kpool;        /* this layer's K pages: [max_pages][4][16][256] */
    const float *vpool;
    const int32_t *page_table; /* the sequence's row of the page table */
    const float *q;            /* [n_tokens][24][256] for positions base_pos.. */
    const float *gate;         /* [n_tokens][24][256] or NULL */
    float *out;                /* [n_tokens][24][256] */
    void *images;              /* [4 kv heads][img_stride] block images */
    int32_t base_pos;
    int32_t n_tokens;
    int32_t n_qblocks;
    int32_t n_kblocks;         /* blocks of keys 0 .. base_pos + n_tokens - 1 */
    /* 0: grid (12 * n_qblocks), one (kv head, head pair, query block) job per
     * workgroup over all its key blocks.  Else grid (4 * Q38_PREFILL_BINS):
     * workgroup L serves kv head (L % 8) / 2 and runs the jobs of bin
     * 2 (L / 8) + L % 2, job i of bin b at jobs[b * jobs_per_wg + i];
     * n_qblocks <= 64. */
    int32_t jobs_per_wg;
    int32_t n_slots;           /* partial slots per kv head (pieces of split jobs) */
    int32_t img_stride;        /* blocks per kv head in `images` (>= n_kblocks) */
    int32_t kb0;               /* q38_kv_split_mfma converts blocks kb0 .. n_kblocks-1 */
    float *part_o;             /* [4][n_slots][64 rows][2 heads][256] unnormalised O of a piece */
    float *part_ml;            /* [4][n_slots][64][2][2]: its (reference, weight sum) per row */
    q38_prefill_job jobs[Q38_PREFILL_BINS * Q38_PREFILL_JOBS_MAX];
} q38_prefill_args;

/* Combines the pieces of split prefill jobs: grid (n_split, 4 kv heads, 32),
 * 256 threads; workgroup (g, j, y) forms rows/heads 4y .. 4y+3 of split job
 * g of kv head j, a thread 4 output dims of one (row, head). */
typedef struct {
    const float *part_o;
    const float *part_ml;
    const float *gate;
    float *out;
    int32_t n_tokens;
    int32_t n_slots;
    int32_t n_split;
    int32_t pad_;
    q38_prefill_split split[Q38_PREFILL_SPLITS_MAX];
} q38_prefill_merge_args;

/* Weight projections.  Q8_K activations are planar: for T tokens of width
 * W (B = W/256 blocks each) int8 quants [T][W] | int16 group sums [T][B][16]
 * | f32 scales [T][B] -- Q38_Q8K_BYTES(T, W) bytes. */
#define Q38_Q8K_BLOCK 256
#define Q38_Q8K_BYTES(T, W) ((size_t)(T) * ((W) / Q38_Q8K_BLOCK) * (Q38_Q8K_BLOCK + 32 + 4))
#define Q38_GGML_F32 0
#define Q38_GGML_F16 1
#define Q38_GGML_Q8_0 8
#define Q38_GGML_Q2_K 10
#define Q38_GGML_Q3_K 11
#define Q38_GGML_IQ4_NL 20
#define Q38_GGML_Q4_K 12
#define Q38_GGML_Q5_K 13
#define Q38_GGML_Q6_K 14
#define Q38_GGML_IQ4_XS 23
#define Q38_GGML_IQ2_XXS 16
#define Q38_GGML_IQ2_XS 17
#define Q38_GGML_IQ3_XXS 18
#define Q38_GGML_IQ1_S 19
#define Q38_GGML_IQ3_S 21
#define Q38_GGML_IQ2_S 22
#define Q38_GGML_IQ1_M 29
#define Q38_GGML_BF16 30
#define Q38_GEMV_TOKENS 8 /* most tokens one GEMV workgroup serves per pass over its weights */
#define Q38_GEMV_MAX_BLOCKS 192 /* 256-wide blocks per row (width 49152): one token's blocks fit LDS */
#define Q38_GEMV_UNITS_MAX 1024 /* (row, block) units per GEMV workgroup: four steps of 256 */
#define Q38_GEMV_REC_BYTES (272 + 32 + 4) /* LDS bytes of one staged Q8_K block: padded quants, sums, scale */
#define Q38_GEMV_ACT_LDS (64 * 1024) /* LDS for staged activations when tokens > 1 */

/* quantize_q8_k: grid (ceil(B / 16), T), 256 threads (16 per block). */
typedef struct {
    const float *x; /* [T][W] */
    void *q8k;      /* planar, Q38_Q8K_BYTES(T, W) */
    int32_t width;
    int32_t n_tokens;
} q38_quantize_args;

/* K-quant x Q8_K GEMV / GEMM over up to Q38_GEMV_MAX_MATS matrices of one
 * type and width that read the same activations: G = wg_begin[n_mats] row
 * groups times P = tok_groups = ceil(T / tok_pass) token passes, 256
 * threads, one lane per (row, block) unit; matrix i takes row groups
 * wg_begin[i] .. wg_begin[i+1]-1, rows_per_wg[i] * B <= Q38_GEMV_UNITS_MAX;
 * dynamic LDS tok_pass * B * Q38_GEMV_REC_BYTES + tok_pass *
 * max_i(rows_per_wg[i]) * B * 4 bytes.  One token pass (P == 1): grid (G).
 * Several: grid (8 * P * ceil(G / 8)), workgroup L serving pass (L / 8) % P
 * of row group 8 (L / (8 P)) + L % 8 (none past G), so the passes of a row
 * group are dispatched together onto one XCD and share its L2. */
#define Q38_GEMV_MAX_MATS 4
/* From this many tokens the projections may run on the int8 matrix unit
 * (q38_gemm_q8k_*: grid (ceil(rows / 128), ceil(T / 64)), 256 threads, the
 * same arguments with one matrix); IQ4_NL, which has only that form, from
 * Q38_GEMM_IQ4NL_MIN_TOKENS (half as many for matrices of 8192+ rows). */
#define Q38_GEMM_MIN_TOKENS 8
#define Q38_GEMM_IQ4NL_MIN_TOKENS 32
#define Q38_GEMM_ROWS 128
#define Q38_GEMM_TOKENS 64
/* Where that grid holds few workgroups (few rows or tokens), the blocks of a
 * row are split over the waves instead (q38_gemm_ks_q8k_*: grid (ceil(rows /
 * 32), ceil(T / 32)), Q38_GEMM_KS_WAVES waves of 64 threads, the same
 * arguments with one matrix). */
#define Q38_GEMM_KS_ROWS 32
#define Q38_GEMM_KS_TOKENS 32
#define Q38_GEMM_KS_WAVES 8
/* ... 16 waves (q38_gemm_ks16_q8k_*, 1024 threads, one workgroup per CU)
 * where that grid has at most one workgroup per CU, and 4 waves
 * (q38_gemm_ks4_q8k_*, 256 threads) where it has more than 1.5 */
#define Q38_GEMM_KS_WAVES_WIDE 16
#define Q38_GEMM_KS_WAVES_NARROW 4
typedef struct {
    const uint8_t *weights[Q38_GEMV_MAX_MATS]; /* [rows][B * block_bytes], 16-byte aligned */
    float *out[Q38_GEMV_MAX_MATS];             /* [T][rows] */
    int32_t rows[Q38_GEMV_MAX_MATS];
    int32_t rows_per_wg[Q38_GEMV_MAX_MATS];
    int32_t wg_begin[Q38_GEMV_MAX_MATS + 1];
    int32_t n_mats;
    const void *q8k; /* planar Q8_K of T tokens */
    /* GEMV only: when set, the f32 input [T][width] -- each workgroup
     * quantises the tokens of its pass itself, and the first row group of
     * each pass also writes them to q8k */
    const float *x;
    int32_t width;
    int32_t n_tokens;
    int32_t tok_pass;
    int32_t tok_groups;
} q38_gemv_args;

/* f32-input projections (F32, F16, BF16, Q8_0 weights): the GEMV, grid
 * (ceil(rows / 4), ceil(T / Q38_GEMV_TOKENS)), 256 threads, one wave per
 * row; the bf16 matrix-unit forms (width a multiple of Q38_GEMM_F32_K):
 * q38_gemm_f32_*, grid (ceil(rows / Q38_GEMM_F32_ROWS), ceil(T /
 * Q38_GEMM_F32_TOKENS)), q38_gemm_f32w_*, the same with
 * Q38_GEMM_F32_WIDE_TOKENS tokens per workgroup, and q38_gemm_f32s_*, grid
 * (ceil(rows / 64), ceil(T / 32)), 256 threads. */
#define Q38_GEMM_F32_ROWS 128
#define Q38_GEMM_F32_TOKENS 64
#define Q38_GEMM_F32_WIDE_TOKENS 128
#define Q38_GEMM_F32_K 64
/* q38_gemv_f32_q8_0s_r{RW}_t{TP} (Q8_0 weights, few tokens): grid
 * (ceil(rows / (4 RW)), ceil(T / TP)), 256 threads; (RW, TP) one of (2, 1),
 * (2, 2), (2, 4), (4, 8) */
typedef struct {
    const uint8_t *weights; /* [rows][row_bytes], 4-byte aligned (16 for F32/F16/BF16) */
    const float *x;         /* [T][width], 16-byte aligned */
    float *out;             /* [T][rows] */
    int64_t row_bytes;
    int32_t rows;
    int32_t width;
    int32_t n_tokens;
    int32_t pad_;
} q38_gemv_f32_args;

/* Merge of split-K partials.  grid (n_seq, 24, 4). */
typedef struct {
    const float *part_o;
    const float *part_ml;
    const float *gate;
    float *out;
    int32_t n_seq;
    int32_t gate_head_stride; /* floats between heads' gates: 256, or 512 in q|gate rows */
    int32_t split_base[Q38_MAX_BATCH + 1];
} q38_merge_args;

#endif
