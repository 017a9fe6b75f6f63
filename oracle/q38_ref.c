/*
 * q38_ref.c -- CPU restatement of the reference engine's attention path.
 *
 * TEST INFRASTRUCTURE ONLY: the oracle for the HIP kernels and the CPU
 * baseline timed beside them.  The product library never links or calls it.
 *
 * Each function cites the reference function it restates
 * (src/model/ops.rs of StepfenShawn/qwen3.8_27b_in_rust).  Build with
 * -ffp-contract=off: the reference's Rust never fuses a multiply and an add
 * unless it calls mul_add, which is fmaf() here.
 */
#define _GNU_SOURCE
#include "q38_ref.h"

/* Q38R_MUTANT > 0 plants one known mistake (tests/test_oracle_mutants.py
 * builds each and checks that the fixtures and closed forms reject it).
 * The oracle itself is built with Q38R_MUTANT 0. */
#ifndef Q38R_MUTANT
#define Q38R_MUTANT 0
#endif

#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- primitives */

/* ops.rs:476-483 -- f64 sum of squares, mean rounded to f32, 1/sqrt(mean+eps). */
float q38r_rms_scale(const float *values, int length) {
    double sum = 0.0;
    for (int i = 0; i < length; ++i) sum += (double)values[i] * (double)values[i];
    float mean = (float)(sum / (double)length);
#if Q38R_MUTANT == 8
    return 1.0f / sqrtf(mean);
#endif
    return 1.0f / sqrtf(mean + Q38R_RMS_EPS);
}

/* ops.rs:493-498 -- values[i] * scale * weight[i], left to right. */
void q38r_rmsnorm_inplace(float *values, const float *weight, int n) {
    float scale = q38r_rms_scale(values, n);
    for (int i = 0; i < n; ++i) values[i] = values[i] * scale * weight[i];
}

/* ops.rs:501-503 */
float q38r_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* ops.rs:506-508 */
float q38r_silu(float x) { return x / (1.0f + expf(-x)); }

/* ops.rs:511-516 -- identity above 20. */
float q38r_softplus(float x) {
#if Q38R_MUTANT != 7
    if (x > 20.0f) return x;
#endif
    return logf(1.0f + expf(x));
}

/* ops.rs:562-571 -- f64 sum, f32 sqrt, floor 1e-6, then scale. */
void q38r_l2norm(float *values, int length) {
    double sum = 0.0;
    for (int i = 0; i < length; ++i) sum += (double)values[i] * (double)values[i];
    float norm = sqrtf((float)sum);
#if Q38R_MUTANT != 6
    if (norm < Q38R_RMS_EPS) norm = Q38R_RMS_EPS;
#endif
    float scale = 1.0f / norm;
    for (int i = 0; i < length; ++i) values[i] *= scale;
}

/* ops.rs:573-579 -- sequential mul_add chain from 0. */
float q38r_dot_128(const float *left, const float *right) {
    float total = 0.0f;
    for (int i = 0; i < Q38R_LINEAR_HEAD_DIM; ++i) total = fmaf(left[i], right[i], total);
    return total;
}

/* ops.rs:584-591 -- output += input*scale (fused), dot of the new output. */
float q38r_mad_dot_128(float *output, const float *input, float scale, const float *right) {
    float total = 0.0f;
    for (int i = 0; i < Q38R_LINEAR_HEAD_DIM; ++i) {
        output[i] = fmaf(input[i], scale, output[i]);
        total = fmaf(output[i], right[i], total);
    }
    return total;
}

/* ops.rs:596 -- 1e7^(-2/64) in f32. */
float q38r_rope_theta_scale(void) { return powf(10000000.0f, -2.0f / 64.0f); }

/* ops.rs:595-610 -- lanes p and p+32 (p < 32) rotate by theta_p; theta starts
 * at the position and is multiplied by the scale after every pair, in f32. */
void q38r_rope(float *values, int heads, uint32_t position) {
    const float theta_scale = q38r_rope_theta_scale();
    for (int head = 0; head < heads; ++head) {
        float *vector = values + (size_t)head * Q38R_ATTN_HEAD_DIM;
        float theta = (float)position;
        for (int pair = 0; pair < 32; ++pair) {
#if Q38R_MUTANT == 3
            theta = (float)position * powf(theta_scale, (float)pair);
#endif
            float cosine = cosf(theta);
            float sine = sinf(theta);
            float x0 = vector[pair];
            float x1 = vector[pair + 32];
            vector[pair] = x0 * cosine - x1 * sine;
            vector[pair + 32] = x0 * sine + x1 * cosine;
            theta *= theta_scale;
        }
    }
}

/* ---------------------------------------------------- head-parallel dispatch */

/* The reference fans heads out over rayon when q38_parallel_over says so
 * (kernel/mod.rs:15-17).  Per-head work is serial, so any split of the heads
 * over threads gives bit-identical results; a static block split is used. */
typedef void (*q38r_head_fn)(void *arg, int head);

typedef struct {
    q38r_head_fn fn;
    void *arg;
    int begin, end;
} q38r_span;

static void *q38r_run_span(void *p) {
    q38r_span *s = (q38r_span *)p;
    for (int h = s->begin; h < s->end; ++h) s->fn(s->arg, h);
    return NULL;
}

static void q38r_parallel_heads(int heads, int n_threads, q38r_head_fn fn, void *arg) {
    if (n_threads > heads) n_threads = heads;
    if (n_threads <= 1) {
        for (int h = 0; h < heads; ++h) fn(arg, h);
        return;
    }
    pthread_t tids[256];
    q38r_span spans[256];
    if (n_threads > 256) n_threads = 256;
    int started = 0;
    for (int t = 0; t < n_threads; ++t) {
        spans[t].fn = fn;
        spans[t].arg = arg;
        spans[t].begin = (int)((long)heads * t / n_threads);
        spans[t].end = (int)((long)heads * (t + 1) / n_threads);
        if (t == 0) continue; /* the calling thread takes span 0 */
        if (pthread_create(&tids[t], NULL, q38r_run_span, &spans[t]) != 0) {
            /* could not start a worker: run its span here instead */
            q38r_run_span(&spans[t]);
            tids[t] = 0;
        } else {
            ++started;
        }
    }
    q38r_run_span(&spans[0]);
    for (int t = 1; t < n_threads; ++t)
        if (tids[t]) pthread_join(tids[t], NULL);
    (void)started;
}

/* kernel/mod.rs:5-17 */
static int q38r_parallel_over(size_t items, size_t per_item) {
    return items >= 2 && items * per_item >= ((size_t)1 << 18);
}

/* ----------------------------------------------------------- full attention */

typedef struct {
    const float *q, *gate, *key_rows, *value_rows;
    size_t row_stride;
    int positions;
    float *scores, *out;
} q38r_attn_args;

/* ops.rs:879-918 -- one query head: scores, max, exp, sequential sum, then
 * the probability-weighted sum of value rows and the sigmoid gate. */
static void q38r_attn_run_head(void *p, int head) {
    const q38r_attn_args *a = (const q38r_attn_args *)p;
    const int groups = Q38R_ATTN_HEADS / Q38R_ATTN_KV_HEADS;
#if Q38R_MUTANT == 1
    const int kv_head = head % Q38R_ATTN_KV_HEADS;
    (void)groups;
#else
    const int kv_head = head / groups;
#endif
#if Q38R_MUTANT == 5
    const float score_scale = 1.0f;
#else
    const float score_scale = 1.0f / sqrtf((float)Q38R_ATTN_HEAD_DIM);
#endif
    const float *q_head = a->q + (size_t)head * Q38R_ATTN_HEAD_DIM;
    float *head_scores = a->scores + (size_t)head * a->positions;
    float *head_output = a->out + (size_t)head * Q38R_ATTN_HEAD_DIM;

    float maximum = -INFINITY;
    for (int position = 0; position < a->positions; ++position) {
        const float *k = a->key_rows + (size_t)position * a->row_stride +
                         (size_t)kv_head * Q38R_ATTN_HEAD_DIM;
        float score = 0.0f;
        for (int i = 0; i < Q38R_ATTN_HEAD_DIM; ++i) score = fmaf(q_head[i], k[i], score);
        score *= score_scale;
        head_scores[position] = score;
        if (score > maximum) maximum = score;
    }
    float denominator = 0.0f;
    for (int position = 0; position < a->positions; ++position) {
        head_scores[position] = expf(head_scores[position] - maximum);
        denominator += head_scores[position];
    }
    for (int i = 0; i < Q38R_ATTN_HEAD_DIM; ++i) head_output[i] = 0.0f;
    for (int position = 0; position < a->positions; ++position) {
        const float *v = a->value_rows + (size_t)position * a->row_stride +
                         (size_t)kv_head * Q38R_ATTN_HEAD_DIM;
        float probability = head_scores[position] / denominator;
        for (int i = 0; i < Q38R_ATTN_HEAD_DIM; ++i)
            head_output[i] = fmaf(probability, v[i], head_output[i]);
    }
    if (a->gate) {
        const float *head_gate = a->gate + (size_t)head * Q38R_ATTN_HEAD_DIM;
#if Q38R_MUTANT == 10
        for (int i = 0; i < Q38R_ATTN_HEAD_DIM; ++i) head_output[i] *= q38r_silu(head_gate[i]);
#else
        for (int i = 0; i < Q38R_ATTN_HEAD_DIM; ++i) head_output[i] *= q38r_sigmoid(head_gate[i]);
#endif
    }
}

/* ops.rs:868-938 */
void q38r_attn_heads(const float *q, const float *gate, const float *key_rows,
                     const float *value_rows, size_t row_stride, int positions, float *scores,
                     float *out, int n_threads) {
    q38r_attn_args a = {q, gate, key_rows, value_rows, row_stride, positions, scores, out};
    size_t work = (size_t)positions * Q38R_ATTN_HEAD_DIM;
    int threads = q38r_parallel_over(Q38R_ATTN_HEADS, work) ? n_threads : 1;
    q38r_parallel_heads(Q38R_ATTN_HEADS, threads, q38r_attn_run_head, &a);
}

/* ops.rs:813-940 */
int q38r_full_core(const float *q_norm, const float *k_norm, const float *q_and_gate,
                   float *key, const float *value, float *q, float *gate, float *scores,
                   float *attention, float *key_cache, float *value_cache,
                   size_t cache_len_floats, size_t context_length, uint32_t current_position,
                   int layer, int n_threads) {
    for (int head = 0; head < Q38R_ATTN_HEADS; ++head) {
        const float *source = q_and_gate + (size_t)head * 2 * Q38R_ATTN_HEAD_DIM;
        memcpy(q + (size_t)head * Q38R_ATTN_HEAD_DIM, source, Q38R_ATTN_HEAD_DIM * sizeof(float));
        memcpy(gate + (size_t)head * Q38R_ATTN_HEAD_DIM, source + Q38R_ATTN_HEAD_DIM,
               Q38R_ATTN_HEAD_DIM * sizeof(float));
        q38r_rmsnorm_inplace(q + (size_t)head * Q38R_ATTN_HEAD_DIM, q_norm, Q38R_ATTN_HEAD_DIM);
    }
    for (int head = 0; head < Q38R_ATTN_KV_HEADS; ++head)
        q38r_rmsnorm_inplace(key + (size_t)head * Q38R_ATTN_HEAD_DIM, k_norm, Q38R_ATTN_HEAD_DIM);
    q38r_rope(q, Q38R_ATTN_HEADS, current_position);
    q38r_rope(key, Q38R_ATTN_KV_HEADS, current_position);

    size_t full_index = (size_t)layer / 4;
    size_t cache_row = (full_index * context_length + current_position) * Q38R_ATTN_KV_DIM;
    if (cache_row + Q38R_ATTN_KV_DIM > cache_len_floats) return -1;
    memcpy(key_cache + cache_row, key, Q38R_ATTN_KV_DIM * sizeof(float));
    memcpy(value_cache + cache_row, value, Q38R_ATTN_KV_DIM * sizeof(float));

    const float *rows_k = key_cache + full_index * context_length * Q38R_ATTN_KV_DIM;
    const float *rows_v = value_cache + full_index * context_length * Q38R_ATTN_KV_DIM;
    q38r_attn_heads(q, gate, rows_k, rows_v, Q38R_ATTN_KV_DIM, (int)current_position + 1,
                    scores, attention, n_threads);
    return 0;
}

/* ------------------------------------------------------------ Gated DeltaNet */

typedef struct {
    float *state;
    const float *q, *k, *v, *beta, *g;
    float *out;
} q38r_gdn_args;

/* ops.rs:698-714 -- decay the whole head state first, then per row c: the
 * prediction, the delta, and the fused update + readout. */
static void q38r_gdn_run_head(void *p, int value_head) {
    const q38r_gdn_args *a = (const q38r_gdn_args *)p;
    const int D = Q38R_LINEAR_HEAD_DIM;
#if Q38R_MUTANT == 12
    const float query_scale = 1.0f;
#else
    const float query_scale = 1.0f / sqrtf((float)D);
#endif
#if Q38R_MUTANT == 2
    const int key_head = value_head / 3;
#else
    const int key_head = value_head % Q38R_LINEAR_QK_HEADS;
#endif
    const float *query_head = a->q + (size_t)key_head * D;
    const float *key_vec = a->k + (size_t)key_head * D;
    const float *value_vec = a->v + (size_t)value_head * D;
    float *state = a->state + (size_t)value_head * D * D;
    float *head_output = a->out + (size_t)value_head * D;

    float decay = expf(a->g[value_head]);
#if Q38R_MUTANT != 4
    for (int e = 0; e < D * D; ++e) state[e] *= decay;
#endif
    for (int column = 0; column < D; ++column) {
        float *state_column = state + (size_t)column * D;
        float prediction = q38r_dot_128(state_column, key_vec);
#if Q38R_MUTANT == 4
        for (int i = 0; i < D; ++i) state_column[i] *= decay;
#endif
#if Q38R_MUTANT == 11
        float delta = (prediction - value_vec[column]) * a->beta[value_head];
#else
        float delta = (value_vec[column] - prediction) * a->beta[value_head];
#endif
        float result = q38r_mad_dot_128(state_column, key_vec, delta, query_head);
        head_output[column] = result * query_scale;
    }
}

/* ops.rs:689-733 */
void q38r_gdn_heads(float *state, const float *q, const float *k, const float *v,
                    const float *beta, const float *g, float *out, int n_threads) {
    q38r_gdn_args a = {state, q, k, v, beta, g, out};
    int threads = q38r_parallel_over(Q38R_LINEAR_V_HEADS,
                                     (size_t)Q38R_LINEAR_HEAD_DIM * Q38R_LINEAR_HEAD_DIM)
                      ? n_threads
                      : 1;
    q38r_parallel_heads(Q38R_LINEAR_V_HEADS, threads, q38r_gdn_run_head, &a);
}

/* ops.rs:648-742 */
void q38r_linear_core(const float *conv_w, const float *dt, const float *a,
                      const float *norm_w, float *conv_state, float *delta_state, float *qkv,
                      const float *z, float *beta, float *alpha, float *attention,
                      int n_threads) {
    /* ops.rs:665-675: separate multiplies and adds, then the state shift. */
    for (int channel = 0; channel < Q38R_LINEAR_QKV_DIM; ++channel) {
        float *state = conv_state + (size_t)channel * 3;
        const float *w = conv_w + (size_t)channel * 4;
#if Q38R_MUTANT == 9
        float value = state[0] * w[3];
        value += state[1] * w[2];
        value += state[2] * w[1];
        value += qkv[channel] * w[0];
#else
        float value = state[0] * w[0];
        value += state[1] * w[1];
        value += state[2] * w[2];
        value += qkv[channel] * w[3];
#endif
        state[0] = state[1];
        state[1] = state[2];
        state[2] = qkv[channel];
        qkv[channel] = value;
    }
    /* ops.rs:676 */
    for (int i = 0; i < Q38R_LINEAR_QKV_DIM; ++i) qkv[i] = q38r_silu(qkv[i]);
    /* ops.rs:678-683 */
    float *query = qkv;
    float *key = qkv + Q38R_LINEAR_QK_DIM;
    float *value = qkv + 2 * Q38R_LINEAR_QK_DIM;
    for (int head = 0; head < Q38R_LINEAR_QK_HEADS; ++head) {
        q38r_l2norm(query + (size_t)head * Q38R_LINEAR_HEAD_DIM, Q38R_LINEAR_HEAD_DIM);
        q38r_l2norm(key + (size_t)head * Q38R_LINEAR_HEAD_DIM, Q38R_LINEAR_HEAD_DIM);
    }
    /* ops.rs:684-687 */
    for (int head = 0; head < Q38R_LINEAR_V_HEADS; ++head) {
        beta[head] = q38r_sigmoid(beta[head]);
        alpha[head] = a[head] * q38r_softplus(alpha[head] + dt[head]);
    }
    /* ops.rs:689-733 */
    q38r_gdn_heads(delta_state, query, key, value, beta, alpha, attention, n_threads);
    /* ops.rs:735-740 */
    for (int value_head = 0; value_head < Q38R_LINEAR_V_HEADS; ++value_head) {
        float *head_output = attention + (size_t)value_head * Q38R_LINEAR_HEAD_DIM;
        q38r_rmsnorm_inplace(head_output, norm_w, Q38R_LINEAR_HEAD_DIM);
        const float *gate = z + (size_t)value_head * Q38R_LINEAR_HEAD_DIM;
        for (int i = 0; i < Q38R_LINEAR_HEAD_DIM; ++i) head_output[i] *= q38r_silu(gate[i]);
    }
}

/* ops.rs:38-47 (layer 64 is the MTP block, a full-attention layer) */
int q38r_is_full_attention(int layer) { return (layer + 1) % 4 == 0 || layer == 64; }
int q38r_recurrent_index(int layer) { return layer - (layer + 1) / 4; }

int q38r_available_cores(void) {
    cpu_set_t set;
    CPU_ZERO(&set);
    if (sched_getaffinity(0, sizeof(set), &set) != 0) return 1;
    int n = CPU_COUNT(&set);
    return n > 0 ? n : 1;
}
