/*
 * Gated DeltaNet (gfx950, wave64).
 *
 * Reference semantics: linear_core, src/model/ops.rs:648-742.
 *
 * q38_gdn_recurrent -- the delta-rule recurrence (ops.rs:698-714): for value
 * head vh (key head vh % 16) and each state row c:
 *     S_c *= exp(g);  pred = S_c.k;  delta = (v_c - pred) * beta;
 *     S_c += k * delta;  o_c = (S_c.q) / sqrt(128)
 * Rows are independent given (q, k, v_c, beta, g).  One workgroup owns one
 * head of one sequence: 512 threads, 16 lanes per row, 4 rows per 16-lane
 * group, lane i holding columns 4i..4i+3 and 64+4i..64+4i+3 of its rows in
 * VGPRs.  The state is read from HBM once, carried in registers through all
 * n_tokens tokens, and written back once: a decode step is n_tokens = 1, a
 * sequential prefill is the same code over the prompt.  Both 128-long dots
 * are 8 FMAs per lane plus a 4-step DPP row reduction (no LDS).  The next
 * token's q/k/v/beta/g are loaded while the current one computes.
 *
 * With z != NULL the gated RMSNorm of ops.rs:735-740 is fused as an epilogue:
 * the head's 128 outputs meet in LDS, one wave forms the f64 sum of squares.
 *
 * q38_gdn_pre -- conv1d (kernel 4) with state shift (ops.rs:665-675), SiLU
 * (:676), per-head L2 norm of q and k (:678-683) and the beta / decay gates
 * (:684-687).
 */
#include "q38_device.h"

namespace {

struct GdnTok {
    f32x4 k0, k1, q0, q1;
    f32x4 v; /* v for rows 4*grp .. 4*grp+3 */
    float beta, g;
};

Q38_DEV GdnTok gdn_load(const q38_gdn_args &a, size_t tok, int kh, int vh, int grp, int d0,
                        int d1) {
    GdnTok x;
    const float *kp = a.k + tok * a.q_stride + kh * Q38_LIN_HEAD_DIM;
    const float *qp = a.q + tok * a.q_stride + kh * Q38_LIN_HEAD_DIM;
    x.k0 = q38_ld4(kp + d0);
    x.k1 = q38_ld4(kp + d1);
    x.q0 = q38_ld4(qp + d0);
    x.q1 = q38_ld4(qp + d1);
    x.v = q38_ld4(a.v + tok * a.v_stride + vh * Q38_LIN_HEAD_DIM + 4 * grp);
    x.beta = a.beta[tok * Q38_LIN_V_HEADS + vh];
    x.g = a.g[tok * Q38_LIN_V_HEADS + vh];
    return x;
}

}  // namespace

extern "C" __global__ __launch_bounds__(512) void q38_gdn_recurrent(q38_gdn_args a) {
    __shared__ float o_lds[2][Q38_LIN_HEAD_DIM];
    const int vh = blockIdx.x;
    const int s = blockIdx.y;
    const int kh = vh % Q38_LIN_QK_HEADS;
    const int tid = threadIdx.x;
    const int grp = tid >> 4; /* 0..31: rows 4*grp .. 4*grp+3 */
    const int li = tid & 15;
    const int d0 = 4 * li;
    const int d1 = 64 + 4 * li;
    const float query_scale = 1.0f / sqrtf((float)Q38_LIN_HEAD_DIM);

    float *st = a.state + (size_t)s * a.state_stride + (size_t)vh * Q38_LIN_HEAD_DIM * Q38_LIN_HEAD_DIM;
    f32x4 S0[4], S1[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = 4 * grp + r;
        S0[r] = q38_ld4(st + row * Q38_LIN_HEAD_DIM + d0);
        S1[r] = q38_ld4(st + row * Q38_LIN_HEAD_DIM + d1);
    }

    const size_t tok0 = (size_t)s * a.n_tokens;
    GdnTok cur = gdn_load(a, tok0, kh, vh, grp, d0, d1);
    for (int t = 0; t < a.n_tokens; ++t) {
        const size_t tok = tok0 + t;
        GdnTok nxt = cur;
        if (t + 1 < a.n_tokens) nxt = gdn_load(a, tok + 1, kh, vh, grp, d0, d1);

        const float decay = expf(cur.g);
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            S0[r] *= decay;
            S1[r] *= decay;
            float pred = q38_dot4(S0[r], cur.k0, 0.0f);
            pred = q38_dot4(S1[r], cur.k1, pred);
            pred = q38_sum16(pred);
            const float delta = (cur.v[r] - pred) * cur.beta;
            S0[r] = q38_fma4(delta, cur.k0, S0[r]);
            S1[r] = q38_fma4(delta, cur.k1, S1[r]);
            float res = q38_dot4(S0[r], cur.q0, 0.0f);
            res = q38_dot4(S1[r], cur.q1, res);
            res = q38_sum16(res);
            o[r] = res * query_scale;
        }
        float *out_tok = a.out + tok * Q38_LIN_V_DIM + vh * Q38_LIN_HEAD_DIM;
        if (a.z == nullptr) {
            if (li == 0) q38_st4(out_tok + 4 * grp, f32x4{o[0], o[1], o[2], o[3]});
        } else {
            /* gated RMSNorm epilogue (ops.rs:735-740); double-buffered LDS so
             * one barrier per token suffices */
            float *ob = o_lds[t & 1];
            if (li == 0) q38_st4(ob + 4 * grp, f32x4{o[0], o[1], o[2], o[3]});
            __syncthreads();
            if (tid < 64) {
                const float x0 = ob[tid];
                const float x1 = ob[tid + 64];
                double ss = (double)x0 * (double)x0 + (double)x1 * (double)x1;
                ss = q38_wave_sum_f64(ss);
                const float mean = (float)(ss / (double)Q38_LIN_HEAD_DIM);
                const float scale = 1.0f / sqrtf(mean + 1e-6f);
                const float *zt = a.z + tok * Q38_LIN_V_DIM + vh * Q38_LIN_HEAD_DIM;
                float y0 = x0 * scale * a.norm_w[tid];
                float y1 = x1 * scale * a.norm_w[tid + 64];
                y0 *= q38_silu(zt[tid]);
                y1 *= q38_silu(zt[tid + 64]);
                out_tok[tid] = y0;
                out_tok[tid + 64] = y1;
            }
        }
        cur = nxt;
    }

#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = 4 * grp + r;
        q38_st4(st + row * Q38_LIN_HEAD_DIM + d0, S0[r]);
        q38_st4(st + row * Q38_LIN_HEAD_DIM + d1, S1[r]);
    }
}

/* grid (81, n_chunks, n_seq), 128 threads.  x < 80: channels 128x..128x+127
 * (x < 16 the q heads, 16 <= x < 32 the k heads, then v) for tokens
 * 64y..64y+63; x == 80: the gates of those tokens.  Each thread rebuilds its
 * channel's 3-tap window from the raw inputs of the three previous tokens (or
 * from conv_state_in before the first token), so chunks are independent; the
 * chunk holding the last token writes the shifted state to conv_state_out,
 * which must differ from conv_state_in when there is more than one chunk. */
extern "C" __global__ __launch_bounds__(128) void q38_gdn_pre(q38_gdn_pre_args a) {
    __shared__ double red[2][2];
    const int gx = blockIdx.x;
    const int chunk = blockIdx.y;
    const int s = blockIdx.z;
    const int tid = threadIdx.x;
    const int T = a.n_tokens;
    const int t0 = chunk * 64;
    const int t1 = min(T, t0 + 64);
    const size_t tok0 = (size_t)s * T;

    if (gx == 80) {
        for (int i = tid; i < (t1 - t0) * Q38_LIN_V_HEADS; i += 128) {
            const int t = t0 + i / Q38_LIN_V_HEADS;
            const int h = i % Q38_LIN_V_HEADS;
            const size_t at = (tok0 + t) * Q38_LIN_V_HEADS + h;
            a.beta_out[at] = q38_sigmoid(a.beta_raw[at]);
            a.g_out[at] = a.a[h] * q38_softplus(a.alpha_raw[at] + a.dt[h]);
        }
        return;
    }

    const int c = gx * 128 + tid;
    const float w0 = a.conv_w[(size_t)c * 4 + 0];
    const float w1 = a.conv_w[(size_t)c * 4 + 1];
    const float w2 = a.conv_w[(size_t)c * 4 + 2];
    const float w3 = a.conv_w[(size_t)c * 4 + 3];
    const float *st_in = a.conv_state_in + (size_t)s * Q38_LIN_QKV_DIM * 3 + (size_t)c * 3;
    /* window of the three raw inputs before t0: x_{t0-3}, x_{t0-2}, x_{t0-1} */
    float win[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int tp = t0 - 3 + i;
        win[i] = tp < 0 ? st_in[tp + 3] : a.qkv_raw[(tok0 + tp) * Q38_LIN_QKV_DIM + c];
    }
    const bool normed = gx < 32;
    const int wave = tid >> 6;
    for (int t = t0; t < t1; ++t) {
        const float x = a.qkv_raw[(tok0 + t) * Q38_LIN_QKV_DIM + c];
        float y = win[0] * w0;
        y += win[1] * w1;
        y += win[2] * w2;
        y += x * w3;
        win[0] = win[1];
        win[1] = win[2];
        win[2] = x;
        y = q38_silu(y);
        if (normed) {
            /* l2norm (ops.rs:562-571): f64 sum, f32 sqrt, floor 1e-6 */
            double ss = q38_wave_sum_f64((double)y * (double)y);
            if ((tid & 63) == 0) red[t & 1][wave] = ss;
            __syncthreads();
            const double sum = red[t & 1][0] + red[t & 1][1];
            float norm = sqrtf((float)sum);
            norm = fmaxf(norm, 1e-6f);
            y *= 1.0f / norm;
        }
        a.qkv_out[(tok0 + t) * Q38_LIN_QKV_DIM + c] = y;
    }
    if (t1 == T) {
        float *st_out = a.conv_state_out + (size_t)s * Q38_LIN_QKV_DIM * 3 + (size_t)c * 3;
        st_out[0] = win[0];
        st_out[1] = win[1];
        st_out[2] = win[2];
    }
}

/* One recurrent step (n_tokens == 1) spread over the whole chip: the 128
 * rows of a value head are independent (ops.rs:707-713 touches row c only
 * through k, q, v_c, beta and the decay), so a workgroup takes 16 rows of
 * one head -- grid (48 heads x 8 row blocks, n_seq), 256 threads, 16 lanes
 * per row, lane i holding columns 4i..4i+3 and 64+4i..64+4i+3.  Every load
 * of a thread (its 8 state values, k, q, v_c, beta, g) is issued at once,
 * so the step costs one memory round trip; the state is read and written
 * exactly once.  Arithmetic per row is the same as q38_gdn_recurrent's. */
extern "C" __global__ __launch_bounds__(256) void q38_gdn_step_rows(q38_gdn_args a) {
    constexpr int kRowBlocks = Q38_LIN_HEAD_DIM / 16;
    const int vh = blockIdx.x / kRowBlocks;
    const int rb = blockIdx.x % kRowBlocks;
    const size_t s = blockIdx.y;
    const int kh = vh % Q38_LIN_QK_HEADS;
    const int tid = threadIdx.x;
    const int row = rb * 16 + (tid >> 4);
    const int li = tid & 15;
    const int d0 = 4 * li;
    const int d1 = 64 + 4 * li;
    const float query_scale = 1.0f / sqrtf((float)Q38_LIN_HEAD_DIM);

    float *st = a.state + s * a.state_stride + ((size_t)vh * Q38_LIN_HEAD_DIM + row) * Q38_LIN_HEAD_DIM;
    f32x4 S0 = q38_ld4_stream(st + d0);
    f32x4 S1 = q38_ld4_stream(st + d1);
    const float *kp = a.k + s * a.q_stride + kh * Q38_LIN_HEAD_DIM;
    const float *qp = a.q + s * a.q_stride + kh * Q38_LIN_HEAD_DIM;
    const f32x4 k0 = q38_ld4(kp + d0), k1 = q38_ld4(kp + d1);
    const f32x4 q0 = q38_ld4(qp + d0), q1 = q38_ld4(qp + d1);
    const float v = a.v[s * a.v_stride + vh * Q38_LIN_HEAD_DIM + row];
    const float beta = a.beta[s * Q38_LIN_V_HEADS + vh];
    const float decay = expf(a.g[s * Q38_LIN_V_HEADS + vh]);

    S0 *= decay;
    S1 *= decay;
    float pred = q38_dot4(S0, k0, 0.0f);
    pred = q38_dot4(S1, k1, pred);
    pred = q38_sum16(pred);
    const float delta = (v - pred) * beta;
    S0 = q38_fma4(delta, k0, S0);
    S1 = q38_fma4(delta, k1, S1);
    float res = q38_dot4(S0, q0, 0.0f);
    res = q38_dot4(S1, q1, res);
    res = q38_sum16(res);
    q38_st4_stream(st + d0, S0);
    q38_st4_stream(st + d1, S1);
    if (li == 0) a.out[s * Q38_LIN_V_DIM + vh * Q38_LIN_HEAD_DIM + row] = res * query_scale;
}
