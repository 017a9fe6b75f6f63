/*
 * Gated DeltaNet (gfx950, wave64).
 *
 * Reference semantics: linear_core, src/model/ops.rs:648-742.
 *
 * q38_gdn_decode -- one linear_core token in one launch: conv1d, SiLU, L2
 * norms and gates, the delta-rule recurrence with readout, and the gated
 * RMSNorm, one workgroup per value head.
 *
 * q38_gdn_step_rows -- the recurrence alone, one token, 8 workgroups per
 * value head (the rows of a head are independent).
 *
 * q38_gdn_pre -- conv1d (kernel 4) with state shift (ops.rs:665-675), SiLU
 * (:676), per-head L2 norm of q and k (:678-683) and the beta / decay gates
 * (:684-687).
 */
#include "q38_device.h"

/* One linear_core token (ops.rs:648-742) in ONE launch: grid (48 value
 * heads, n_seq), Q38_GDN_DECODE_THREADS threads.  The workgroup of value head vh (key head kh =
 * vh % 16):
 *  1. issues the loads of its head's 128x128 state first (16 lanes per row,
 *     128 * 16 / threads rows per 16-lane group, lane i holding columns
 *     4i..4i+3 and 64+4i..64+4i+3), so the state streams in while the
 *     prologue runs;
 *  2. prologue (ops.rs:665-687): threads 0..383 take one channel each -- q
 *     and k of key head kh and v of value head vh -- conv1d over the 3-tap
 *     state and the raw input (separate multiplies and adds, left to right),
 *     SiLU, then the f64 L2 norm of q and k (waves 0-1 and 2-3); thread 384
 *     forms beta = sigmoid and g = a * softplus(alpha + dt);
 *  3. the recurrence of ops.rs:698-714 on the 128 rows in registers (decay,
 *     prediction, delta-rule update and readout; two 4-step DPP reductions
 *     per row), the new state streamed back with non-temporal stores;
 *  4. the gated RMSNorm of ops.rs:735-740 over the head's 128 outputs in LDS.
 * Conv state: the v channels of vh belong to this workgroup alone and are
 * shifted in place.  The q/k channels of kh are read by the three value
 * heads kh, kh+16, kh+32: each of their workgroups counts its arrival on
 * arrivals[s][kh] after its reads have been consumed, and the third to
 * arrive writes the shifted q/k state and resets the counter to zero for the
 * next call.  No workgroup waits on another.  The arithmetic is that of
 * q38_gdn_pre followed by the recurrence, operation for operation. */
/* 1024 threads (2 state rows per 16-lane group): 4.77 us per layer back to
 * back against 4.88 us with 512 (4 rows per group), the same results bit
 * for bit */
#ifndef Q38_GDN_DECODE_THREADS
#define Q38_GDN_DECODE_THREADS 1024
#endif
extern "C" __global__ __launch_bounds__(Q38_GDN_DECODE_THREADS) void q38_gdn_decode(q38_gdn_decode_args a) {
    /* state rows per 16-lane group */
    constexpr int R = Q38_LIN_HEAD_DIM * 16 / Q38_GDN_DECODE_THREADS;
    static_assert(R >= 1 && Q38_GDN_DECODE_THREADS >= 512, "at least 385 threads for the prologue");
    __shared__ __attribute__((aligned(16))) float xqkv[3][Q38_LIN_HEAD_DIM]; /* q, k (normed), v */
    __shared__ __attribute__((aligned(16))) float o_lds[Q38_LIN_HEAD_DIM];
    __shared__ double red[4];
    __shared__ float gates[2];
    __shared__ int last_arrival;
    const int vh = blockIdx.x;
    const size_t s = blockIdx.y;
    const int kh = vh % Q38_LIN_QK_HEADS;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int grp = tid >> 4; /* rows R*grp .. R*grp+R-1 */
    const int li = tid & 15;
    const int d0 = 4 * li;
    const int d1 = 64 + 4 * li;
    const float query_scale = 1.0f / sqrtf((float)Q38_LIN_HEAD_DIM);

    /* the prologue's loads first: one channel per thread (q, k of key head
     * kh, v of value head vh; thread 384 the gates) */
    const int part = tid >> 7; /* 0: q, 1: k, 2: v, 3: gates */
    const int ci = tid & 127;
    int c = 0;
    if (part == 0) c = kh * Q38_LIN_HEAD_DIM + ci;
    else if (part == 1) c = Q38_LIN_QK_DIM + kh * Q38_LIN_HEAD_DIM + ci;
    else if (part == 2) c = 2 * Q38_LIN_QK_DIM + vh * Q38_LIN_HEAD_DIM + ci;
    float *conv = a.conv_state + s * (Q38_LIN_QKV_DIM * 3) + (size_t)c * 3;
    f32x4 w = {0.f, 0.f, 0.f, 0.f};
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, x = 0.0f, g_beta = 0.0f, g_alpha = 0.0f;
    if (part < 3) {
        w = q38_ld4(a.conv_w + (size_t)c * 4);
        s0 = conv[0];
        s1 = conv[1];
        s2 = conv[2];
        x = a.qkv_raw[s * Q38_LIN_QKV_DIM + c];
    } else if (ci == 0) {
        g_beta = a.beta_raw[s * Q38_LIN_V_HEADS + vh];
        g_alpha = a.alpha_raw[s * Q38_LIN_V_HEADS + vh] + a.dt[vh];
        g_alpha = a.a[vh] * q38_softplus(g_alpha);
    }
    /* the epilogue's gate and norm weight (wave 0 forms the outputs) */
    float z0 = 0.0f, z1 = 0.0f, nw0 = 0.0f, nw1 = 0.0f;
    if (tid < 64) {
        const float *zt = a.z + s * Q38_LIN_V_DIM + vh * Q38_LIN_HEAD_DIM;
        z0 = zt[tid];
        z1 = zt[tid + 64];
        nw0 = a.norm_w[tid];
        nw1 = a.norm_w[tid + 64];
    }
    /* then the state, in flight while the prologue computes (the memory
     * counter is in issue order, so these stay outstanding) */
    float *st = a.state + s * Q38_LIN_STATE_FLOATS + (size_t)vh * Q38_LIN_HEAD_DIM * Q38_LIN_HEAD_DIM;
    f32x4 S0[R], S1[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = R * grp + r;
        S0[r] = q38_ld4_stream(st + row * Q38_LIN_HEAD_DIM + d0);
        S1[r] = q38_ld4_stream(st + row * Q38_LIN_HEAD_DIM + d1);
    }

    /* prologue (ops.rs:665-687) */
    float y = 0.0f;
    if (part < 3) {
        y = s0 * w.x;
        y += s1 * w.y;
        y += s2 * w.z;
        y += x * w.w;
        y = q38_silu(y);
    } else if (ci == 0) {
        gates[0] = q38_sigmoid(g_beta);
        gates[1] = g_alpha;
    }
    if (part < 2) {
        /* l2norm (ops.rs:562-571): f64 sum, f32 sqrt, floor 1e-6 */
        const double ss = q38_wave_sum_f64((double)y * (double)y);
        if (lane == 0) red[wave] = ss;
    }
    __syncthreads();
    if (part < 2) {
        const double sum = red[2 * part] + red[2 * part + 1];
        float norm = sqrtf((float)sum);
        norm = fmaxf(norm, 1e-6f);
        y *= 1.0f / norm;
    }
    if (part < 3) xqkv[part][ci] = y;
    if (part == 2) {
        /* this value head's own channels: shift in place */
        conv[0] = s1;
        conv[1] = s2;
        conv[2] = x;
    }
    __syncthreads();
    /* every q/k conv-state value this workgroup read has been consumed:
     * count the arrival now, use the count at the end (the atomic's round
     * trip overlaps the recurrence) */
    int before = 0;
    if (tid == 0) before = atomicAdd(&a.arrivals[s * Q38_GDN_ARRIVALS + kh], 1);

    /* 3. the recurrence (ops.rs:698-714) */
    const f32x4 k0 = q38_ld4(&xqkv[1][d0]), k1 = q38_ld4(&xqkv[1][d1]);
    const f32x4 q0 = q38_ld4(&xqkv[0][d0]), q1 = q38_ld4(&xqkv[0][d1]);
    float v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = xqkv[2][R * grp + r];
    const float beta = gates[0];
    const float decay = expf(gates[1]);
    float o[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        S0[r] *= decay;
        S1[r] *= decay;
        float pred = q38_dot4(S0[r], k0, 0.0f);
        pred = q38_dot4(S1[r], k1, pred);
        pred = q38_sum16(pred);
        const float delta = (v[r] - pred) * beta;
        S0[r] = q38_fma4(delta, k0, S0[r]);
        S1[r] = q38_fma4(delta, k1, S1[r]);
        float res = q38_dot4(S0[r], q0, 0.0f);
        res = q38_dot4(S1[r], q1, res);
        res = q38_sum16(res);
        o[r] = res * query_scale;
        const int row = R * grp + r;
        q38_st4_stream(st + row * Q38_LIN_HEAD_DIM + d0, S0[r]);
        q38_st4_stream(st + row * Q38_LIN_HEAD_DIM + d1, S1[r]);
    }

    /* 4. gated RMSNorm (ops.rs:735-740) */
    if (li == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) o_lds[R * grp + r] = o[r];
    }
    __syncthreads();
    if (tid < 64) {
        const float x0 = o_lds[tid];
        const float x1 = o_lds[tid + 64];
        double ss = (double)x0 * (double)x0 + (double)x1 * (double)x1;
        ss = q38_wave_sum_f64(ss);
        const float mean = (float)(ss / (double)Q38_LIN_HEAD_DIM);
        const float scale = 1.0f / sqrtf(mean + 1e-6f);
        float y0 = x0 * scale * nw0;
        float y1 = x1 * scale * nw1;
        y0 *= q38_silu(z0);
        y1 *= q38_silu(z1);
        float *out = a.out + s * Q38_LIN_V_DIM + vh * Q38_LIN_HEAD_DIM;
        out[tid] = y0;
        out[tid + 64] = y1;
        /* the count is first read here, so the wait for the atomic lands
         * here and not before the recurrence */
        asm volatile("" : "+v"(before));
        if (tid == 0) last_arrival = before == Q38_LIN_V_HEADS / Q38_LIN_QK_HEADS - 1;
    }
    __syncthreads();
    /* the third of the key head's value heads shifts its q/k conv state */
    if (last_arrival) {
        if (part < 2) {
            conv[0] = s1;
            conv[1] = s2;
            conv[2] = x;
        }
        if (tid == 0)
            __hip_atomic_store(&a.arrivals[s * Q38_GDN_ARRIVALS + kh], 0, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
}

/* grid (11, ceil(n_tokens / C), n_seq), 256 threads, C = Q38_GDN_PRE_TOKENS.
 * x < 10: channels 1024x..1024x+1023, 4 adjacent channels per lane, so a
 * half-wave holds one 128-channel head (x < 2 the q heads, 2 <= x < 4 the k
 * heads, then v), for tokens Cy..Cy+C-1; x == 10: the gates of those tokens.
 * Each lane rebuilds its channels' 3-tap windows from the raw inputs of the
 * three previous tokens (or from conv_state_in before the first token), so
 * runs are independent; the run holding the last token writes the shifted
 * state to conv_state_out, which must differ from conv_state_in when there is
 * more than one run.
 *
 * A lane issues the 16-byte loads of all its tokens at once (one memory round
 * trip per workgroup, not one per token), runs the conv backwards in place
 * over the window + tokens array, and the q/k half-waves form the C per-token
 * L2 norms with one transposing reduction: at each xor distance a lane keeps
 * the half of its partial sums whose token bit it owns and adds the partner's
 * copy of that half (C/2 + C/4 + ... exchanges instead of 5 per token); the
 * distances left once one sum remains add whole sums, so every lane ends with
 * one token's sum over the head, and a lane holding each token hands its
 * norm to the others.  Runs of 8 tokens (78 registers, 6 waves per SIMD)
 * measured fastest at 4096 tokens: 67 us against 71 (4) and 75 (16). */
extern "C" __global__ __launch_bounds__(256) void q38_gdn_pre(q38_gdn_pre_args a) {
    constexpr int C = Q38_GDN_PRE_TOKENS;
    constexpr int kLanesPerToken = 32 / C; /* lanes of a half-wave holding one token's sum */
    static_assert(C >= 4 && C <= 32 && (C & (C - 1)) == 0, "tokens per run: a power of two, 4 to 32");
    constexpr int kGroups = Q38_LIN_QKV_DIM / 1024;
    const int gx = blockIdx.x;
    const int run = blockIdx.y;
    const int s = blockIdx.z;
    const int tid = threadIdx.x;
    const int T = a.n_tokens;
    const int t0 = run * C;
    const int n = min(T - t0, C);
    const size_t tok0 = (size_t)s * T + t0;

    if (gx == kGroups) {
        /* n * 48 gates, up to C * 48 / 256 per thread: every load before
         * the first store */
        constexpr int kPer = (C * Q38_LIN_V_HEADS + 255) / 256;
        const int m = n * Q38_LIN_V_HEADS;
        const float *br = a.beta_raw + tok0 * Q38_LIN_V_HEADS;
        const float *ar = a.alpha_raw + tok0 * Q38_LIN_V_HEADS;
        float bv[kPer], av[kPer], dtv[kPer], aav[kPer];
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int i = min(tid + 256 * j, m - 1);
            const int h = i % Q38_LIN_V_HEADS;
            bv[j] = br[i];
            av[j] = ar[i];
            dtv[j] = a.dt[h];
            aav[j] = a.a[h];
        }
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int i = tid + 256 * j;
            if (i < m) {
                a.beta_out[tok0 * Q38_LIN_V_HEADS + i] = q38_sigmoid(bv[j]);
                a.g_out[tok0 * Q38_LIN_V_HEADS + i] = aav[j] * q38_softplus(av[j] + dtv[j]);
            }
        }
        return;
    }

    const int c = gx * 1024 + 4 * tid;
    f32x4 w[4]; /* w[k]: tap k of the 4 channels */
    {
        f32x4 r[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) r[j] = q38_ld4(a.conv_w + (size_t)(c + j) * 4);
#pragma unroll
        for (int k = 0; k < 4; ++k) w[k] = f32x4{r[0][k], r[1][k], r[2][k], r[3][k]};
    }
    const float *st_in = a.conv_state_in + (size_t)s * Q38_LIN_QKV_DIM * 3 + (size_t)c * 3;
    const float *src = a.qkv_raw + tok0 * Q38_LIN_QKV_DIM + c;
    /* e[0..2]: x_{t0-3}, x_{t0-2}, x_{t0-1}; e[3+i]: x_{t0+i} (the last
     * token repeated past n) */
    f32x4 e[3 + C];
    if (t0 == 0) {
        /* [4 channels][3 taps] from the state */
        const f32x4 r0 = q38_ld4(st_in), r1 = q38_ld4(st_in + 4), r2 = q38_ld4(st_in + 8);
        e[0] = f32x4{r0.x, r0.w, r1.z, r2.y};
        e[1] = f32x4{r0.y, r1.x, r1.w, r2.z};
        e[2] = f32x4{r0.z, r1.y, r2.x, r2.w};
    } else {
#pragma unroll
        for (int i = 0; i < 3; ++i) e[i] = q38_ld4(src - (long)(3 - i) * Q38_LIN_QKV_DIM);
    }
#pragma unroll
    for (int i = 0; i < C; ++i) e[3 + i] = q38_ld4(src + (size_t)min(i, n - 1) * Q38_LIN_QKV_DIM);
    /* conv1d + SiLU, last token first so e[3+i] is overwritten only after
     * the windows of tokens i+1..i+3 have read it */
#pragma unroll
    for (int i = C - 1; i >= 0; --i) {
        f32x4 y;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float v = e[i][j] * w[0][j];
            v += e[i + 1][j] * w[1][j];
            v += e[i + 2][j] * w[2][j];
            v += e[i + 3][j] * w[3][j];
            y[j] = q38_silu(v);
        }
        e[i + 3] = y;
    }
    if (gx < 4) {
        /* l2norm (ops.rs:562-571): f64 sum, f32 sqrt, floor 1e-6 */
        const int lane = tid & 63;
        double p[C];
#pragma unroll
        for (int i = 0; i < C; ++i) {
            const f32x4 y = e[3 + i];
            p[i] = (double)y.x * (double)y.x + (double)y.y * (double)y.y + (double)y.z * (double)y.z +
                   (double)y.w * (double)y.w;
        }
        int cnt = C; /* partial sums a lane still holds */
#pragma unroll
        for (int d = 16; d >= 1; d >>= 1) {
            if (cnt > 1) {
                const int h = cnt / 2;
                const bool hi = lane & d;
#pragma unroll
                for (int j = 0; j < h; ++j) {
                    const double keep = hi ? p[h + j] : p[j];
                    const double send = hi ? p[j] : p[h + j];
                    p[j] = keep + __shfl_xor(send, d, 64);
                }
                cnt = h;
            } else {
                p[0] += __shfl_xor(p[0], d, 64);
            }
        }
        /* lane l of a half-wave holds token (l % 32) / kLanesPerToken */
        float norm = sqrtf((float)p[0]);
        norm = fmaxf(norm, 1e-6f);
        const float inv = 1.0f / norm;
        const int half = lane & 32;
#pragma unroll
        for (int i = 0; i < C; ++i) e[3 + i] *= __shfl(inv, half + i * kLanesPerToken, 64);
    }
    float *dst = a.qkv_out + tok0 * Q38_LIN_QKV_DIM + c;
#pragma unroll
    for (int i = 0; i < C; ++i)
        if (i < n) q38_st4(dst + (size_t)i * Q38_LIN_QKV_DIM, e[3 + i]);
    if (t0 + n == T) {
        /* the window after the last token: x_{T-3}, x_{T-2}, x_{T-1} */
        const float *raw = a.qkv_raw + (size_t)s * T * Q38_LIN_QKV_DIM + c;
        f32x4 v[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const int tp = T - 3 + i;
            if (tp >= 0) {
                v[i] = q38_ld4(raw + (size_t)tp * Q38_LIN_QKV_DIM);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) v[i][j] = st_in[3 * j + tp + 3];
            }
        }
        float *st_out = a.conv_state_out + (size_t)s * Q38_LIN_QKV_DIM * 3 + (size_t)c * 3;
        q38_st4(st_out, f32x4{v[0].x, v[1].x, v[2].x, v[0].y});
        q38_st4(st_out + 4, f32x4{v[1].y, v[2].y, v[0].z, v[1].z});
        q38_st4(st_out + 8, f32x4{v[2].z, v[0].w, v[1].w, v[2].w});
    }
}

/* One recurrent step (n_tokens == 1) spread over the whole chip: the 128
 * rows of a value head are independent (ops.rs:707-713 touches row c only
 * through k, q, v_c, beta and the decay), so a workgroup takes 16 rows of
 * one head -- grid (48 heads x 8 row blocks, n_seq), 256 threads, 16 lanes
 * per row, lane i holding columns 4i..4i+3 and 64+4i..64+4i+3.  Every load
 * of a thread (its 8 state values, k, q, v_c, beta, g) is issued at once,
 * so the step costs one memory round trip; the state is read and written
 * exactly once.  Arithmetic per row is the same as q38_gdn_decode's. */
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
