/*
 * Chunked Gated-DeltaNet prefill (gfx950): the recurrence of linear_core
 * (src/model/ops.rs:698-714) over a prompt, 64 tokens at a time, with the
 * intra-chunk products on bf16x3 MFMA (q38_mma16).
 *
 * The reference runs the recurrence token by token (ops.rs:1084-1099):
 *     S_t = d_t S_{t-1} + u_t k_t^T,  u_t = beta_t (v_t - d_t S_{t-1} k_t),
 *     o_t = S_t q_t / sqrt(128)
 * with S [128 value rows][128 key columns], d_t = exp(g_t).  Unrolled over a
 * chunk that starts from S_0, with G_t = g_1 + ... + g_t and gamma_t = exp(G_t):
 *     S_t = gamma_t S_0 + sum_{s<=t} exp(G_t - G_s) u_s k_s^T
 *     u_t = beta_t (v_t - gamma_t S_0 k_t - sum_{s<t} exp(G_t - G_s) (k_s.k_t) u_s)
 * i.e. (I + A) U = diag(beta) (V - diag(gamma) K S_0^T) with the strictly lower
 * A_ts = beta_t exp(G_t - G_s) k_t.k_s.  With T = (I + A)^-1:
 *     W  = T diag(beta gamma) K,   U' = T diag(beta) V,   U = U' - W S_0^T
 *     O  = (diag(gamma) Q S_0^T + Bm U) / sqrt(128),  Bm_ts = exp(G_t - G_s) q_t.k_s (s <= t)
 *     S_C = gamma_C S_0 + U^T diag(exp(G_C - G)) K
 * Every decay factor is exp of a difference G_t - G_s (s <= t) or of G_t
 * itself, never exp(-G), so nothing overflows when decays are strong.
 *
 * q38_gdn_chunk_prep (grid (48 heads, chunks, sequences)) computes W, U', Bm
 * and G of every chunk in parallel; T comes from a blocked forward
 * substitution in f32 (16x16 diagonal blocks inverted by substitution, the
 * off-diagonal blocks by T_ij = -T_ii sum_k A_ik T_kj).
 * q38_gdn_chunk_scan (grid (48 heads x 4 slabs of 32 value rows, sequences))
 * carries its slab of the state through the chunks: value rows are
 * independent in every formula above, so a slab needs only its own rows.
 * q38_gdn_post applies the gated RMSNorm of ops.rs:735-740.
 */
#include "q38_device.h"

namespace {
constexpr int C = Q38_GDN_CHUNK;     /* tokens per chunk */
constexpr int D = Q38_LIN_HEAD_DIM;  /* 128 */
constexpr int P = D + 4;             /* padded LDS row (floats) */
constexpr int kSlabs = 4;
constexpr int R = D / kSlabs;        /* value rows per scan slab */
}  // namespace

extern "C" __global__ __launch_bounds__(256) void q38_gdn_chunk_prep(q38_gdn_chunk_args a) {
    __shared__ __attribute__((aligned(16))) float sK[C][P];
    __shared__ __attribute__((aligned(16))) float sQ[C][P];
    __shared__ __attribute__((aligned(16))) float sV[C][P];
    __shared__ float sA[C][C + 1];
    __shared__ float sT[C][C + 1];
    __shared__ float sX[3][16][17];
    __shared__ float sG[C], sBeta[C], sGraw[C], sBG[C];

    const int vh = blockIdx.x;
    const int n = blockIdx.y;
    const int s = blockIdx.z;
    const int kh = vh % Q38_LIN_QK_HEADS;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g4 = lane >> 4;
    const int r = lane & 15;
    const int t0 = n * C;
    const int cnt = min(C, a.n_tokens - t0);
    const size_t tok0 = (size_t)s * a.n_tokens + t0;

    /* rows of the chunk (zero past the prompt: such rows add nothing) */
    for (int i = tid; i < C * (D / 4); i += 256) {
        const int t = i >> 5, c4 = i & 31;
        f32x4 kv = {0.f, 0.f, 0.f, 0.f}, qv = kv, vv = kv;
        if (t < cnt) {
            const size_t tok = tok0 + t;
            kv = q38_ld4(a.k + tok * a.q_stride + kh * D + 4 * c4);
            qv = q38_ld4(a.q + tok * a.q_stride + kh * D + 4 * c4);
            vv = q38_ld4(a.v + tok * a.v_stride + vh * D + 4 * c4);
        }
        q38_st4(&sK[t][4 * c4], kv);
        q38_st4(&sQ[t][4 * c4], qv);
        q38_st4(&sV[t][4 * c4], vv);
    }
    if (tid < C) {
        const bool in = tid < cnt;
        sBeta[tid] = in ? a.beta[(tok0 + tid) * Q38_LIN_V_HEADS + vh] : 0.0f;
        sGraw[tid] = in ? a.g[(tok0 + tid) * Q38_LIN_V_HEADS + vh] : 0.0f;
    }
    __syncthreads();
    if (tid < C) {
        float acc = 0.0f;
        for (int i = 0; i <= tid; ++i) acc += sGraw[i];
        sG[tid] = acc;
        sBG[tid] = sBeta[tid] * expf(acc);
    }
    __syncthreads();

    float *wk = a.work + (((size_t)s * Q38_LIN_V_HEADS + vh) * a.n_chunks + n) * Q38_GDN_CHUNK_FLOATS;
    float *gW = wk;
    float *gU = wk + C * D;
    float *gB = wk + 2 * C * D;
    float *gG = wk + 2 * C * D + C * C;
    if (tid < C) gG[tid] = sG[tid];

    /* A (strictly lower) into LDS and Bm (lower, with the diagonal) to the
     * workspace: wave w takes row block w */
    {
        const int ti = wave;
#pragma unroll
        for (int tj = 0; tj < 4; ++tj) {
            f32x4 kk = {0.f, 0.f, 0.f, 0.f}, qk = kk;
            if (tj <= ti) {
                kk = q38_mma16<D>(kk, [&](int m, int k) { return sK[16 * ti + m][k]; },
                                  [&](int k, int nn) { return sK[16 * tj + nn][k]; });
                qk = q38_mma16<D>(qk, [&](int m, int k) { return sQ[16 * ti + m][k]; },
                                  [&](int k, int nn) { return sK[16 * tj + nn][k]; });
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = 16 * ti + 4 * g4 + i;
                const int sc = 16 * tj + r;
                const float dec = sc <= t ? expf(sG[t] - sG[sc]) : 0.0f;
                sA[t][sc] = sc < t ? sBeta[t] * dec * kk[i] : 0.0f;
                gB[t * C + sc] = sc <= t ? dec * qk[i] : 0.0f;
            }
        }
    }
    __syncthreads();

    /* T = (I + A)^-1.  Diagonal blocks: wave w, lane j < 16 owns column j of
     * block w (it reads only A and its own column, so no barrier inside). */
    if (r == lane) { /* lanes 0..15 */
        const int b0 = 16 * wave;
        const int j = lane;
        for (int row = 0; row < 16; ++row) {
            float v;
            if (row < j) v = 0.0f;
            else if (row == j) v = 1.0f;
            else {
                v = -sA[b0 + row][b0 + j];
                for (int k = j + 1; k < row; ++k) v = __builtin_fmaf(-sA[b0 + row][b0 + k], sT[b0 + k][b0 + j], v);
            }
            sT[b0 + row][b0 + j] = v;
        }
    }
    /* above the diagonal blocks T is zero */
    for (int i = tid; i < C * C; i += 256) {
        const int row = i >> 6, col = i & 63;
        if ((col >> 4) > (row >> 4)) sT[row][col] = 0.0f;
    }
    __syncthreads();
    /* off-diagonal blocks by distance: X_ij = sum_{k=j}^{i-1} A_ik T_kj, then
     * T_ij = -T_ii X_ij; wave q handles block q of the current distance */
    for (int dist = 1; dist < 4; ++dist) {
        const int nb = 4 - dist;
        const bool mine = wave < nb;
        const int bj = wave, bi = wave + dist;
        if (mine) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int idx = lane * 4 + e; /* 0..255 */
                const int row = idx >> 4, col = idx & 15;
                float x = 0.0f;
                for (int bk = bj; bk < bi; ++bk)
                    for (int k = 0; k < 16; ++k)
                        x = __builtin_fmaf(sA[16 * bi + row][16 * bk + k], sT[16 * bk + k][16 * bj + col], x);
                sX[wave][row][col] = x;
            }
        }
        __syncthreads();
        if (mine) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int idx = lane * 4 + e;
                const int row = idx >> 4, col = idx & 15;
                float y = 0.0f;
                for (int k = 0; k < 16; ++k) y = __builtin_fmaf(sT[16 * bi + row][16 * bi + k], sX[wave][k][col], y);
                sT[16 * bi + row][16 * bj + col] = -y;
            }
        }
        __syncthreads();
    }

    /* W = T diag(beta gamma) K and U' = T diag(beta) V: 32 + 32 tiles, 16 per wave */
    for (int tile = wave; tile < 64; tile += 4) {
        const bool is_w = tile < 32;
        const int ti = (tile & 31) >> 3, tn = tile & 7;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        if (is_w)
            acc = q38_mma16<C>(acc, [&](int m, int k) { return sT[16 * ti + m][k]; },
                               [&](int k, int nn) { return sBG[k] * sK[k][16 * tn + nn]; });
        else
            acc = q38_mma16<C>(acc, [&](int m, int k) { return sT[16 * ti + m][k]; },
                               [&](int k, int nn) { return sBeta[k] * sV[k][16 * tn + nn]; });
        float *dst = is_w ? gW : gU;
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[(16 * ti + 4 * g4 + i) * D + 16 * tn + r] = acc[i];
    }
}

extern "C" __global__ __launch_bounds__(256) void q38_gdn_chunk_scan(q38_gdn_chunk_args a) {
    __shared__ __attribute__((aligned(16))) float sS[R][P];
    __shared__ __attribute__((aligned(16))) float sW[C][P];
    __shared__ __attribute__((aligned(16))) float sQ[C][P];
    __shared__ __attribute__((aligned(16))) float sK[C][P];
    __shared__ __attribute__((aligned(16))) float sB[C][C + 4];
    __shared__ float sU[C][R + 4];
    __shared__ float sG[C], sKd[C];

    const int vh = blockIdx.x / kSlabs;
    const int slab = blockIdx.x % kSlabs;
    const int s = blockIdx.y;
    const int kh = vh % Q38_LIN_QK_HEADS;
    const int c0 = slab * R;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g4 = lane >> 4;
    const int r = lane & 15;
    const float query_scale = 1.0f / sqrtf((float)D);

    float *st = a.state + (size_t)s * a.state_stride + ((size_t)vh * D + c0) * D;
    for (int i = tid; i < R * (D / 4); i += 256) {
        const int row = i >> 5, c4 = i & 31;
        q38_st4(&sS[row][4 * c4], q38_ld4(st + row * D + 4 * c4));
    }

    for (int n = 0; n < a.n_chunks; ++n) {
        const int t0 = n * C;
        const int cnt = min(C, a.n_tokens - t0);
        const size_t tok0 = (size_t)s * a.n_tokens + t0;
        const float *wk = a.work + (((size_t)s * Q38_LIN_V_HEADS + vh) * a.n_chunks + n) * Q38_GDN_CHUNK_FLOATS;
        const float *gW = wk;
        const float *gU = wk + C * D;
        const float *gB = wk + 2 * C * D;
        const float *gG = wk + 2 * C * D + C * C;
        for (int i = tid; i < C * (D / 4); i += 256) {
            const int t = i >> 5, c4 = i & 31;
            f32x4 kv = {0.f, 0.f, 0.f, 0.f}, qv = kv;
            if (t < cnt) {
                kv = q38_ld4(a.k + (tok0 + t) * a.q_stride + kh * D + 4 * c4);
                qv = q38_ld4(a.q + (tok0 + t) * a.q_stride + kh * D + 4 * c4);
            }
            q38_st4(&sK[t][4 * c4], kv);
            q38_st4(&sQ[t][4 * c4], qv);
            q38_st4(&sW[t][4 * c4], q38_ld4(gW + t * D + 4 * c4));
        }
        for (int i = tid; i < C * (C / 4); i += 256) {
            const int t = i >> 4, c4 = i & 15;
            q38_st4(&sB[t][4 * c4], q38_ld4(gB + t * C + 4 * c4));
        }
        for (int i = tid; i < C * (R / 4); i += 256) {
            const int t = i >> 3, c4 = i & 7;
            const f32x4 u = q38_ld4(gU + t * D + c0 + 4 * c4);
#pragma unroll
            for (int e = 0; e < 4; ++e) sU[t][4 * c4 + e] = u[e];
        }
        if (tid < C) sG[tid] = gG[tid];
        __syncthreads();
        const float g_last = sG[C - 1]; /* G of the chunk's last token (padding adds 0) */
        if (tid < C) sKd[tid] = expf(g_last - sG[tid]);

        /* U = U' - W S^T (64 x 32): wave w takes token block w; each lane
         * rewrites only the elements it read */
        {
            const int ti = wave;
#pragma unroll
            for (int tc = 0; tc < 2; ++tc) {
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                acc = q38_mma16<D>(acc, [&](int m, int k) { return sW[16 * ti + m][k]; },
                                   [&](int k, int nn) { return sS[16 * tc + nn][k]; });
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = 16 * ti + 4 * g4 + i;
                    sU[t][16 * tc + r] -= acc[i];
                }
            }
        }
        __syncthreads();

        /* O = (diag(gamma) Q S^T + Bm U) / sqrt(128) */
        {
            const int ti = wave;
#pragma unroll
            for (int tc = 0; tc < 2; ++tc) {
                f32x4 qs = {0.f, 0.f, 0.f, 0.f}, bu = qs;
                qs = q38_mma16<D>(qs, [&](int m, int k) { return sQ[16 * ti + m][k]; },
                                  [&](int k, int nn) { return sS[16 * tc + nn][k]; });
                bu = q38_mma16<C>(bu, [&](int m, int k) { return sB[16 * ti + m][k]; },
                                  [&](int k, int nn) { return sU[k][16 * tc + nn]; });
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = 16 * ti + 4 * g4 + i;
                    if (t < cnt) {
                        const float o = (expf(sG[t]) * qs[i] + bu[i]) * query_scale;
                        a.out[(tok0 + t) * Q38_LIN_V_DIM + vh * D + c0 + 16 * tc + r] = o;
                    }
                }
            }
        }
        __syncthreads();

        /* S <- gamma_C S + U^T diag(exp(G_C - G)) K: 2 x 8 tiles, 4 per wave */
        {
            const float gC = expf(g_last);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int tile = wave * 4 + q;
                const int tc = tile >> 3, tk = tile & 7;
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                acc = q38_mma16<C>(acc, [&](int m, int k) { return sU[k][16 * tc + m]; },
                                   [&](int k, int nn) { return sKd[k] * sK[k][16 * tk + nn]; });
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = 16 * tc + 4 * g4 + i;
                    const int col = 16 * tk + r;
                    sS[row][col] = __builtin_fmaf(gC, sS[row][col], acc[i]);
                }
            }
        }
        __syncthreads();
    }

    for (int i = tid; i < R * (D / 4); i += 256) {
        const int row = i >> 5, c4 = i & 31;
        q38_st4(st + row * D + 4 * c4, q38_ld4(&sS[row][4 * c4]));
    }
}

/* Gated RMSNorm (ops.rs:735-740) of one (token, value head): rmsnorm of the
 * 128 outputs with the f64 sum of squares, weight, times silu(z). */
extern "C" __global__ __launch_bounds__(64) void q38_gdn_post(q38_gdn_post_args a) {
    const size_t tok = blockIdx.x;
    const int vh = blockIdx.y;
    const int lane = threadIdx.x;
    const size_t base = tok * Q38_LIN_V_DIM + vh * D;
    const float x0 = a.o[base + lane];
    const float x1 = a.o[base + lane + 64];
    double ss = (double)x0 * (double)x0 + (double)x1 * (double)x1;
    ss = q38_wave_sum_f64(ss);
    const float mean = (float)(ss / (double)D);
    const float scale = 1.0f / sqrtf(mean + 1e-6f);
    float y0 = x0 * scale * a.norm_w[lane];
    float y1 = x1 * scale * a.norm_w[lane + 64];
    y0 *= q38_silu(a.z[base + lane]);
    y1 *= q38_silu(a.z[base + lane + 64]);
    a.out[base + lane] = y0;
    a.out[base + lane + 64] = y1;
}
