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
constexpr int WR = Q38_GDN_WROW;
constexpr int BR = Q38_GDN_BROW;
constexpr int kPrepWaves = 8; /* two per SIMD: the prep's phases are latency-bound */
/* the image's three parts, in 1 KiB pieces: W, then Q' and Bm, then K'^T */
constexpr int kPiecesW = Q38_GDN_W_BYTES / 1024;
constexpr int kPiecesQB = Q38_GDN_QB_BYTES / 1024;
constexpr int kPiecesKt = Q38_GDN_KT_BYTES / 1024;
static_assert(2 * C * WR * 2 <= Q38_GDN_W_BYTES && 2 * C * WR * 2 + 2 * C * BR * 2 == Q38_GDN_QB_BYTES &&
                  2 * D * BR * 2 == Q38_GDN_KT_BYTES,
              "image parts");
static_assert(kPiecesW % 4 == 0 && kPiecesQB % 4 == 0 && kPiecesKt % 4 == 0,
              "each of the 4 moving scan waves moves the same number of pieces of every part");
constexpr int kPrepThreads = 64 * kPrepWaves;

/* One head-chunk record of the workspace: the scan's operand image (bf16
 * hi/lo, LDS layout), then U' and gamma_C. */
struct Record {
    __bf16 *w_hi, *w_lo, *q_hi, *q_lo, *b_hi, *b_lo, *kt_hi, *kt_lo;
    float *u;
    float *gamma_c;
    char *image;
};

Q38_DEV Record record_at(char *base) {
    Record r;
    r.image = base;
    r.w_hi = reinterpret_cast<__bf16 *>(base);
    r.w_lo = r.w_hi + C * WR;
    r.q_hi = reinterpret_cast<__bf16 *>(base + Q38_GDN_W_BYTES);
    r.q_lo = r.q_hi + C * WR;
    r.b_hi = r.q_lo + C * WR;
    r.b_lo = r.b_hi + C * BR;
    r.kt_hi = reinterpret_cast<__bf16 *>(base + Q38_GDN_W_BYTES + Q38_GDN_QB_BYTES);
    r.kt_lo = r.kt_hi + D * BR;
    r.u = reinterpret_cast<float *>(base + Q38_GDN_IMAGE_BYTES);
    r.gamma_c = r.u + C * D;
    return r;
}

Q38_DEV Record record_of(const q38_gdn_chunk_args &a, int s, int vh, int n) {
    return record_at(static_cast<char *>(a.work) +
                     (((size_t)s * Q38_LIN_V_HEADS + vh) * a.n_chunks + n) * Q38_GDN_RECORD_BYTES);
}

Q38_DEV void split_store(__bf16 *hi, __bf16 *lo, int idx, float x) {
    const __bf16 h = (__bf16)x;
    hi[idx] = h;
    lo[idx] = (__bf16)(x - (float)h);
}
}  // namespace

extern "C" __global__ __launch_bounds__(kPrepThreads) void q38_gdn_chunk_prep(q38_gdn_chunk_args a) {
    __shared__ __attribute__((aligned(16))) float sK[C][P];
    __shared__ __attribute__((aligned(16))) float sQ[C][P]; /* Q, then the staging of W */
    __shared__ __attribute__((aligned(16))) float sV[C][P];
    __shared__ float sA[C][C + 1];
    __shared__ __attribute__((aligned(16))) float sT[C][C + 4]; /* staging of Bm, then T */
    __shared__ float sX[3][16][17];
    __shared__ float sG[C], sBeta[C], sGraw[C], sBG[C], sGam[C], sKd[C];

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
    Record rec = record_of(a, s, vh, n);

    /* rows of the chunk (zero past the prompt: such rows add nothing) */
    for (int i = tid; i < C * (D / 4); i += kPrepThreads) {
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
    if (tid < C) { /* inclusive prefix sum of the log-decays over the chunk (one wave) */
        float acc = sGraw[tid];
#pragma unroll
        for (int d = 1; d < C; d <<= 1) {
            const float o = __shfl_up(acc, d, 64);
            if (tid >= d) acc += o;
        }
        sG[tid] = acc;
        const float g_last = __shfl(acc, C - 1, 64);
        sGam[tid] = expf(acc);
        sBG[tid] = sBeta[tid] * sGam[tid];
        sKd[tid] = expf(g_last - acc);
        if (tid == 0) *rec.gamma_c = expf(g_last);
    }
    __syncthreads();

    /* A (strictly lower) into LDS and Bm (lower, with the diagonal) staged in
     * sT: the 16 tile pairs (ti, tj) are 4 per wave; tiles above the diagonal
     * are zero without a product (2 per wave) */
    for (int job = wave; job < 16; job += kPrepWaves) {
        const int ti = job >> 2, tj = job & 3;
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
            sT[t][sc] = sc <= t ? dec * qk[i] : 0.0f;
        }
    }
    __syncthreads();
    /* Bm out as bf16 hi/lo rows (16-byte stores); Q' = diag(gamma) Q rows;
     * K'^T = (diag(exp(G_C - G)) K)^T by columns */
    for (int it = tid; it < C * (C / 8); it += kPrepThreads) {
        const int t = it >> 3, c8 = it & 7;
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = sT[t][8 * c8 + e];
        bf16x8 hi, lo;
        q38_split8(x, hi, lo);
        *reinterpret_cast<bf16x8 *>(rec.b_hi + t * BR + 8 * c8) = hi;
        *reinterpret_cast<bf16x8 *>(rec.b_lo + t * BR + 8 * c8) = lo;
    }
    for (int it = tid; it < C * (D / 8); it += kPrepThreads) {
        const int t = it >> 4, c8 = it & 15;
        const float gam = sGam[t];
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = gam * sQ[t][8 * c8 + e];
        bf16x8 hi, lo;
        q38_split8(x, hi, lo);
        *reinterpret_cast<bf16x8 *>(rec.q_hi + t * WR + 8 * c8) = hi;
        *reinterpret_cast<bf16x8 *>(rec.q_lo + t * WR + 8 * c8) = lo;
    }
    for (int it = tid; it < D * (C / 8); it += kPrepThreads) {
        const int i = it >> 3, t8 = it & 7;
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = sKd[8 * t8 + e] * sK[8 * t8 + e][i];
        bf16x8 hi, lo;
        q38_split8(x, hi, lo);
        *reinterpret_cast<bf16x8 *>(rec.kt_hi + i * BR + 8 * t8) = hi;
        *reinterpret_cast<bf16x8 *>(rec.kt_lo + i * BR + 8 * t8) = lo;
    }
    __syncthreads();

    /* T = (I + A)^-1, blockwise (16 x 16 blocks).  Diagonal block w: wave w,
     * lane j < 16 keeps column j of the block in registers and substitutes
     * row by row, T_rj = -A_rj - sum_{j<k<r} A_rk T_kj, reading each row of A
     * once (the same address in every lane). */
    if (wave < 4 && lane < 16) {
        const int b0 = 16 * wave;
        const int j = lane;
        float tc[16];
#pragma unroll
        for (int row = 0; row < 16; ++row) {
            float arow[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) arow[k] = sA[b0 + row][b0 + k];
            float v = -sA[b0 + row][b0 + j];
#pragma unroll
            for (int k = 0; k < row; ++k) v = k > j ? __builtin_fmaf(-arow[k], tc[k], v) : v;
            tc[row] = row < j ? 0.0f : (row == j ? 1.0f : v);
        }
#pragma unroll
        for (int row = 0; row < 16; ++row) sT[b0 + row][b0 + j] = tc[row];
    }
    /* above the diagonal blocks T is zero */
    for (int i = tid; i < C * C; i += kPrepThreads) {
        const int row = i >> 6, col = i & 63;
        if ((col >> 4) > (row >> 4)) sT[row][col] = 0.0f;
    }
    __syncthreads();
    /* off-diagonal blocks by distance: X_ij = sum_{k=j}^{i-1} A_ik T_kj, then
     * T_ij = -T_ii X_ij; wave q handles block q of the current distance, lane l
     * row l/4 and columns 4(l%4) .. +3 */
#pragma unroll
    for (int dist = 1; dist < 4; ++dist) {
        const bool mine = wave < 4 - dist;
        const int bj = wave, bi = wave + dist;
        const int row = lane >> 2, c4 = 4 * (lane & 3);
        if (mine) {
            float x[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int bk = 0; bk < dist; ++bk) {
#pragma unroll
                for (int kk = 0; kk < 16; ++kk) {
                    const int k = 16 * (bj + bk) + kk;
                    const float av = sA[16 * bi + row][k];
                    const f32x4 tv = *reinterpret_cast<const f32x4 *>(&sT[k][16 * bj + c4]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) x[e] = __builtin_fmaf(av, tv[e], x[e]);
                }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) sX[wave][row][c4 + e] = x[e];
        }
        __syncthreads();
        if (mine) {
            float y[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const float tv = sT[16 * bi + row][16 * bi + k];
#pragma unroll
                for (int e = 0; e < 4; ++e) y[e] = __builtin_fmaf(tv, sX[wave][k][c4 + e], y[e]);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) sT[16 * bi + row][16 * bj + c4 + e] = -y[e];
        }
        __syncthreads();
    }

    /* W = T diag(beta gamma) K (staged in sQ, then out as bf16 hi/lo rows) and
     * U' = T diag(beta) V (f32 out): 32 + 32 tiles, 8 per wave */
    for (int tile = wave; tile < 64; tile += kPrepWaves) {
        const bool is_w = tile < 32;
        const int ti = (tile & 31) >> 3, tn = tile & 7;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        if (is_w)
            acc = q38_mma16<C>(acc, [&](int m, int k) { return sT[16 * ti + m][k]; },
                               [&](int k, int nn) { return sBG[k] * sK[k][16 * tn + nn]; });
        else
            acc = q38_mma16<C>(acc, [&](int m, int k) { return sT[16 * ti + m][k]; },
                               [&](int k, int nn) { return sBeta[k] * sV[k][16 * tn + nn]; });
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = 16 * ti + 4 * g4 + i, col = 16 * tn + r;
            if (is_w)
                sQ[t][col] = acc[i];
            else
                rec.u[t * D + col] = acc[i];
        }
    }
    __syncthreads();
    for (int it = tid; it < C * (D / 8); it += kPrepThreads) {
        const int t = it >> 4, c8 = it & 15;
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = sQ[t][8 * c8 + e];
        bf16x8 hi, lo;
        q38_split8(x, hi, lo);
        *reinterpret_cast<bf16x8 *>(rec.w_hi + t * WR + 8 * c8) = hi;
        *reinterpret_cast<bf16x8 *>(rec.w_lo + t * WR + 8 * c8) = lo;
    }
}

/* 8 waves, two per SIMD: every phase of a chunk is a short dependent chain of
 * LDS reads and matrix steps, and a second wave per SIMD fills the gaps.
 * Waves 0-3 move the image (each every 4th piece of a part); all 8 compute. */
constexpr int kScanWaves = Q38_GDN_SCAN_WAVES;
static_assert(kScanWaves == 8, "steps a and b give each wave one of 8 tiles");

extern "C" __global__ __launch_bounds__(64 * kScanWaves) void q38_gdn_chunk_scan(q38_gdn_chunk_args a) {
    /* the chunk image in three arrays, one per part, so the compiler sees that
     * loads into one part do not alias reads of another */
    __shared__ __attribute__((aligned(16))) char imgW[Q38_GDN_W_BYTES];
    __shared__ __attribute__((aligned(16))) char imgQB[Q38_GDN_QB_BYTES];
    __shared__ __attribute__((aligned(16))) char imgK[Q38_GDN_KT_BYTES];
    __shared__ __attribute__((aligned(16))) __bf16 sSh[R][WR];
    __shared__ __attribute__((aligned(16))) __bf16 sSl[R][WR];
    __shared__ __attribute__((aligned(16))) __bf16 sUh[R][BR]; /* U^T: row = value row, col = token */
    __shared__ __attribute__((aligned(16))) __bf16 sUl[R][BR];

    /* workgroup -> (head, slab): consecutive workgroups go to the 8 XCDs in
     * turn, so a head's 4 slabs share one XCD and its L2 serves the image */
    const int L = blockIdx.x;
    const int vh = (L & 7) + 8 * (L >> 5);
    const int slab = (L >> 3) & 3;
    const int s = blockIdx.y;
    const int c0 = slab * R;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g4 = lane >> 4;
    const int r = lane & 15;
    const float query_scale = 1.0f / sqrtf((float)D);
    /* the image's arrays, in LDS */
    Record li;
    li.w_hi = reinterpret_cast<__bf16 *>(imgW);
    li.w_lo = li.w_hi + C * WR;
    li.q_hi = reinterpret_cast<__bf16 *>(imgQB);
    li.q_lo = li.q_hi + C * WR;
    li.b_hi = li.q_lo + C * WR;
    li.b_lo = li.b_hi + C * BR;
    li.kt_hi = reinterpret_cast<__bf16 *>(imgK);
    li.kt_lo = li.kt_hi + D * BR;

    /* f32 state of the slab in registers, in the layout of the state-update
     * tiles: wave w owns tiles 2w, 2w+1, tile -> (row block tc, column block tk) */
    float *st = a.state + (size_t)s * a.state_stride + ((size_t)vh * D + c0) * D;
    float S[2][4];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int tile = 2 * wave + q, tc = tile >> 3, tk = tile & 7;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 16 * tc + 4 * g4 + i, col = 16 * tk + r;
            S[q][i] = st[row * D + col];
            split_store(&sSh[0][0], &sSl[0][0], row * WR + col, S[q][i]);
        }
    }

    /* The next chunk's image streams in behind the compute, each part once
     * the step that reads it is done: W after step a, Q' and Bm (with U')
     * after step b, K'^T after step c.  Waves 0-3 each move every 4th piece
     * of a part; a wave's waits count its own operations, and the barrier
     * after the wait makes the pieces of all waves visible (waves 4-7 move
     * no pieces, so their waits pass at once). */
    /* steps a and b: wave w computes token block ti of value-row block tb */
    const int ti = wave & 3;
    const int tb = wave >> 2;
    const bool mover = wave < 4;
    auto fetch = [&](const char *src, char *dst, auto n_pieces) {
        if (!mover) return;
#pragma unroll
        for (int j = 0; j < decltype(n_pieces)::value / 4; ++j) {
            const int p = 4 * j + wave;
            __builtin_amdgcn_global_load_lds(src + p * 1024 + lane * 16,
                                             (__attribute__((address_space(3))) void *)(dst + p * 1024), 16, 0, 0);
        }
    };
    using PiecesW = std::integral_constant<int, kPiecesW>;
    using PiecesQB = std::integral_constant<int, kPiecesQB>;
    using PiecesKt = std::integral_constant<int, kPiecesKt>;
    auto fetch_w = [&](const Record &rec) { fetch(rec.image, imgW, PiecesW{}); };
    auto fetch_qb = [&](const Record &rec) { fetch(rec.image + Q38_GDN_W_BYTES, imgQB, PiecesQB{}); };
    auto fetch_kt = [&](const Record &rec) {
        fetch(rec.image + Q38_GDN_W_BYTES + Q38_GDN_QB_BYTES, imgK, PiecesKt{});
    };
    float up[4];
    float gamma_c;
    auto fetch_u = [&](const Record &rec) {
#pragma unroll
        for (int i = 0; i < 4; ++i) up[i] = rec.u[(16 * ti + 4 * g4 + i) * D + c0 + 16 * tb + r];
        gamma_c = *rec.gamma_c;
    };
    {
        const Record rec0 = record_of(a, s, vh, 0);
        fetch_w(rec0);
        fetch_qb(rec0);
        fetch_u(rec0);
        fetch_kt(rec0);
        q38_barrier_vm<0>();
    }

    for (int n = 0; n < a.n_chunks; ++n) {
        const int t0 = n * C;
        const int cnt = min(C, a.n_tokens - t0);
        const size_t tok0 = (size_t)s * a.n_tokens + t0;
        const bool more = n + 1 < a.n_chunks;
        const Record next = record_of(a, s, vh, more ? n + 1 : n);

        /* a: U = U' - W S^T (64 x 32): wave w takes tile (ti, tb); U^T to LDS */
        {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            acc = q38_mma16_split<D>(acc, li.w_hi + 16 * ti * WR, li.w_lo + 16 * ti * WR, WR, &sSh[16 * tb][0],
                                     &sSl[16 * tb][0], WR);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                split_store(&sUh[0][0], &sUl[0][0], (16 * tb + r) * BR + 16 * ti + 4 * g4 + i, up[i] - acc[i]);
        }
        const float gc = gamma_c;
        q38_barrier_vm<63>(); /* U^T in LDS; W free */
        if (more) fetch_w(next);

        /* b: O = (Q' S^T + Bm U) / sqrt(128), Q' = diag(gamma) Q */
        f32x4 o;
        {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            acc = q38_mma16_split<D>(acc, li.q_hi + 16 * ti * WR, li.q_lo + 16 * ti * WR, WR, &sSh[16 * tb][0],
                                     &sSl[16 * tb][0], WR);
            o = q38_mma16_split<C>(acc, li.b_hi + 16 * ti * BR, li.b_lo + 16 * ti * BR, BR, &sUh[16 * tb][0],
                                   &sUl[16 * tb][0], BR);
        }
        /* this chunk's K'^T has landed: only the next W is younger.  The
         * output stores come after the wait, as their number varies. */
        if (more)
            __builtin_amdgcn_s_waitcnt(q38_waitcnt(kPiecesW / 4, 15));
        else
            __builtin_amdgcn_s_waitcnt(q38_waitcnt(0, 15));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = 16 * ti + 4 * g4 + i;
            if (t < cnt) a.out[(tok0 + t) * Q38_LIN_V_DIM + vh * D + c0 + 16 * tb + r] = o[i] * query_scale;
        }
        q38_barrier_vm<63>(); /* K'^T of every wave in LDS; Q', Bm free */
        if (more) {
            fetch_qb(next);
            fetch_u(next);
        }

        /* c: S <- gamma_C S + U^T K' (tiles of the register layout) */
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int tile = 2 * wave + q, tc = tile >> 3, tk = tile & 7;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            acc = q38_mma16_split<C>(acc, &sUh[16 * tc][0], &sUl[16 * tc][0], BR, li.kt_hi + 16 * tk * BR,
                                     li.kt_lo + 16 * tk * BR, BR);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                S[q][i] = __builtin_fmaf(gc, S[q][i], acc[i]);
                /* opaque stores: the next chunk's Q' and Bm are loading */
                const int idx = (16 * tc + 4 * g4 + i) * WR + 16 * tk + r;
                const __bf16 h = (__bf16)S[q][i];
                q38_lds_store_bf16(&sSh[0][0] + idx, h);
                q38_lds_store_bf16(&sSl[0][0] + idx, (__bf16)(S[q][i] - (float)h));
            }
        }
        q38_barrier_vm<63>(); /* the new S in LDS; K'^T free */
        if (more) {
            fetch_kt(next);
            /* the next W, Q', Bm and U' (every wave); K'^T still in flight */
            q38_barrier_vm<kPiecesKt / 4>();
        }
    }

#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int tile = 2 * wave + q, tc = tile >> 3, tk = tile & 7;
#pragma unroll
        for (int i = 0; i < 4; ++i) st[(16 * tc + 4 * g4 + i) * D + 16 * tk + r] = S[q][i];
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
