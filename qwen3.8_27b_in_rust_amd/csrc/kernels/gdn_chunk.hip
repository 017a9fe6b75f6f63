/*
 * Chunked Gated-DeltaNet prefill (gfx950): the recurrence of linear_core
 * (src/model/ops.rs:698-714) over a prompt, 64 tokens at a time, with the
 * intra-chunk products on bf16x3 MFMA (q38_mma16_split).
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
 * q38_gdn_chunk_prep (grid (16 q/k heads, chunks, sequences)) computes W, U',
 * Bm and G of every chunk in parallel, for the 3 value heads that read one
 * q/k head; T comes from a blocked inverse in f32 (16x16 diagonal blocks by
 * substitution, the off-diagonal blocks by T_ij = -T_ii sum_k A_ik T_kj on
 * fp32 matrix instructions).
 * q38_gdn_chunk_scan (grid (48 heads x 4 slabs of 32 value rows, sequences))
 * carries its slab of the state through the chunks: value rows are
 * independent in every formula above, so a slab needs only its own rows.
 * q38_gdn_post applies the gated RMSNorm of ops.rs:735-740.
 */
#include "q38_device.h"

namespace {
constexpr int C = Q38_GDN_CHUNK;     /* tokens per chunk */
constexpr int D = Q38_LIN_HEAD_DIM;  /* 128 */
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

/* gamma_C sits in the padding after W hi/lo, so it travels with W */
constexpr int kGammaOffset = 2 * C * WR * 2;
static_assert(kGammaOffset + 4 <= Q38_GDN_W_BYTES, "gamma_C in the W part");

/* One head-chunk record of the workspace: the scan's operand image (bf16
 * hi/lo, LDS layout; gamma_C in the W part), then U'. */
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
    r.gamma_c = reinterpret_cast<float *>(base + kGammaOffset);
    return r;
}

Q38_DEV Record record_of(const q38_gdn_chunk_args &a, int s, int vh, int n) {
    return record_at(static_cast<char *>(a.work) +
                     (((size_t)s * Q38_LIN_V_HEADS + vh) * a.n_chunks + n) * Q38_GDN_RECORD_BYTES);
}

/* Workgroup barrier after this wave's LDS operations: the prep's waves share
 * data only through LDS, so its barriers need not wait for the record's
 * global stores (as __syncthreads() would) and those drain behind the
 * compute. */
Q38_DEV void lds_barrier() { q38_barrier_vm<63>(); }

/* LDS byte address of a __shared__ object */
Q38_DEV uint32_t lds_address(const void *p) {
    return (uint32_t)(size_t)(const __attribute__((address_space(3))) char *)p;
}

/* One 1 KiB piece, 16 bytes per lane from base + off, straight to LDS at
 * lds + 16 * lane.  Written in assembly so that the compiler's wait-count
 * pass does not track it (it would otherwise wait for every piece in flight
 * at the top of the chunk loop): every read of a piece follows an explicit
 * vector-memory wait and a barrier.  M0 carries the LDS address; nothing
 * else in the kernel uses M0. */
Q38_DEV void dma_piece(uint32_t lds, const void *base, uint32_t off) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(off), "s"(base)
                 : "memory");
}

Q38_DEV void split_store(__bf16 *hi, __bf16 *lo, int idx, float x) {
    const __bf16 h = (__bf16)x;
    hi[idx] = h;
    lo[idx] = (__bf16)(x - (float)h);
}

/* 16 x 16 tiles (ti, tj) on or below the block diagonal of a 64 x 64 matrix,
 * numbered row by row: p = ti (ti + 1) / 2 + tj. */
constexpr int kLowerTiles = 10;
Q38_DEV int lower_tile_row(int p) { return p < 1 ? 0 : (p < 3 ? 1 : (p < 6 ? 2 : 3)); }

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

/* x = hi + lo as bf16 (8-byte stores of 4 elements each) */
Q38_DEV void split4_store(__bf16 *hi, __bf16 *lo, f32x4 x) {
    bf16x4 h, l;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        h[e] = (__bf16)x[e];
        l[e] = (__bf16)(x[e] - (float)h[e]);
    }
    *reinterpret_cast<bf16x4 *>(hi) = h;
    *reinterpret_cast<bf16x4 *>(lo) = l;
}

/* One 16 x 16 tile on bf16x3 products, c += A B, with A given by columns,
 * A(m, k) = a[k * lda_k + m] (8 two-byte reads per fragment half), and B by
 * columns contiguous in k, B(k, n) = b[n * ldb + k] (one 16-byte read). */
template <int KD>
Q38_DEV f32x4 mma16_split_acol(f32x4 c, const __bf16 *a_hi, const __bf16 *a_lo, int lda_k, const __bf16 *b_hi,
                               const __bf16 *b_lo, int ldb) {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4;
    const int r = lane & 15;
#pragma unroll
    for (int k0 = 0; k0 < KD; k0 += 32) {
        bf16x8 ah, al;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            ah[j] = a_hi[(k0 + 8 * g + j) * lda_k + r];
            al[j] = a_lo[(k0 + 8 * g + j) * lda_k + r];
        }
        const int bo = r * ldb + k0 + 8 * g;
        const bf16x8 bh = *reinterpret_cast<const bf16x8 *>(b_hi + bo);
        const bf16x8 bl = *reinterpret_cast<const bf16x8 *>(b_lo + bo);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, c, 0, 0, 0);
    }
    return c;
}
/* T = (I + A)^-1 for the strictly lower 64 x 64 A, blockwise (16 x 16 blocks).
 * Diagonal block w: wave w, lane j < 16 keeps column j of the block in
 * registers and substitutes row by row, T_rj = -A_rj - sum_{j<k<r} A_rk T_kj,
 * reading each row of A once (the same address in every lane).  Off-diagonal
 * blocks by distance, block (w + dist, w) by wave w on fp32 matrix steps
 * (v_mfma_f32_16x16x4_f32): X = sum_{k=j}^{i-1} A_ik T_kj, then
 * T_ij = -T_ii X.  Each 16x16x16 product runs its contraction index as
 * k = 4g + s (lane group g, step s), so X, held as the accumulator (lane (g, r):
 * rows 4g .. 4g+3 of column r), is already the right operand of the second
 * product.  Blocks above the diagonal are zero.  Ends with a barrier. */
Q38_DEV void invert_unit_lower(const float (*sA)[BR], float (*sT)[C + 4], int wave, int lane) {
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
    for (int i = threadIdx.x; i < C * C; i += kPrepThreads) {
        const int row = i >> 6, col = i & 63;
        if ((col >> 4) > (row >> 4)) sT[row][col] = 0.0f;
    }
    lds_barrier();
    const int g = lane >> 4, r = lane & 15;
#pragma unroll
    for (int dist = 1; dist < 4; ++dist) {
        if (wave < 4 - dist) {
            const int bj = wave, bi = wave + dist;
            f32x4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int bk = bj; bk < bi; ++bk) {
                const f32x4 av = *reinterpret_cast<const f32x4 *>(&sA[16 * bi + r][16 * bk + 4 * g]);
#pragma unroll
                for (int st = 0; st < 4; ++st)
                    x = __builtin_amdgcn_mfma_f32_16x16x4f32(av[st], sT[16 * bk + 4 * g + st][16 * bj + r], x, 0, 0,
                                                             0);
            }
            const f32x4 tv = *reinterpret_cast<const f32x4 *>(&sT[16 * bi + r][16 * bi + 4 * g]);
            f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < 4; ++st) y = __builtin_amdgcn_mfma_f32_16x16x4f32(tv[st], x[st], y, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) sT[16 * bi + 4 * g + i][16 * bj + r] = -y[i];
        }
        lds_barrier();
    }
}
}  // namespace

/*
 * One workgroup per (q/k head, chunk): the 3 value heads that read q/k head
 * kh (value heads kh, kh + 16, kh + 32; ops.rs:691) share K, Q, their bf16
 * splits and the products K K^T and Q K^T; the decays, betas, T, W, U' and
 * the images are per value head, formed one head after another.
 */
extern "C" __global__ __launch_bounds__(kPrepThreads) void q38_gdn_chunk_prep(q38_gdn_chunk_args a) {
    constexpr int kGroup = Q38_LIN_V_HEADS / Q38_LIN_QK_HEADS;
    /* K as bf16 hi/lo rows, for all three heads */
    __shared__ __attribute__((aligned(16))) __bf16 sKh[C][WR];
    __shared__ __attribute__((aligned(16))) __bf16 sKl[C][WR];
    /* the 10 tiles on or below the block diagonal of K K^T and of Q K^T */
    __shared__ float sKK[kLowerTiles][16][17];
    __shared__ float sQK[kLowerTiles][16][17];
    /* Q as bf16 hi/lo rows while K K^T and Q K^T are formed; then V^T of the
     * current head as bf16 hi/lo rows of the chunk's 64 tokens */
    __shared__ __attribute__((aligned(16))) __bf16 sVh[D][BR];
    __shared__ __attribute__((aligned(16))) __bf16 sVl[D][BR];
    /* A (f32); once T is complete, T diag(beta) as bf16 hi/lo (U''s left operand) */
    __shared__ __attribute__((aligned(16))) float sA[C][BR];
    __shared__ __attribute__((aligned(16))) float sT[C][C + 4];
    /* T diag(beta gamma) as bf16 hi/lo (W's left operand) */
    __shared__ __attribute__((aligned(16))) __bf16 sWh[C][BR];
    __shared__ __attribute__((aligned(16))) __bf16 sWl[C][BR];
    __shared__ float sG[C], sBeta[C], sBG[C], sKd[C];
    __shared__ float sG3[3][C], sBeta3[3][C]; /* G and beta of the three heads */
    static_assert(2 * C * BR * 2 == sizeof(float) * C * BR, "T diag(beta) fits over A");
    static_assert(C * WR <= D * BR, "Q rows fit over V^T");
    __bf16 *const sQh = &sVh[0][0]; /* [C][WR] */
    __bf16 *const sQl = &sVl[0][0];

    const int kh = blockIdx.x;
    const int n = blockIdx.y;
    const int s = blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g4 = lane >> 4;
    const int r = lane & 15;
    const int t0 = (a.chunk0 + n) * C;
    const int cnt = min(C, a.n_tokens - t0);
    const size_t tok0 = (size_t)s * a.n_tokens + t0;

    /* rows of the chunk (zero past the prompt: such rows add nothing).  Pass p,
     * lane l of wave w: token 8 (2p + w/4) + l/8, columns 4c .. 4c+3 with
     * c = 8 (w%4) + l%8, so 8 lanes read 128 contiguous bytes of a row.  Every
     * load is unconditional (a row past the prompt reads the chunk's last
     * row) and rows past the prompt are zeroed where they are used: a load
     * under a branch makes the compiler wait for it at the branch's end. */
    auto row_t = [&](int p) { return 8 * (2 * p + (wave >> 2)) + (lane >> 3); };
    auto col_c4 = [&]() { return 8 * (wave & 3) + (lane & 7); };
    f32x4 kv[4], qv[4], vv[4];
    auto load_v = [&](int vh) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const size_t tok = tok0 + min(row_t(p), cnt - 1);
            vv[p] = q38_ld4(a.v + tok * a.v_stride + vh * D + 4 * col_c4());
        }
    };
    auto live = [&](int p, f32x4 x) { return row_t(p) < cnt ? x : f32x4{0.f, 0.f, 0.f, 0.f}; };
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const size_t tok = tok0 + min(row_t(p), cnt - 1);
        kv[p] = q38_ld4(a.k + tok * a.q_stride + kh * D + 4 * col_c4());
        qv[p] = q38_ld4(a.q + tok * a.q_stride + kh * D + 4 * col_c4());
    }
    load_v(kh);
    /* log-decays and betas of the three heads, one token per lane; every
     * wave forms the inclusive prefix sums G of the log-decays for its own
     * use */
    float beta_in[kGroup], acc_g[kGroup];
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
        const int vh = kh + Q38_LIN_QK_HEADS * j;
        const size_t tok = tok0 + min(lane, cnt - 1);
        beta_in[j] = a.beta[tok * Q38_LIN_V_HEADS + vh];
        acc_g[j] = a.g[tok * Q38_LIN_V_HEADS + vh];
    }
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
        beta_in[j] = lane < cnt ? beta_in[j] : 0.0f;
        acc_g[j] = lane < cnt ? acc_g[j] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
#pragma unroll
        for (int d = 1; d < C; d <<= 1) {
            const float o = __shfl_up(acc_g[j], d, 64);
            if (lane >= d) acc_g[j] += o;
        }
        if (wave == 0) {
            sG3[j][lane] = acc_g[j];
            sBeta3[j][lane] = beta_in[j];
        }
    }
    /* K and Q split into LDS; Q' = diag(gamma) Q of every head straight to
     * its record */
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const int t = row_t(p), c4 = col_c4();
        const f32x4 kx = live(p, kv[p]), qx = live(p, qv[p]);
        split4_store(&sKh[t][4 * c4], &sKl[t][4 * c4], kx);
        split4_store(sQh + t * WR + 4 * c4, sQl + t * WR + 4 * c4, qx);
#pragma unroll
        for (int j = 0; j < kGroup; ++j) {
            const Record rec = record_of(a, s, kh + Q38_LIN_QK_HEADS * j, n);
            const float gam = expf(__shfl(acc_g[j], t, 64));
            split4_store(rec.q_hi + t * WR + 4 * c4, rec.q_lo + t * WR + 4 * c4, gam * qx);
        }
    }
    lds_barrier();

    /* K K^T and Q K^T over the 10 tiles on or below the block diagonal: 20
     * products, 5 per SIMD (waves w and w + 4 share one) */
    for (int u = wave; u < 2 * kLowerTiles; u += kPrepWaves) {
        const int p = u >> 1;
        const bool is_qk = u & 1;
        const int ti = lower_tile_row(p), tj = p - ti * (ti + 1) / 2;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        acc = q38_mma16_split<D>(acc, is_qk ? sQh + 16 * ti * WR : &sKh[16 * ti][0],
                                 is_qk ? sQl + 16 * ti * WR : &sKl[16 * ti][0], WR, &sKh[16 * tj][0],
                                 &sKl[16 * tj][0], WR);
#pragma unroll
        for (int i = 0; i < 4; ++i) (is_qk ? sQK : sKK)[p][4 * g4 + i][r] = acc[i];
    }
    lds_barrier();

#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
        const int vh = kh + Q38_LIN_QK_HEADS * j;
        const Record rec = record_of(a, s, vh, n);

        /* this head's G and betas (wave 0 publishes them) */
        if (wave == 0) {
            const float g_l = sG3[j][lane];
            const float beta_l = sBeta3[j][lane];
            const float g_last = __shfl(g_l, C - 1, 64);
            sG[lane] = g_l;
            sBeta[lane] = beta_l;
            sBG[lane] = beta_l * expf(g_l);
            sKd[lane] = expf(g_last - g_l);
            if (lane == 0) *rec.gamma_c = expf(g_last);
        }
        /* V^T of this head split into LDS; the next head's V rows load behind
         * the rest of this head's work */
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int t = row_t(p), c4 = col_c4();
            const f32x4 vx = live(p, vv[p]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const __bf16 h = (__bf16)vx[e];
                sVh[4 * c4 + e][t] = h;
                sVl[4 * c4 + e][t] = (__bf16)(vx[e] - (float)h);
            }
        }
        if (j + 1 < kGroup) load_v(vh + Q38_LIN_QK_HEADS);
        lds_barrier();

        /* A (strictly lower) into LDS and Bm (lower, with the diagonal; zero
         * above the diagonal blocks) out as bf16 hi/lo rows: thread (t, c8)
         * forms columns 8 c8 .. 8 c8 + 7 of row t */
        {
            const int t = tid >> 3, c8 = tid & 7;
            const int ti = t >> 4, tj = c8 >> 1;
            float bm[8];
            if (tj > ti) {
#pragma unroll
                for (int e = 0; e < 8; ++e) bm[e] = 0.0f;
            } else {
                const int p = ti * (ti + 1) / 2 + tj;
                const float gt = sG[t], bt = sBeta[t];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int sc = 8 * c8 + e;
                    const float dec = sc <= t ? expf(gt - sG[sc]) : 0.0f;
                    sA[t][sc] = sc < t ? bt * dec * sKK[p][t & 15][sc & 15] : 0.0f;
                    bm[e] = sc <= t ? dec * sQK[p][t & 15][sc & 15] : 0.0f;
                }
            }
            bf16x8 hi, lo;
            q38_split8(bm, hi, lo);
            *reinterpret_cast<bf16x8 *>(rec.b_hi + t * BR + 8 * c8) = hi;
            *reinterpret_cast<bf16x8 *>(rec.b_lo + t * BR + 8 * c8) = lo;
        }
        /* K'^T = (diag(exp(G_C - G)) K)^T by rows of 8 tokens, K read as hi + lo */
        for (int it = tid; it < D * (C / 8); it += kPrepThreads) {
            const int i = it & (D - 1), t8 = it >> 7;
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e)
                x[e] = sKd[8 * t8 + e] * ((float)sKh[8 * t8 + e][i] + (float)sKl[8 * t8 + e][i]);
            bf16x8 hi, lo;
            q38_split8(x, hi, lo);
            *reinterpret_cast<bf16x8 *>(rec.kt_hi + i * BR + 8 * t8) = hi;
            *reinterpret_cast<bf16x8 *>(rec.kt_lo + i * BR + 8 * t8) = lo;
        }
        lds_barrier();

        invert_unit_lower(sA, sT, wave, lane);

        /* the left operands of W and U' as bf16 hi/lo rows: T diag(beta gamma)
         * and T diag(beta) (over A, free now) */
        __bf16 *const t2h = reinterpret_cast<__bf16 *>(&sA[0][0]);
        __bf16 *const t2l = t2h + C * BR;
        {
            const int t = tid >> 3, c8 = tid & 7;
            float x1[8], x2[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float tv = sT[t][8 * c8 + e];
                x1[e] = tv * sBG[8 * c8 + e];
                x2[e] = tv * sBeta[8 * c8 + e];
            }
            bf16x8 hi, lo;
            q38_split8(x1, hi, lo);
            *reinterpret_cast<bf16x8 *>(&sWh[t][8 * c8]) = hi;
            *reinterpret_cast<bf16x8 *>(&sWl[t][8 * c8]) = lo;
            q38_split8(x2, hi, lo);
            *reinterpret_cast<bf16x8 *>(t2h + t * BR + 8 * c8) = hi;
            *reinterpret_cast<bf16x8 *>(t2l + t * BR + 8 * c8) = lo;
        }
        lds_barrier();

        /* W = T diag(beta gamma) K, out as bf16 hi/lo rows, and U' = T diag(beta) V
         * (f32 out): 32 + 32 tiles, 4 + 4 per wave.  W is formed transposed
         * (W^T = K^T (T diag(beta gamma))^T) so that a lane holds 4 adjacent
         * columns of a W row.  Token blocks 0 and 1 contract over tokens 0..31
         * only: T is lower triangular. */
        for (int tile = wave; tile < 64; tile += kPrepWaves) {
            const bool is_w = tile < 32;
            const int ti = (tile & 31) >> 3, tn = tile & 7;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            if (is_w) {
                if (ti < 2)
                    acc = mma16_split_acol<32>(acc, &sKh[0][16 * tn], &sKl[0][16 * tn], WR, &sWh[16 * ti][0],
                                               &sWl[16 * ti][0], BR);
                else
                    acc = mma16_split_acol<C>(acc, &sKh[0][16 * tn], &sKl[0][16 * tn], WR, &sWh[16 * ti][0],
                                              &sWl[16 * ti][0], BR);
                const int t = 16 * ti + r, col = 16 * tn + 4 * g4;
                split4_store(rec.w_hi + t * WR + col, rec.w_lo + t * WR + col, acc);
            } else {
                if (ti < 2)
                    acc = q38_mma16_split<32>(acc, t2h + 16 * ti * BR, t2l + 16 * ti * BR, BR, &sVh[16 * tn][0],
                                              &sVl[16 * tn][0], BR);
                else
                    acc = q38_mma16_split<C>(acc, t2h + 16 * ti * BR, t2l + 16 * ti * BR, BR, &sVh[16 * tn][0],
                                             &sVl[16 * tn][0], BR);
#pragma unroll
                for (int i = 0; i < 4; ++i) rec.u[(16 * ti + 4 * g4 + i) * D + 16 * tn + r] = acc[i];
            }
        }
        if (j + 1 < kGroup) lds_barrier(); /* the next head reuses every per-head array */
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
    __shared__ __attribute__((aligned(16))) float sUp[C][R]; /* the slab's columns of U' */

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
     * the step that reads it is done: W after step a, U' with Q' and Bm
     * after step b, K'^T after step c.  Each part is awaited only before the
     * step that reads it: W and U' before step a, Q' and Bm before step b,
     * K'^T before step c.  Waves 0-3 each move every 4th piece of a part; a
     * wave's waits count its own operations, and the barrier after the wait
     * makes the pieces of all waves visible (waves 4-7 move no pieces, so
     * their waits pass at once). */
    /* steps a and b: wave w computes token block ti of value-row block tb */
    const int ti = wave & 3;
    const int tb = wave >> 2;
    const bool mover = wave < 4;
    auto fetch = [&](const char *src, char *dst, auto n_pieces) {
        if (!mover) return;
#pragma unroll
        for (int j = 0; j < decltype(n_pieces)::value / 4; ++j) {
            const int p = 4 * j + wave;
            dma_piece(lds_address(dst + p * 1024), src, p * 1024 + lane * 16);
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
    /* U' columns c0 .. c0+31: piece j holds rows 8j .. 8j+7 (a lane gathers
     * 16 bytes of one row), 2 pieces per moving wave */
    auto fetch_u = [&](const Record &rec) {
        if (!mover) return;
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const int j = 4 * jj + wave;
            const int row = 8 * j + (lane >> 3);
            dma_piece(lds_address(&sUp[8 * j][0]), rec.u, (row * D + c0 + 4 * (lane & 7)) * 4);
        }
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
        const int t0 = (a.chunk0 + n) * C;
        const int cnt = min(C, a.n_tokens - t0);
        const size_t tok0 = (size_t)s * a.n_tokens + t0;
        const bool more = n + 1 < a.n_chunks;
        const Record next = record_of(a, s, vh, more ? n + 1 : n);

        /* a: U = U' - W S^T (64 x 32): wave w takes tile (ti, tb); U^T to LDS.
         * gamma_C is read here, before the next W overwrites the W part. */
        const float gamma_c = *reinterpret_cast<const float *>(imgW + kGammaOffset);
        {
            float up[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) up[i] = sUp[16 * ti + 4 * g4 + i][16 * tb + r];
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            acc = q38_mma16_split<D>(acc, li.w_hi + 16 * ti * WR, li.w_lo + 16 * ti * WR, WR, &sSh[16 * tb][0],
                                     &sSl[16 * tb][0], WR);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                split_store(&sUh[0][0], &sUl[0][0], (16 * tb + r) * BR + 16 * ti + 4 * g4 + i, up[i] - acc[i]);
        }
        /* U^T in LDS, W and U' free; this chunk's Q' and Bm have landed
         * (only its K'^T is younger) */
        q38_barrier_vm<kPiecesKt / 4>();
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
            fetch_u(next);
            fetch_qb(next);
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
                S[q][i] = __builtin_fmaf(gamma_c, S[q][i], acc[i]);
                split_store(&sSh[0][0], &sSl[0][0], (16 * tc + 4 * g4 + i) * WR + 16 * tk + r, S[q][i]);
            }
        }
        q38_barrier_vm<63>(); /* the new S in LDS; K'^T free */
        if (more) {
            fetch_kt(next);
            /* the next W and U'; its Q', Bm and K'^T stay in flight into
             * step a */
            q38_barrier_vm<(kPiecesQB + kPiecesKt) / 4>();
        }
    }

#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int tile = 2 * wave + q, tc = tile >> 3, tk = tile & 7;
#pragma unroll
        for (int i = 0; i < 4; ++i) st[(16 * tc + 4 * g4 + i) * D + 16 * tk + r] = S[q][i];
    }
}

/* Gated RMSNorm (ops.rs:735-740) of (token, value head) rows: rmsnorm of the
 * 128 outputs with the f64 sum of squares, weight, times silu(z).  grid
 * (n_rows / 16), 256 threads: each wave takes 4 rows, a half-wave one row
 * at a time with 4 consecutive columns per lane, both rows' loads issued
 * before the first reduction. */
extern "C" __global__ __launch_bounds__(256) void q38_gdn_post(q38_gdn_post_args a) {
    const int lane = threadIdx.x & 63;
    const int col = 4 * (lane & 31);
    const size_t row0 = ((size_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 4 + (lane >> 5);
    const f32x4 nw = q38_ld4(a.norm_w + col);
    f32x4 x[2], z[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const size_t at = (row0 + 2 * p) * D + col;
        x[p] = q38_ld4(a.o + at);
        z[p] = q38_ld4(a.z + at);
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        double ss = (double)x[p].x * (double)x[p].x + (double)x[p].y * (double)x[p].y +
                    (double)x[p].z * (double)x[p].z + (double)x[p].w * (double)x[p].w;
#pragma unroll
        for (int m = 16; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
        const float mean = (float)(ss / (double)D);
        const float scale = 1.0f / sqrtf(mean + 1e-6f);
        f32x4 y;
        y.x = x[p].x * scale * nw.x;
        y.y = x[p].y * scale * nw.y;
        y.z = x[p].z * scale * nw.z;
        y.w = x[p].w * scale * nw.w;
        y.x *= q38_silu(z[p].x);
        y.y *= q38_silu(z[p].y);
        y.z *= q38_silu(z[p].z);
        y.w *= q38_silu(z[p].w);
        q38_st4(a.out + (row0 + 2 * p) * D + col, y);
    }
}
