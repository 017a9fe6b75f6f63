/*
 * Causal prefill attention over the paged KV cache on bf16 MFMA (gfx950).
 *
 * Reference semantics: batch_full_attention (src/model/ops.rs:1153-1172)
 * calls full_core for tokens base, base+1, ... in order, so token t attends
 * over positions 0..base+t (ops.rs:879-913) and is gated by sigmoid(gate)
 * (ops.rs:914-917).  Scores are q.k / 16, softmax in f32.
 *
 * Precision: every f32 operand x is split into bf16 hi = bf16(x) and
 * lo = bf16(x - hi), and each product is hi*hi + hi*lo + lo*hi on
 * v_mfma_f32_16x16x32_bf16 with f32 accumulation: the represented value is
 * within ~2^-16 of x, far inside the 1e-3 output bound that plain bf16
 * (2^-8) would miss.
 *
 * Layout (wave64, v_mfma_f32_16x16x32_bf16: A lane l = row l%16, k =
 * 8(l/16)..+7; B lane l = column l%16, same k; C lane l = rows 4(l/16)+i,
 * column l%16):
 *  - a workgroup serves 32 query tokens of all 6 query heads of kv head j
 *    from one copy of each K/V block: 12 (head, 16-query) tiles over 4 waves
 *    (one per SIMD, so 512 registers per lane hold 3 tiles' Q and O), and
 *    each K or V fragment read from LDS feeds 3 tiles x 3 MFMAs;
 *  - scores are computed transposed, S^T = K Q^T (A = K rows from LDS, B =
 *    Q^T from registers), so lane (g = l/16, c = l%16) holds query c's
 *    scores for keys 16kt + 4g + i -- exactly the P values it supplies as
 *    the A operand of O += P V when the key order inside the 32-key block
 *    is permuted to slot 8g + 4kt + i; V is stored transposed in LDS in that
 *    slot order, so P never leaves registers;
 *  - q38_kv_split_mfma first splits the prompt's K/V (f32 pages) once into
 *    bf16 hi/lo block images laid out exactly as the LDS tile (V already
 *    transposed and slot-permuted); the attention kernel moves each 32-key
 *    image HBM -> LDS with direct-to-LDS loads one block ahead
 *    (double-buffered), one barrier per block, no conversion in its loop;
 *  - online softmax in base 2 per query row; the rows' max and sum cross the
 *    4 lane groups with permlane swaps.
 */
#include "q38_device.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

/* 1/sqrt(256) (ops.rs:869) times log2(e). */
#define Q38_SCORE_LOG2 0.09016844005556021f

namespace {

constexpr int kQ = Q38_PREFILL_QUERIES;   /* query tokens per workgroup */
constexpr int kWaves = 4;                 /* one per SIMD: 512 registers per lane */
constexpr int kTiles = Q38_ATTN_GROUP * (kQ / 16) / kWaves; /* (head, 16-query) tiles per wave: 3 */
constexpr int kKB = Q38_PREFILL_KEYS;     /* keys per block */
constexpr int kKRow = Q38_PREFILL_KROW;   /* bf16 per K row: 16 B pad, conflict-free b128 reads */
constexpr int kVRow = Q38_PREFILL_VROW;   /* bf16 per transposed V row (one head dim) */
constexpr int kThreads = 64 * kWaves;
constexpr int kPieces = Q38_PREFILL_IMAGE_BYTES / 1024; /* 1 KiB direct-to-LDS pieces of an image */
static_assert(Q38_PREFILL_IMAGE_BYTES % 1024 == 0, "image in 1 KiB pieces");
static_assert(kTiles * kWaves == Q38_ATTN_GROUP * (kQ / 16), "tiles cover the group");

struct Split4 {
    bf16x4 hi, lo;
};

Q38_DEV Split4 split4(f32x4 x) {
    Split4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const __bf16 h = (__bf16)x[e];
        r.hi[e] = h;
        r.lo[e] = (__bf16)(x[e] - (float)h);
    }
    return r;
}

/* slot of key k (0..31) inside a block: 8g + 4kt + i for k = 16kt + 4g + i */
Q38_DEV int key_slot(int k) { return 8 * ((k & 15) >> 2) + 4 * (k >> 4) + (k & 3); }

Q38_DEV float max_over_groups(float x) {
    x = fmaxf(x, __shfl_xor(x, 16, 64));
    return fmaxf(x, __shfl_xor(x, 32, 64));
}

Q38_DEV float sum_over_groups(float x) {
    x += __shfl_xor(x, 16, 64);
    return x + __shfl_xor(x, 32, 64);
}

/* Element offset of key position kp (clamped to the last needed one) in
 * kv head j's pages. */
Q38_DEV size_t key_row(const q38_prefill_args &a, int j, int kp, int kmax) {
    kp = min(kp, kmax);
    const int phys = a.page_table[kp >> 4];
    return ((size_t)phys * Q38_ATTN_KV_HEADS + j) * Q38_PAGE_TOKENS * Q38_ATTN_HEAD_DIM +
           (size_t)(kp & 15) * Q38_ATTN_HEAD_DIM;
}

/* The LDS tile of one block, and the image of the same bytes in HBM. */
struct Tile {
    __bf16 k[2][kKB][kKRow];                /* [hi/lo][key][dim] */
    __bf16 vt[2][Q38_ATTN_HEAD_DIM][kVRow]; /* [hi/lo][dim][key slot] */
};
static_assert(sizeof(Tile) == Q38_PREFILL_IMAGE_BYTES, "tile and image agree");

Q38_DEV const uint4 *image_of(const q38_prefill_args &a, int j, int kb) {
    return reinterpret_cast<const uint4 *>(static_cast<const char *>(a.images) +
                                           ((size_t)j * a.n_kblocks + kb) * Q38_PREFILL_IMAGE_BYTES);
}

}  // namespace

/* Split K/V blocks 0 .. n_kblocks-1 of kv head blockIdx.y into bf16 hi/lo
 * block images (grid (n_kblocks, 4), 256 threads).  Keys past the prompt's
 * last position read that position (finite data; the causal mask gives them
 * weight 0 in every row that can see them). */
extern "C" __global__ __launch_bounds__(256) void q38_kv_split_mfma(q38_prefill_args a) {
    const int kb = blockIdx.x;
    const int j = blockIdx.y;
    const int tid = threadIdx.x;
    const int kmax = a.base_pos + a.n_tokens - 1;
    Tile *img = reinterpret_cast<Tile *>(static_cast<char *>(a.images) +
                                         ((size_t)j * a.n_kblocks + kb) * Q38_PREFILL_IMAGE_BYTES);
    for (int i = tid; i < kKB * Q38_ATTN_HEAD_DIM / 4; i += 256) {
        const int r = i >> 6, c4 = i & 63;
        const Split4 sp = split4(q38_ld4(a.kpool + key_row(a, j, kb * kKB + r, kmax) + 4 * c4));
        *reinterpret_cast<bf16x4 *>(&img->k[0][r][4 * c4]) = sp.hi;
        *reinterpret_cast<bf16x4 *>(&img->k[1][r][4 * c4]) = sp.lo;
    }
    for (int i = tid; i < kKB / 2 * Q38_ATTN_HEAD_DIM / 4; i += 256) {
        const int r = 2 * (i >> 6), c4 = i & 63;
        const int slot = key_slot(r); /* key r+1 sits at slot + 1 */
        const Split4 s0 = split4(q38_ld4(a.vpool + key_row(a, j, kb * kKB + r, kmax) + 4 * c4));
        const Split4 s1 = split4(q38_ld4(a.vpool + key_row(a, j, kb * kKB + r + 1, kmax) + 4 * c4));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int d = 4 * c4 + e;
            *reinterpret_cast<bf16x2 *>(&img->vt[0][d][slot]) = bf16x2{s0.hi[e], s1.hi[e]};
            *reinterpret_cast<bf16x2 *>(&img->vt[1][d][slot]) = bf16x2{s0.lo[e], s1.lo[e]};
        }
    }
}

extern "C" __global__ __launch_bounds__(kThreads, 1) void q38_attn_prefill_mfma(q38_prefill_args a) {
    __shared__ __attribute__((aligned(16))) Tile tiles[2];

    /* workgroup -> (kv head, query block): consecutive workgroups go to the
     * 8 XCDs in turn, so XCDs 2j and 2j+1 take kv head j and its K/V blocks
     * stay in those two L2s; the longest causal rows start first */
    const int L = blockIdx.x;
    const int nq = a.n_qblocks;
    int j, qi;
    if ((nq & 1) == 0) {
        j = (L & 7) >> 1;
        qi = (L >> 3) * 2 + (L & 1);
    } else {
        j = L & 3;
        qi = L >> 2;
    }
    const int qb = nq - 1 - qi;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4;
    const int c = lane & 15;
    const int qt0 = qb * kQ;                            /* first query token of the block */
    const int q_last = min(qt0 + kQ, a.n_tokens) - 1;   /* last real query token */
    const int kmax = a.base_pos + q_last;               /* last key position any row needs */
    const int n_kb = kmax / kKB + 1;

    /* the wave's tiles: (head, 16-query tile) combos 3w .. 3w+2 of the 12 */
    int head[kTiles], q0[kTiles], qpos[kTiles];
    bf16x8 q_hi[kTiles][8], q_lo[kTiles][8];
#pragma unroll
    for (int u = 0; u < kTiles; ++u) {
        const int combo = kTiles * wave + u;
        head[u] = j * Q38_ATTN_GROUP + (combo >> 1);
        q0[u] = qt0 + 16 * (combo & 1);
        qpos[u] = a.base_pos + q0[u] + c;
        const int tq = min(q0[u] + c, q_last);
        const float *qp = a.q + ((size_t)tq * Q38_ATTN_HEADS + head[u]) * Q38_ATTN_HEAD_DIM + 8 * g;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            const Split4 s0 = split4(q38_ld4(qp + 32 * kk));
            const Split4 s1 = split4(q38_ld4(qp + 32 * kk + 4));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                q_hi[u][kk][e] = s0.hi[e];
                q_hi[u][kk][4 + e] = s1.hi[e];
                q_lo[u][kk][e] = s0.lo[e];
                q_lo[u][kk][4 + e] = s1.lo[e];
            }
        }
    }

    float m[kTiles], l[kTiles];
    f32x4 O[kTiles][16];
#pragma unroll
    for (int u = 0; u < kTiles; ++u) {
        m[u] = -INFINITY;
        l[u] = 0.0f;
#pragma unroll
        for (int n = 0; n < 16; ++n) O[u][n] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    /* block images go HBM -> LDS by direct-to-LDS loads (no registers):
     * wave w moves 1 KiB pieces w, w+4, ...; lane l's 16 bytes land at the
     * piece's LDS base + 16 l */
    auto fetch = [&](int kb, int buf) {
        const char *img = reinterpret_cast<const char *>(image_of(a, j, kb));
        char *dst = reinterpret_cast<char *>(&tiles[buf]);
        for (int p = wave; p < kPieces; p += kWaves)
            __builtin_amdgcn_global_load_lds(img + p * 1024 + lane * 16,
                                             (__attribute__((address_space(3))) void *)(dst + p * 1024), 16, 0, 0);
    };
    fetch(0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    for (int kb = 0; kb < n_kb; ++kb) {
        const int buf = kb & 1;
        if (kb + 1 < n_kb) fetch(kb + 1, buf ^ 1);

        /* S^T tiles: s[u][kt][i] = score of the tile's query c and key 16kt + 4g + i;
         * each K fragment read from LDS feeds 3 tiles x 3 products */
        f32x4 s[kTiles][2];
#pragma unroll
        for (int u = 0; u < kTiles; ++u)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) s[u][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                const bf16x8 kh = *reinterpret_cast<const bf16x8 *>(&tiles[buf].k[0][16 * kt + c][32 * kk + 8 * g]);
                const bf16x8 kl = *reinterpret_cast<const bf16x8 *>(&tiles[buf].k[1][16 * kt + c][32 * kk + 8 * g]);
#pragma unroll
                for (int u = 0; u < kTiles; ++u) {
                    s[u][kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, q_hi[u][kk], s[u][kt], 0, 0, 0);
                    s[u][kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, q_lo[u][kk], s[u][kt], 0, 0, 0);
                    s[u][kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl, q_hi[u][kk], s[u][kt], 0, 0, 0);
                }
                /* keep each fragment's LDS read inside its step (hoisting them
                 * all would need 128 more registers) */
                __builtin_amdgcn_sched_barrier(0);
            }
        }

        bf16x8 p_hi[kTiles], p_lo[kTiles];
#pragma unroll
        for (int u = 0; u < kTiles; ++u) {
            /* scale, causal mask, block max of the row */
            float bm = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int key = kb * kKB + 16 * kt + 4 * g + i;
                    const float x = key <= qpos[u] ? s[u][kt][i] * Q38_SCORE_LOG2 : -INFINITY;
                    s[u][kt][i] = x;
                    bm = fmaxf(bm, x);
                }
            bm = max_over_groups(bm);
            const float m_new = fmaxf(m[u], bm); /* finite: key 0 is in every row's block 0 */
            const float f = q38_exp2(m[u] - m_new); /* 0 while m is -inf */
            float ps = 0.0f;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float p = q38_exp2(s[u][kt][i] - m_new);
                    ps += p;
                    const __bf16 ph = (__bf16)p;
                    p_hi[u][4 * kt + i] = ph;
                    p_lo[u][4 * kt + i] = (__bf16)(p - (float)ph);
                }
            l[u] = l[u] * f + sum_over_groups(ps);
            m[u] = m_new;
            /* rescale O: lane (g, c) holds rows 4g+i, whose factor lives in lane 4g+i */
            if (__any(f != 1.0f)) {
                float fr[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) fr[i] = __shfl(f, 4 * g + i, 64);
#pragma unroll
                for (int n = 0; n < 16; ++n)
#pragma unroll
                    for (int i = 0; i < 4; ++i) O[u][n][i] *= fr[i];
            }
        }

        /* O += P V: B = V^T rows (head dims 16n + c), key slots 8g .. 8g+7;
         * each V fragment feeds 3 tiles x 3 products */
#pragma unroll
        for (int n = 0; n < 16; ++n) {
            const bf16x8 vh = *reinterpret_cast<const bf16x8 *>(&tiles[buf].vt[0][16 * n + c][8 * g]);
            const bf16x8 vl = *reinterpret_cast<const bf16x8 *>(&tiles[buf].vt[1][16 * n + c][8 * g]);
#pragma unroll
            for (int u = 0; u < kTiles; ++u) {
                O[u][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(p_hi[u], vh, O[u][n], 0, 0, 0);
                O[u][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(p_hi[u], vl, O[u][n], 0, 0, 0);
                O[u][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(p_lo[u], vh, O[u][n], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }

        /* the next block's pieces have landed (this wave's), and every wave is
         * done with this block */
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    }

    /* normalise, gate, store rows 4g+i of each tile */
#pragma unroll
    for (int u = 0; u < kTiles; ++u) {
        float inv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) inv[i] = 1.0f / __shfl(l[u], 4 * g + i, 64);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = q0[u] + 4 * g + i;
            if (t > q_last) continue;
            const size_t row = ((size_t)t * Q38_ATTN_HEADS + head[u]) * Q38_ATTN_HEAD_DIM;
#pragma unroll
            for (int n = 0; n < 16; ++n) {
                const int d = 16 * n + c;
                float r = O[u][n][i] * inv[i];
                if (a.gate != nullptr) r *= q38_sigmoid(a.gate[row + d]);
                a.out[row + d] = r;
            }
        }
    }
}
