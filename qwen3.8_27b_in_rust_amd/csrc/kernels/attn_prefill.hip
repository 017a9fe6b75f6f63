/*
 * Causal prefill attention over the paged KV cache on bf16 MFMA (gfx950).
 *
 * Reference semantics: batch_full_attention (src/model/ops.rs:1153-1172)
 * calls full_core for tokens base, base+1, ... in order, so token t attends
 * over positions 0..base+t (ops.rs:879-913) and is gated by sigmoid(gate)
 * (ops.rs:914-917).  Scores are q.k / 16, softmax in f32.
 *
 * Precision: every f32 operand x is split into bf16 hi = bf16(x) and
 * lo = bf16(x - hi), and each product is hi*hi + hi*lo + lo*hi with f32
 * accumulation: the represented value is within ~2^-16 of x, far inside
 * the 1e-3 output bound that plain bf16 (2^-8) would miss.
 *
 * Layout (wave64, v_mfma_f32_32x32x16_bf16: A lane l = row l%32, k =
 * 8(l/32)..+7; B lane l = column l%32, same k; C lane l = column l%32,
 * element 4J+i = row 8J + 4(l/32) + i):
 *  - a workgroup serves 64 query tokens of 2 query heads of kv head j; each
 *    wave owns 32 tokens x 1 head: its Q (bf16 hi/lo, 128 registers) and
 *    its O (32 x 256 f32, 128 accumulation registers), no spills;
 *  - scores are computed transposed, S^T = K Q^T (A = K rows from LDS, B =
 *    Q^T from registers), so lane l holds query l%32's scores for keys
 *    8J + 4(l/32) + i -- the P values it supplies as the A operand of
 *    O += P V once the keys of a 32-key block are permuted to slot
 *    16(J/2) + 8(l/32) + 4(J%2) + i; V is stored transposed in LDS in that
 *    slot order, so P never leaves registers;
 *  - q38_kv_split_mfma first splits the prompt's K/V (f32 pages) once into
 *    bf16 hi/lo block images laid out exactly as the LDS tile (V already
 *    transposed and slot-permuted); the attention kernel moves each 32-key
 *    image HBM -> LDS with direct-to-LDS loads one block ahead
 *    (double-buffered), one barrier per block, no conversion in its loop;
 *  - softmax in base 2 against a fixed per-query reference max (the max
 *    over the first key block), so O is never rescaled; the two lane halves
 *    of a query combine with v_permlane32_swap; a block whose scores pass
 *    the reference by more than 2^64 restarts the workgroup's key loop with
 *    a raised reference (kRefSlack below); blocks wholly after a wave's
 *    queries are skipped, and only diagonal blocks are masked;
 *  - the loads of block kb+1's image are issued between the MFMA steps of
 *    block kb, so the direct-to-LDS traffic runs under the matrix work.
 */
#include "q38_device.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

/* 1/sqrt(256) (ops.rs:869) times log2(e). */
#define Q38_SCORE_LOG2 0.09016844005556021f

namespace {

constexpr int kQ = Q38_PREFILL_QUERIES;   /* query tokens per workgroup */
constexpr int kQW = 32;                   /* query tokens per wave */
constexpr int kWaves = 4;                 /* 2 heads x 2 token halves */
constexpr int kKB = Q38_PREFILL_KEYS;     /* keys per block */
constexpr int kKRow = Q38_PREFILL_KROW;   /* bf16 per K row: 16 B pad, conflict-free b128 reads */
constexpr int kVRow = Q38_PREFILL_VROW;   /* bf16 per transposed V row (one head dim) */
constexpr int kThreads = 64 * kWaves;
constexpr int kPieces = Q38_PREFILL_IMAGE_BYTES / 1024; /* 1 KiB direct-to-LDS pieces of an image */
/* A query's reference max m is its max over the first key block (which
 * holds key 0, visible to every query) and O is never rescaled: weights
 * exp2(s - m) stay <= 2^kRefSlack while no later score passes m by more, so
 * sums over 2^20 keys stay < 2^84, and the largest score's weight is >= 1.
 * A block whose max does pass m + kRefSlack for some query raises that
 * query's m and restarts the workgroup's key loop from block 0 (with O and
 * l cleared) -- never for scores of RMS-normalised q and k, which span a
 * few tens of log2 units. */
constexpr float kRefSlack = 64.0f;
static_assert(Q38_PREFILL_IMAGE_BYTES % 1024 == 0, "image in 1 KiB pieces");
static_assert(kQ == 2 * kQW && kWaves == 4 && kKB == 32, "2 heads x 2 halves of 32 tokens, 32-key blocks");
static_assert(2 * Q38_PREFILL_HEAD_PAIRS == Q38_ATTN_GROUP, "head pairs cover the group");

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

/* slot of key k = 8J + 4h + i (J < 4, h < 2, i < 4) inside a block: the
 * 8 keys lane half h supplies for k-step t of O += P V (J = 2t, 2t+1) sit
 * at slots 16t + 8h .. 16t + 8h + 7 */
Q38_DEV int key_slot(int k) {
    const int J = k >> 3, h = (k >> 2) & 1, i = k & 3;
    return 16 * (J >> 1) + 8 * h + 4 * (J & 1) + i;
}

/* The LDS tile of one block, and the image of the same bytes in HBM. */
struct Tile {
    __bf16 k[2][kKB][kKRow];                /* [hi/lo][key][dim] */
    __bf16 vt[2][Q38_ATTN_HEAD_DIM][kVRow]; /* [hi/lo][dim][key slot] */
};
static_assert(sizeof(Tile) == Q38_PREFILL_IMAGE_BYTES, "tile and image agree");

Q38_DEV const uint4 *image_of(const q38_prefill_args &a, int j, int kb) {
    return reinterpret_cast<const uint4 *>(static_cast<const char *>(a.images) +
                                           ((size_t)j * a.img_stride + kb) * Q38_PREFILL_IMAGE_BYTES);
}

}  // namespace

/* Split K/V blocks kb0 .. n_kblocks-1 of kv head blockIdx.y into bf16 hi/lo
 * block images (grid (n_kblocks - kb0, 4), 256 threads; blocks before kb0
 * hold images of unchanged keys from earlier calls).  Keys past the prompt's
 * last position read that position (finite data; the causal mask gives them
 * weight 0 in every row that can see them).  The K part goes out row by row;
 * the transposed V part is assembled in LDS (a 4-byte write per key pair and
 * dim) and then streamed to the image in 16-byte stores, so neither part is
 * written with scattered small stores. */
extern "C" __global__ __launch_bounds__(256) void q38_kv_split_mfma(q38_prefill_args a) {
    __shared__ __attribute__((aligned(16))) __bf16 vimg[2][Q38_ATTN_HEAD_DIM][kVRow];
    const int kb = a.kb0 + blockIdx.x;
    const int j = blockIdx.y;
    const int tid = threadIdx.x;
    const int kmax = a.base_pos + a.n_tokens - 1;
    Tile *img = reinterpret_cast<Tile *>(static_cast<char *>(a.images) +
                                         ((size_t)j * a.img_stride + kb) * Q38_PREFILL_IMAGE_BYTES);
    /* the block's two page ids first, then every K and V row load of this
     * thread at once (one memory round trip each, where a copy loop would
     * wait for each page id and row in turn).  Keys past the last position
     * read it: key r is at min(kb*32 + r, kmax), whose page is the block's
     * first for r < 16 and its second otherwise. */
    const int kp0 = kb * kKB;
    const int pg0 = a.page_table[min(kp0, kmax) >> 4];
    const int pg1 = a.page_table[min(kp0 + 16, kmax) >> 4];
    auto row_of = [&](const float *pool, int r) {
        const int kp = min(kp0 + r, kmax);
        return pool + ((size_t)(r < 16 ? pg0 : pg1) * Q38_ATTN_KV_HEADS + j) * Q38_PAGE_TOKENS * Q38_ATTN_HEAD_DIM +
               (size_t)(kp & 15) * Q38_ATTN_HEAD_DIM;
    };
    constexpr int kKPer = kKB * Q38_ATTN_HEAD_DIM / 4 / 256;     /* K float4s per thread */
    constexpr int kVPer = kKB / 2 * Q38_ATTN_HEAD_DIM / 4 / 256; /* V key pairs per thread */
    f32x4 kx[kKPer], vx[2 * kVPer];
#pragma unroll
    for (int m = 0; m < kKPer; ++m) {
        const int i = tid + 256 * m;
        kx[m] = q38_ld4(row_of(a.kpool, i >> 6) + 4 * (i & 63));
    }
#pragma unroll
    for (int m = 0; m < kVPer; ++m) {
        const int i = tid + 256 * m;
        const int r = 2 * (i >> 6), c4 = i & 63;
        vx[2 * m] = q38_ld4(row_of(a.vpool, r) + 4 * c4);
        vx[2 * m + 1] = q38_ld4(row_of(a.vpool, r + 1) + 4 * c4);
    }
#pragma unroll
    for (int m = 0; m < kKPer; ++m) {
        const int i = tid + 256 * m;
        const int r = i >> 6, c4 = i & 63;
        const Split4 sp = split4(kx[m]);
        *reinterpret_cast<bf16x4 *>(&img->k[0][r][4 * c4]) = sp.hi;
        *reinterpret_cast<bf16x4 *>(&img->k[1][r][4 * c4]) = sp.lo;
    }
#pragma unroll
    for (int m = 0; m < kVPer; ++m) {
        const int i = tid + 256 * m;
        const int r = 2 * (i >> 6), c4 = i & 63;
        const int slot = key_slot(r); /* key r+1 sits at slot + 1 */
        const Split4 s0 = split4(vx[2 * m]);
        const Split4 s1 = split4(vx[2 * m + 1]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int d = 4 * c4 + e;
            *reinterpret_cast<bf16x2 *>(&vimg[0][d][slot]) = bf16x2{s0.hi[e], s1.hi[e]};
            *reinterpret_cast<bf16x2 *>(&vimg[1][d][slot]) = bf16x2{s0.lo[e], s1.lo[e]};
        }
    }
    __syncthreads();
    /* the V part, padding included, as 16-byte pieces */
    const uint4 *src = reinterpret_cast<const uint4 *>(&vimg[0][0][0]);
    uint4 *dst = reinterpret_cast<uint4 *>(&img->vt[0][0][0]);
    for (int i = tid; i < (int)(sizeof(vimg) / 16); i += 256) dst[i] = src[i];
}

extern "C" __global__ __launch_bounds__(kThreads, 1) void q38_attn_prefill_mfma(q38_prefill_args a) {
    __shared__ __attribute__((aligned(16))) Tile tiles[2];
    /* a wave whose block passed its reference max sets the flag of the
     * block's parity; every wave reads it after the block's barrier */
    __shared__ int restart_flag[2];
    if (threadIdx.x < 2) restart_flag[threadIdx.x] = 0;

    /* Jobs: (kv head j, head pair, query block).  Consecutive workgroups go
     * to the 8 XCDs in turn, so XCDs 2j and 2j+1 take kv head j and its K/V
     * images stay in those two L2s.  With a job table (jobs_per_wg > 0) the
     * grid is 4 kv heads x Q38_PREFILL_BINS workgroups and each runs the jobs
     * the host placed in its bin, so that every CU gets the same number of key
     * blocks; without one, one job per workgroup, the longest causal rows
     * first, the 3 head pairs of a query block side by side. */
    const int L = blockIdx.x;
    const int nq = a.n_qblocks;
    const int n_jobs = a.jobs_per_wg > 0 ? a.jobs_per_wg : 1;
    for (int job = 0; job < n_jobs; ++job) {
        int j, hp, qb;
        int kb_begin = 0, kb_stop = -1; /* the job's key blocks (-1: up to the diagonal) */
        int slot = -1;                  /* a piece's partial slot (-1: the whole job) */
        if (a.jobs_per_wg > 0) {
            j = (L & 7) >> 1;
            const q38_prefill_job jb = a.jobs[(2 * (L >> 3) + (L & 1)) * a.jobs_per_wg + job];
            if (jb.code == 0xFFFF) break; /* the bin's jobs are done (the same for every wave) */
            hp = jb.code >> 6;
            qb = jb.code & 63;
            kb_begin = jb.kb0;
            kb_stop = jb.kb1;
            if (jb.slot != 0xFFFF) slot = jb.slot;
        } else {
            int c;
            if ((nq & 1) == 0) {
                j = (L & 7) >> 1;
                c = 2 * (L >> 3) + (L & 1);
            } else {
                j = L & 3;
                c = L >> 2;
            }
            const int qi = c / Q38_PREFILL_HEAD_PAIRS;
            hp = c - Q38_PREFILL_HEAD_PAIRS * qi;
            qb = nq - 1 - qi;
        }
        const int tid = threadIdx.x;
        const int lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int h = lane >> 5;  /* lane half */
        const int col = lane & 31;
        const int head = j * Q38_ATTN_GROUP + 2 * hp + (wave & 1);
        const int q0 = qb * kQ + kQW * (wave >> 1);      /* the wave's first query token */
        const int q_last = min(qb * kQ + kQ, a.n_tokens) - 1; /* last real query token of the block */
        const int kmax = a.base_pos + q_last;            /* last key position any row needs */
        /* a piece stops before the diagonal; its first block, like block 0,
         * is seen whole by every row of the job (the host splits so) */
        const int n_kb = kb_stop >= 0 ? kb_stop : kmax / kKB + 1;
        const bool active = q0 <= q_last;                /* the wave has real rows */
        const int pos_first = a.base_pos + q0;           /* the wave's first row's position */
        const int pos_last = a.base_pos + min(q0 + kQW - 1, q_last);
        const int qpos = a.base_pos + q0 + col;          /* this lane's query column */

        /* Q^T as the B operand: lane l holds query col, dims 16ks + 8h .. +7 */
        bf16x8 q_hi[16], q_lo[16];
        {
            const int tq = min(q0 + col, q_last);
            const float *qp = a.q + ((size_t)tq * Q38_ATTN_HEADS + head) * Q38_ATTN_HEAD_DIM + 8 * h;
#pragma unroll
            for (int ks = 0; ks < 16; ++ks) {
                /* scaled to base-2 score units before the split */
                const Split4 s0 = split4(q38_ld4(qp + 16 * ks) * Q38_SCORE_LOG2);
                const Split4 s1 = split4(q38_ld4(qp + 16 * ks + 4) * Q38_SCORE_LOG2);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    q_hi[ks][e] = s0.hi[e];
                    q_hi[ks][4 + e] = s1.hi[e];
                    q_lo[ks][e] = s0.lo[e];
                    q_lo[ks][4 + e] = s1.lo[e];
                }
                /* opaque to the compiler, which would otherwise keep f32 Q and
                 * split it again in every block; held in accumulation registers
                 * (the matrix unit reads its B operand from them), which leaves
                 * the vector registers to the scores, P and the fragments */
                asm volatile("" : "+a"(q_hi[ks]), "+a"(q_lo[ks]));
            }
        }

        float m = -INFINITY; /* query col's reference, in both lane halves */
        float l = 0.0f;       /* the sum of this lane's weights (its half of the keys) */
        f32x16 O[8];                   /* O[n][4J+i] = row 8J+4h+i, dim 32n + col */
        /* zeros made by the matrix unit (0 x 0 + 0), so the accumulators start,
         * and stay, in accumulation registers */
        auto clear_o = [&]() {
            const bf16x8 z = {};
            f32x16 zc;
#pragma unroll
            for (int v = 0; v < 16; ++v) zc[v] = 0.0f;
#pragma unroll
            for (int n = 0; n < 8; ++n) O[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(z, z, zc, 0, 0, 0);
        };
        clear_o();

        /* block images go HBM -> LDS by direct-to-LDS loads (no registers):
         * wave w moves 1 KiB pieces w, w+4, ...; lane l's 16 bytes land at the
         * piece's LDS base + 16 l.  Written as assembly so the compiler's
         * wait-count pass does not see them: it cannot tell the two buffers
         * apart and would wait for the next block's image before the first read
         * of the current one.  The loop waits for them itself (s_waitcnt 0 and
         * the barrier that ends each block).  M0 carries the LDS address; nothing
         * else in the kernel uses M0. */
        auto fetch = [&](int kb, int buf) {
            const char *img = reinterpret_cast<const char *>(image_of(a, j, kb));
            char *dst = reinterpret_cast<char *>(&tiles[buf]);
            for (int p = wave; p < kPieces; p += kWaves) {
                const uint32_t lds = (uint32_t)(size_t)(__attribute__((address_space(3))) char *)(dst + p * 1024);
                /* one wait state between the M0 write and the load that reads it */
                asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds),
                             "v"(img + p * 1024 + lane * 16)
                             : "memory");
            }
        };
        fetch(kb_begin, 0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();

        /* this wave's share of an image: pieces wave + 4i, i < kMyPieces */
        constexpr int kMyPieces = (kPieces + kWaves - 1) / kWaves;
        static_assert(kMyPieces <= 16 + 3, "pieces fit the QK steps and the first PV steps");

        int kb = kb_begin;
        while (kb < n_kb) {
            const int buf = (kb - kb_begin) & 1;
            /* The next block's image is loaded a piece at a time between the
             * matrix instructions below: issued all at once, 75 KB per workgroup
             * queue behind the CU's memory path and stall every wave before its
             * first product. */
            const bool prefetch = kb + 1 < n_kb;
            const char *next_img = reinterpret_cast<const char *>(image_of(a, j, min(kb + 1, n_kb - 1)));
            char *next_dst = reinterpret_cast<char *>(&tiles[buf ^ 1]);
            auto piece = [&](int i) {
                const int p = wave + kWaves * i;
                if (prefetch && p < kPieces) {
                    const uint32_t lds = (uint32_t)(size_t)(__attribute__((address_space(3))) char *)(next_dst + p * 1024);
                    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds),
                                 "v"(next_img + p * 1024 + lane * 16)
                                 : "memory");
                }
            };
            const int key0 = kb * kKB;
            const bool computes = active && key0 <= pos_last;
            if (!computes)
                for (int i = 0; i < kMyPieces; ++i) piece(i);
            float bm = -INFINITY; /* this block's max for query col (if computed) */

            if (computes) {
                /* K fragments are read kAhead steps before their products, so
                 * the LDS latency hides behind the matrix work */
                constexpr int kAhead = 4;
                f32x16 s;
#pragma unroll
                for (int v = 0; v < 16; ++v) s[v] = 0.0f;
                bf16x8 kh[kAhead + 1], kl[kAhead + 1];
                auto read_k = [&](int ks, int r) {
                    kh[r] = *reinterpret_cast<const bf16x8 *>(&tiles[buf].k[0][col][16 * ks + 8 * h]);
                    kl[r] = *reinterpret_cast<const bf16x8 *>(&tiles[buf].k[1][col][16 * ks + 8 * h]);
                };
#pragma unroll
                for (int ks = 0; ks < kAhead; ++ks) read_k(ks, ks);
#pragma unroll
                for (int ks = 0; ks < 16; ++ks) {
                    if (ks + kAhead < 16) read_k(ks + kAhead, (ks + kAhead) % (kAhead + 1));
                    piece(ks);
                    const int r = ks % (kAhead + 1);
                    s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh[r], q_hi[ks], s, 0, 0, 0);
                    s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh[r], q_lo[ks], s, 0, 0, 0);
                    s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kl[r], q_hi[ks], s, 0, 0, 0);
                    /* keep the steps in this order: hoisting every read would
                     * need registers the Q fragments hold */
                    __builtin_amdgcn_sched_barrier(0);
                }

                /* causal mask (only a block that reaches past the wave's first
                 * row needs one); the scores are already in base-2 units */
                const bool full = key0 + kKB - 1 <= pos_first;
                if (!full) {
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int key = key0 + 8 * (v >> 2) + 4 * h + (v & 3);
                        s[v] = key <= qpos ? s[v] : -INFINITY;
                    }
                }
                /* this lane's max over its 16 scores (3-input maxima); the
                 * reference needs the query's max over both lane halves only on
                 * the first block and on a restart */
                float lm;
                {
                    float t6[6];
#pragma unroll
                    for (int v = 0; v < 5; ++v) t6[v] = fmaxf(fmaxf(s[3 * v], s[3 * v + 1]), s[3 * v + 2]);
                    t6[5] = s[15];
                    lm = fmaxf(fmaxf(fmaxf(t6[0], t6[1]), t6[2]), fmaxf(fmaxf(t6[3], t6[4]), t6[5]));
                }
                if (m == -INFINITY) { /* first block: finite (key 0) */
                    const q38_halves bh = q38_both_halves(lm);
                    m = fmaxf(bh.a, bh.b);
                }

                if (!__any(lm > m + kRefSlack)) {
                    bf16x8 ph[2], pl[2];
                    float psum[2] = {0.0f, 0.0f};
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const float p = q38_exp2(s[v] - m);
                        psum[v & 1] += p;
                        /* key 8J + 4h + i -> k-step J/2, element 4(J%2) + i.
                         * hi = p with its low 16 mantissa bits cleared, lo =
                         * bf16(p - hi) (the difference is exact in f32) */
                        const int t = v >> 3, e = v & 7;
                        const uint32_t pb = __float_as_uint(p);
                        ph[t][e] = __builtin_bit_cast(__bf16, (uint16_t)(pb >> 16));
                        pl[t][e] = (__bf16)(p - __uint_as_float(pb & 0xFFFF0000u));
                    }
                    l += psum[0] + psum[1];

                    /* O += P V: B = V^T rows (head dims 32n + col), key slots
                     * 16t + 8h .. +7 */
                    bf16x8 vh[kAhead + 1], vl[kAhead + 1];
                    auto read_v = [&](int st, int r) {
                        const int n = st >> 1, t = st & 1;
                        vh[r] = *reinterpret_cast<const bf16x8 *>(&tiles[buf].vt[0][32 * n + col][16 * t + 8 * h]);
                        vl[r] = *reinterpret_cast<const bf16x8 *>(&tiles[buf].vt[1][32 * n + col][16 * t + 8 * h]);
                    };
#pragma unroll
                    for (int st = 0; st < kAhead; ++st) read_v(st, st);
#pragma unroll
                    for (int st = 0; st < 16; ++st) {
                        if (st + kAhead < 16) read_v(st + kAhead, (st + kAhead) % (kAhead + 1));
                        if (st < kMyPieces - 16) piece(16 + st);
                        const int r = st % (kAhead + 1), n = st >> 1, t = st & 1;
                        O[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ph[t], vh[r], O[n], 0, 0, 0);
                        O[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ph[t], vl[r], O[n], 0, 0, 0);
                        O[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pl[t], vh[r], O[n], 0, 0, 0);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                } else {
                    const q38_halves bh = q38_both_halves(lm);
                    bm = fmaxf(bh.a, bh.b); /* the query's max over the block: the raised reference */
                    for (int i = 16; i < kMyPieces; ++i) piece(i);
                    if (lane == 0) restart_flag[kb & 1] = 1;
                }
            }

            /* the next block's pieces have landed (this wave's), and every wave is
             * done with this block */
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (restart_flag[kb & 1]) {
                /* raise the references to cover this block and start over (a
                 * wave that did not pass its reference keeps bm = -inf) */
                m = fmaxf(m, bm);
                l = 0.0f;
                clear_o();
                __syncthreads(); /* every wave has read the flag */
                if (tid < 2) restart_flag[tid] = 0;
                kb = kb_begin;
                fetch(kb_begin, 0);
                __builtin_amdgcn_s_waitcnt(0);
                __syncthreads();
                continue;
            }
            ++kb;
        }

        /* normalise, gate, store rows 8J+4h+i (their sums live in lanes 8J+4h+i);
         * the last block's barrier has released the tiles for the next job */
        if (!active) continue;
        {
            const q38_halves lh = q38_both_halves(l); /* both halves of the keys */
            l = lh.a + lh.b;
        }
        if (slot >= 0) {
            /* a piece: O as it is, and each row's reference and weight sum
             * (row col's, held by lane col), for q38_prefill_merge */
            const size_t sl = (size_t)j * a.n_slots + slot;
            const int hh = wave & 1;
            const int r0 = kQW * (wave >> 1); /* the wave's first row in the job */
            float *po = a.part_o + (sl * kQ * 2 + hh) * Q38_ATTN_HEAD_DIM;
#pragma unroll
            for (int n = 0; n < 8; ++n) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int r = r0 + 8 * (v >> 2) + 4 * h + (v & 3);
                    po[(size_t)r * 2 * Q38_ATTN_HEAD_DIM + 32 * n + col] = O[n][v];
                }
            }
            if (h == 0) {
                float *pml = a.part_ml + ((sl * kQ + r0 + col) * 2 + hh) * 2;
                pml[0] = m;
                pml[1] = l;
            }
            continue;
        }
        /* The inverse sums of this lane's 16 rows; then, per 32 output dims,
         * the 16 rows' gate factors (loads and sigmoids in one straight
         * block) before their stores.  Every branch here is uniform: out may
         * alias gate as far as the compiler knows, and a load or its use
         * after a store or a branch makes it wait for everything in flight,
         * one memory round trip per output. */
        float inv[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) inv[v] = 1.0f / __shfl(l, 8 * (v >> 2) + 4 * h + (v & 3), 64);
        const bool gated = a.gate != nullptr;
        const bool all_rows = q0 + kQW - 1 <= q_last; /* the wave's 32 rows are all real */
        float *const out0 = a.out + (size_t)head * Q38_ATTN_HEAD_DIM;
        const float *const gate0 = a.gate + (size_t)head * Q38_ATTN_HEAD_DIM;
        constexpr size_t kRow = (size_t)Q38_ATTN_HEADS * Q38_ATTN_HEAD_DIM;
#pragma unroll
        for (int n = 0; n < 8; ++n) {
            const int d = 32 * n + col;
            float gf[16];
            if (gated) {
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    gf[v] = gate0[(size_t)min(q0 + 8 * (v >> 2) + 4 * h + (v & 3), q_last) * kRow + d];
#pragma unroll
                for (int v = 0; v < 16; ++v) gf[v] = q38_sigmoid(gf[v]);
            }
            if (all_rows) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    float res = O[n][v] * inv[v];
                    if (gated) res *= gf[v];
                    out0[(size_t)(q0 + 8 * (v >> 2) + 4 * h + (v & 3)) * kRow + d] = res;
                }
            } else {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int t = q0 + 8 * (v >> 2) + 4 * h + (v & 3);
                    float res = O[n][v] * inv[v];
                    if (gated) res *= gf[v];
                    if (t <= q_last) out0[(size_t)t * kRow + d] = res;
                }
            }
        }
    }
}

/* The pieces of split prefill jobs combined (grid (n_split, 4 kv heads, 32),
 * 256 threads): per (row, head) of a split job, each piece's unnormalised O
 * and weight sum rescaled from its own reference to the largest, summed,
 * then normalised and gated as a whole job's rows are.  Up to 8 pieces' loads
 * are issued at once. */
extern "C" __global__ __launch_bounds__(256) void q38_prefill_merge(q38_prefill_merge_args a) {
    constexpr int kBatch = 8;
    const q38_prefill_split sp = a.split[blockIdx.x];
    const int j = blockIdx.y;
    const int pair = 4 * blockIdx.z + (threadIdx.x >> 6); /* (row, head) of the job */
    const int r = pair >> 1, hh = pair & 1;
    const int t = (sp.code & 63) * kQ + r;
    if (t >= a.n_tokens) return;
    const int d = 4 * (threadIdx.x & 63);
    const int head = j * Q38_ATTN_GROUP + 2 * (sp.code >> 6) + hh;
    const size_t out_off = ((size_t)t * Q38_ATTN_HEADS + head) * Q38_ATTN_HEAD_DIM + d;
    const bool gated = a.gate != nullptr;
    const f32x4 g = gated ? q38_ld4(a.gate + out_off) : f32x4{0.f, 0.f, 0.f, 0.f};
    const size_t slot0 = (size_t)j * a.n_slots + sp.slot0;
    const int n = sp.n;
    float M = -INFINITY, Lsum = 0.0f;
    f32x4 O = {0.f, 0.f, 0.f, 0.f};
    for (int i0 = 0; i0 < n; i0 += kBatch) {
        float m[kBatch], l[kBatch];
        f32x4 o[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const bool in = i0 + k < n;
            const size_t row = ((slot0 + (in ? i0 + k : i0)) * kQ + r) * 2 + hh; /* a piece known to exist */
            m[k] = in ? a.part_ml[row * 2] : -INFINITY;
            l[k] = a.part_ml[row * 2 + 1];
            o[k] = q38_ld4(a.part_o + row * Q38_ATTN_HEAD_DIM + d);
        }
        float mx = M;
#pragma unroll
        for (int k = 0; k < kBatch; ++k) mx = fmaxf(mx, m[k]);
        const float f = q38_exp2(M - mx); /* 0 while M is -inf */
        Lsum *= f;
        O *= f;
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const float w = q38_exp2(m[k] - mx); /* 0 for absent pieces */
            Lsum = __builtin_fmaf(w, l[k], Lsum);
            O = q38_fma4(w, o[k], O);
        }
        M = mx;
    }
    const float inv = 1.0f / Lsum;
    f32x4 res = O * inv;
    if (gated) {
        res.x *= q38_sigmoid(g.x);
        res.y *= q38_sigmoid(g.y);
        res.z *= q38_sigmoid(g.z);
        res.w *= q38_sigmoid(g.w);
    }
    q38_st4(a.out + out_off, res);
}
