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
 *  - grid (query block, kv head j); 6 waves, wave w = query head 6j+w; a
 *    workgroup serves 16 query tokens (one 16-token tile per wave) of all 6
 *    heads from one copy of each K/V block, so K and V are read once per
 *    group and block, not once per head;
 *  - scores are computed transposed, S^T = K Q^T (A = K rows from LDS, B =
 *    Q^T from registers), so lane (g = l/16, c = l%16) holds query c's
 *    scores for keys 16kt + 4g + i -- exactly the P values it supplies as
 *    the A operand of O += P V when the key order inside the 32-key block
 *    is permuted to slot 8g + 4kt + i; V is stored transposed in LDS in that
 *    slot order, so P never leaves registers;
 *  - K/V blocks of 32 keys go f32 (HBM) -> registers (prefetched one block
 *    ahead) -> bf16 hi/lo in LDS (double-buffered), one barrier per block;
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

constexpr int kQ = 16;           /* query tokens per workgroup */
constexpr int kQT = kQ / 16;     /* 16-token query tiles per wave */
constexpr int kKB = 32;          /* keys per block */
constexpr int kKRow = 256 + 8;   /* bf16 per K row in LDS: 16 B pad, conflict-free b128 reads */
constexpr int kVRow = kKB + 8;   /* bf16 per transposed V row (one head dim) */
constexpr int kThreads = 64 * Q38_ATTN_GROUP;
constexpr int kKItems = kKB * Q38_ATTN_HEAD_DIM / 4;         /* float4 of a K block: 2048 */
constexpr int kVItems = kKB / 2 * Q38_ATTN_HEAD_DIM / 4;     /* (key pair, dim quad): 1024 */
constexpr int kKPer = (kKItems + kThreads - 1) / kThreads;   /* 6 */
constexpr int kVPer = (kVItems + kThreads - 1) / kThreads;   /* 3 */

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

struct Prefetch {
    f32x4 k[kKPer];
    f32x4 v0[kVPer], v1[kVPer];
};

/* Element offset of key position kp (clamped to the last needed one) in
 * kv head j's pages. */
Q38_DEV size_t key_row(const q38_prefill_args &a, int j, int kp, int kmax) {
    kp = min(kp, kmax);
    const int phys = a.page_table[kp >> 4];
    return ((size_t)phys * Q38_ATTN_KV_HEADS + j) * Q38_PAGE_TOKENS * Q38_ATTN_HEAD_DIM +
           (size_t)(kp & 15) * Q38_ATTN_HEAD_DIM;
}

Q38_DEV void prefetch_block(Prefetch &pf, const q38_prefill_args &a, int j, int kb, int kmax, int tid) {
#pragma unroll
    for (int t = 0; t < kKPer; ++t) {
        const int i = tid + t * kThreads;
        if (i < kKItems) {
            const int r = i >> 6, c4 = i & 63;
            pf.k[t] = q38_ld4(a.kpool + key_row(a, j, kb * kKB + r, kmax) + 4 * c4);
        }
    }
#pragma unroll
    for (int t = 0; t < kVPer; ++t) {
        const int i = tid + t * kThreads;
        if (i < kVItems) {
            const int r = 2 * (i >> 6), c4 = i & 63;
            pf.v0[t] = q38_ld4(a.vpool + key_row(a, j, kb * kKB + r, kmax) + 4 * c4);
            pf.v1[t] = q38_ld4(a.vpool + key_row(a, j, kb * kKB + r + 1, kmax) + 4 * c4);
        }
    }
}

Q38_DEV void store_block(const Prefetch &pf, __bf16 (*k_hi)[kKRow], __bf16 (*k_lo)[kKRow],
                         __bf16 (*vt_hi)[kVRow], __bf16 (*vt_lo)[kVRow], int tid) {
#pragma unroll
    for (int t = 0; t < kKPer; ++t) {
        const int i = tid + t * kThreads;
        if (i < kKItems) {
            const int r = i >> 6, c4 = i & 63;
            const Split4 s = split4(pf.k[t]);
            *reinterpret_cast<bf16x4 *>(&k_hi[r][4 * c4]) = s.hi;
            *reinterpret_cast<bf16x4 *>(&k_lo[r][4 * c4]) = s.lo;
        }
    }
#pragma unroll
    for (int t = 0; t < kVPer; ++t) {
        const int i = tid + t * kThreads;
        if (i < kVItems) {
            const int r = 2 * (i >> 6), c4 = i & 63;
            const int slot = key_slot(r); /* key r+1 sits at slot + 1 */
            const Split4 s0 = split4(pf.v0[t]);
            const Split4 s1 = split4(pf.v1[t]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int d = 4 * c4 + e;
                *reinterpret_cast<bf16x2 *>(&vt_hi[d][slot]) = bf16x2{s0.hi[e], s1.hi[e]};
                *reinterpret_cast<bf16x2 *>(&vt_lo[d][slot]) = bf16x2{s0.lo[e], s1.lo[e]};
            }
        }
    }
}

}  // namespace

extern "C" __global__ __launch_bounds__(kThreads, 1) void q38_attn_prefill_mfma(q38_prefill_args a) {
    __shared__ __attribute__((aligned(16))) __bf16 k_lds[2][2][kKB][kKRow];
    __shared__ __attribute__((aligned(16))) __bf16 vt_lds[2][2][Q38_ATTN_HEAD_DIM][kVRow];

    const int qb = a.n_qblocks - 1 - (int)blockIdx.x; /* longest causal rows first */
    const int j = blockIdx.y;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = j * Q38_ATTN_GROUP + wave;
    const int g = lane >> 4;
    const int c = lane & 15;
    const int qt0 = qb * kQ;                            /* first query token of the block */
    const int q_last = min(qt0 + kQ, a.n_tokens) - 1;   /* last real query token */
    const int kmax = a.base_pos + q_last;               /* last key position any row needs */
    const int n_kb = kmax / kKB + 1;

    /* Q^T operand: lane (g, c) of tile qt holds query qt0 + 16qt + c, dims
     * 32kk + 8g .. +7, as bf16 hi and lo */
    bf16x8 q_hi[kQT][8], q_lo[kQT][8];
    int qpos[kQT];
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
        const int tq = min(qt0 + 16 * qt + c, q_last);
        qpos[qt] = a.base_pos + qt0 + 16 * qt + c;
        const float *qp = a.q + ((size_t)tq * Q38_ATTN_HEADS + h) * Q38_ATTN_HEAD_DIM + 8 * g;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            const Split4 s0 = split4(q38_ld4(qp + 32 * kk));
            const Split4 s1 = split4(q38_ld4(qp + 32 * kk + 4));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                q_hi[qt][kk][e] = s0.hi[e];
                q_hi[qt][kk][4 + e] = s1.hi[e];
                q_lo[qt][kk][e] = s0.lo[e];
                q_lo[qt][kk][4 + e] = s1.lo[e];
            }
        }
    }

    float m[kQT], l[kQT];
    f32x4 O[kQT][16];
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
        m[qt] = -INFINITY;
        l[qt] = 0.0f;
#pragma unroll
        for (int n = 0; n < 16; ++n) O[qt][n] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    Prefetch pf;
    prefetch_block(pf, a, j, 0, kmax, tid);
    store_block(pf, k_lds[0][0], k_lds[0][1], vt_lds[0][0], vt_lds[0][1], tid);
    __syncthreads();

    for (int kb = 0; kb < n_kb; ++kb) {
        const int buf = kb & 1;
        const bool more = kb + 1 < n_kb;
        if (more) prefetch_block(pf, a, j, kb + 1, kmax, tid);

        /* S^T tiles: s[qt][kt][i] = score of query (qt, c) and key 16kt + 4g + i */
        f32x4 s[kQT][2];
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) s[qt][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                const bf16x8 kh = *reinterpret_cast<const bf16x8 *>(&k_lds[buf][0][16 * kt + c][32 * kk + 8 * g]);
                const bf16x8 kl = *reinterpret_cast<const bf16x8 *>(&k_lds[buf][1][16 * kt + c][32 * kk + 8 * g]);
#pragma unroll
                for (int qt = 0; qt < kQT; ++qt) {
                    s[qt][kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, q_hi[qt][kk], s[qt][kt], 0, 0, 0);
                    s[qt][kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, q_lo[qt][kk], s[qt][kt], 0, 0, 0);
                    s[qt][kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl, q_hi[qt][kk], s[qt][kt], 0, 0, 0);
                }
            }
        }

        bf16x8 p_hi[kQT], p_lo[kQT];
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
            /* scale, causal mask, block max of the row */
            float bm = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int key = kb * kKB + 16 * kt + 4 * g + i;
                    const float x = key <= qpos[qt] ? s[qt][kt][i] * Q38_SCORE_LOG2 : -INFINITY;
                    s[qt][kt][i] = x;
                    bm = fmaxf(bm, x);
                }
            bm = max_over_groups(bm);
            const float m_new = fmaxf(m[qt], bm); /* finite: key 0 is in every row's block 0 */
            const float f = q38_exp2(m[qt] - m_new); /* 0 while m is -inf */
            float ps = 0.0f;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float p = q38_exp2(s[qt][kt][i] - m_new);
                    ps += p;
                    const __bf16 ph = (__bf16)p;
                    p_hi[qt][4 * kt + i] = ph;
                    p_lo[qt][4 * kt + i] = (__bf16)(p - (float)ph);
                }
            l[qt] = l[qt] * f + sum_over_groups(ps);
            m[qt] = m_new;
            /* rescale O: lane (g, c) holds rows 4g+i, whose factor lives in lane 4g+i */
            if (__builtin_amdgcn_read_exec() != 0 && __any(f != 1.0f)) {
                float fr[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) fr[i] = __shfl(f, 4 * g + i, 64);
#pragma unroll
                for (int n = 0; n < 16; ++n)
#pragma unroll
                    for (int i = 0; i < 4; ++i) O[qt][n][i] *= fr[i];
            }
        }

        /* O += P V: B = V^T rows (head dims 16n + c), key slots 8g .. 8g+7 */
#pragma unroll
        for (int n = 0; n < 16; ++n) {
            const bf16x8 vh = *reinterpret_cast<const bf16x8 *>(&vt_lds[buf][0][16 * n + c][8 * g]);
            const bf16x8 vl = *reinterpret_cast<const bf16x8 *>(&vt_lds[buf][1][16 * n + c][8 * g]);
#pragma unroll
            for (int qt = 0; qt < kQT; ++qt) {
                O[qt][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(p_hi[qt], vh, O[qt][n], 0, 0, 0);
                O[qt][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(p_hi[qt], vl, O[qt][n], 0, 0, 0);
                O[qt][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(p_lo[qt], vh, O[qt][n], 0, 0, 0);
            }
        }

        if (more) store_block(pf, k_lds[buf ^ 1][0], k_lds[buf ^ 1][1], vt_lds[buf ^ 1][0], vt_lds[buf ^ 1][1], tid);
        __syncthreads();
    }

    /* normalise, gate, store rows 4g+i of each tile */
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
        float inv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) inv[i] = 1.0f / __shfl(l[qt], 4 * g + i, 64);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = qt0 + 16 * qt + 4 * g + i;
            if (t > q_last) continue;
            const size_t row = ((size_t)t * Q38_ATTN_HEADS + h) * Q38_ATTN_HEAD_DIM;
#pragma unroll
            for (int n = 0; n < 16; ++n) {
                const int d = 16 * n + c;
                float r = O[qt][n][i] * inv[i];
                if (a.gate != nullptr) r *= q38_sigmoid(a.gate[row + d]);
                a.out[row + d] = r;
            }
        }
    }
}
