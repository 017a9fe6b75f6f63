/*
 * Full-attention GQA decode over the paged KV cache (gfx950, wave64).
 *
 * Reference semantics: full_core, src/model/ops.rs:813-940 -- for every query
 * head h (kv head j = h/6): scores q.k_p * 1/16 over positions 0..pos,
 * softmax, probability-weighted sum of value rows, times sigmoid(gate).
 *
 * Design:
 *  - grid (split, kv head): one workgroup streams one kv head's K and V rows
 *    of one context split ONCE and serves all 6 query heads of the group from
 *    registers (the reference re-reads each row once per query head);
 *  - a half-wave (32 lanes) owns one token row: lane i holds dims 4i..4i+3 and
 *    128+4i..128+4i+3, loaded as 128-bit vectors, so one row is two fully
 *    coalesced 512-byte segments; the 256-long dot is 8 FMAs per lane plus a
 *    DPP row reduction and one v_permlane16_swap;
 *  - online softmax in base 2 (q is pre-scaled by log2(e)/16) with the running
 *    max/sum per head; the split's 8 half-waves merge through LDS;
 *  - a single split finishes the heads itself (output gate included);
 *    several splits leave unnormalised partials for q38_attn_decode_merge.
 */
#include "q38_device.h"

/* 1/sqrt(256) (ops.rs:869) times log2(e). */
#define Q38_SCORE_LOG2 0.09016844005556021f

namespace {

struct DecodeState {
    float m[Q38_ATTN_GROUP];
    float l[Q38_ATTN_GROUP];
    f32x4 o0[Q38_ATTN_GROUP];
    f32x4 o1[Q38_ATTN_GROUP];
};

/* Where one half-wave reads its 4 rows of the half-page that holds the
 * sequence's last position: the page rows, the new token's row for position
 * `pos`, or -- past the end -- a row known to hold finite data (weight 0). */
struct TailRows {
    const float *k[4];
    const float *v[4];
    bool valid[4];
};

struct Rows {
    f32x4 x0[4], x1[4];
};

/* Full half-page at element offset `base` of the pools: rows 2s+grp. */
Q38_DEV void load_rows(Rows &r, const float *pool, size_t base, int lane_off) {
    const float *p = pool + base + lane_off;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        r.x0[s] = q38_ld4_stream(p + 2 * s * Q38_ATTN_HEAD_DIM);
        r.x1[s] = q38_ld4_stream(p + 2 * s * Q38_ATTN_HEAD_DIM + 128);
    }
}

/* pages: the split's physical page ids in LDS (entry i holds the page of
 * tokens t_begin + 16i ..); tb is relative to t_begin. */
Q38_DEV size_t half_page_base(const int32_t *pages, int j, int tb) {
    const int phys = pages[tb >> 4];
    return ((size_t)phys * Q38_ATTN_KV_HEADS + j) * Q38_PAGE_TOKENS * Q38_ATTN_HEAD_DIM +
           (size_t)(tb & 15) * Q38_ATTN_HEAD_DIM;
}

/* Scores of 4 rows for the 6 heads, online-softmax update, weighted V sum. */
Q38_DEV void decode_rows(DecodeState &st, const f32x4 (&q0)[Q38_ATTN_GROUP],
                         const f32x4 (&q1)[Q38_ATTN_GROUP], const Rows &K, const Rows &V,
                         const bool (&valid)[4]) {
    float sc[4][Q38_ATTN_GROUP];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
        for (int hh = 0; hh < Q38_ATTN_GROUP; ++hh) {
            float x = q38_dot4(q0[hh], K.x0[s], 0.0f);
            x = q38_dot4(q1[hh], K.x1[s], x);
            sc[s][hh] = valid[s] ? q38_sum32(x) : -INFINITY;
        }
    }
#pragma unroll
    for (int hh = 0; hh < Q38_ATTN_GROUP; ++hh) {
        const float mx = fmaxf(fmaxf(sc[0][hh], sc[1][hh]), fmaxf(sc[2][hh], sc[3][hh]));
        if (mx > st.m[hh]) {
            const float f = q38_exp2(st.m[hh] - mx); /* 0 while m is -inf */
            st.l[hh] *= f;
            st.o0[hh] *= f;
            st.o1[hh] *= f;
            st.m[hh] = mx;
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const float p = valid[s] ? q38_exp2(sc[s][hh] - st.m[hh]) : 0.0f;
            st.l[hh] += p;
            st.o0[hh] = q38_fma4(p, V.x0[s], st.o0[hh]);
            st.o1[hh] = q38_fma4(p, V.x1[s], st.o1[hh]);
        }
    }
}

/* RoPE angles of one position, once: pair p gets theta_p = position *
 * scale^p by p repeated f32 multiplications (the reference's rounding), and
 * cs[p] = (cos, sin) of it; lane p < 32 of the calling wave forms pair p. */
Q38_DEV void q38_rope_table(float (*cs)[2], int lane, int position, float theta_scale) {
    if (lane < 32) {
        float theta = (float)position;
        for (int i = 0; i < lane; ++i) theta *= theta_scale;
        cs[lane][0] = cosf(theta);
        cs[lane][1] = sinf(theta);
    }
}

/* RoPE on dims 0..63 (ops.rs:595-610: pairs (p, p+32), theta_0 = position,
 * theta_{p+1} = theta_p * 1e7^(-2/64) by repeated f32 multiplication) of one
 * 256-dim head held 4 dims per lane by a whole wave (lane l: dims 4l ..
 * 4l+3), with the angles' cosines and sines from a q38_rope_table */
Q38_DEV void q38_rope_lanes_cs(f32x4 &x, int l, const float (*cs)[2]) {
    f32x4 partner;
#pragma unroll
    for (int c = 0; c < 4; ++c) partner[c] = __shfl_xor(x[c], 8, 64);
    if (l < 16) {
        const int p0 = 4 * (l & 7);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float cosine = cs[p0 + c][0];
            const float sine = cs[p0 + c][1];
            if (l < 8) {
                const float x0 = x[c], x1 = partner[c];
                x[c] = x0 * cosine - x1 * sine;
            } else {
                const float x0 = partner[c], x1 = x[c];
                x[c] = x0 * sine + x1 * cosine;
            }
        }
    }
}

/* RMS scale of a 256-dim head from its f64 sum of squares */
Q38_DEV float q38_rms_scale_of(double ss) {
    const float mean = (float)(ss / (double)Q38_ATTN_HEAD_DIM);
    return 1.0f / sqrtf(mean + 1e-6f);
}

/* The same for a head held by a half-wave, lane li: dims 4li .. 4li+3 (x0)
 * and 128 + 4li .. (x1); the angles from a q38_rope_table. */
Q38_DEV void q38_norm_rope8(f32x4 &x0, f32x4 &x1, f32x4 w0, f32x4 w1, int li, const float (*cs)[2]) {
    double ss = 0.0;
#pragma unroll
    for (int c = 0; c < 4; ++c) ss += (double)x0[c] * (double)x0[c] + (double)x1[c] * (double)x1[c];
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
    const float scale = q38_rms_scale_of(ss);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        x0[c] = x0[c] * scale * w0[c];
        x1[c] = x1[c] * scale * w1[c];
    }
    q38_rope_lanes_cs(x0, li, cs);
}

/* RMSNorm with weight w (rms_scale / rmsnorm_inplace, ops.rs:476-498: f64 sum
 * of squares, eps 1e-6), then the RoPE of q38_rope_lanes_cs, of a head held 4
 * dims per lane by a whole wave.  Every f32 square is exact in f64, so the f64
 * sum rounds to the same f32 mean in any order. */
Q38_DEV void q38_norm_rope4_cs(f32x4 &x, f32x4 w, int lane, const float (*cs)[2]) {
    double ss = (double)x.x * (double)x.x + (double)x.y * (double)x.y + (double)x.z * (double)x.z +
                (double)x.w * (double)x.w;
    const float scale = q38_rms_scale_of(q38_wave_sum_f64(ss));
#pragma unroll
    for (int c = 0; c < 4; ++c) x[c] = x[c] * scale * w[c];
    q38_rope_lanes_cs(x, lane, cs);
}

}  // namespace

#ifndef Q38_DECODE_MIN_WGS
#define Q38_DECODE_MIN_WGS 1 /* workgroups per CU the register budget is sized for */
#endif

/* kOneSeq: a launch of one sequence (n_seq == 1, split g of that sequence),
 * so every argument a workgroup needs sits at a fixed offset and is loaded
 * in one round, before the first row loads. */
template <bool kPre, bool kArgPages, bool kOneSeq = false>
Q38_DEV void decode_split(const q38_decode_args &a) {
    constexpr int NW = Q38_DECODE_WAVES;
    __shared__ float red_o[NW][Q38_ATTN_GROUP][Q38_ATTN_HEAD_DIM];
    __shared__ float red_m[NW][Q38_ATTN_GROUP];
    __shared__ float red_l[NW][Q38_ATTN_GROUP];
    __shared__ int32_t pages[Q38_MAX_SPLIT_TOKENS / Q38_PAGE_TOKENS];

    const int g = blockIdx.x;
    const int j = blockIdx.y;
    int b = 0;
    if (!kOneSeq)
        while (b + 1 < a.n_seq && a.split_base[b + 1] <= g) ++b;
    const int seq = kOneSeq ? a.seq[0] : a.seq[b];
    const int pos = kOneSeq ? a.pos[0] : a.pos[b];
    const int split = kOneSeq ? g : g - a.split_base[b];
    const int nsplit = kOneSeq ? a.total_splits : a.split_base[b + 1] - a.split_base[b];
    const int t_begin = split * a.split_tokens;
    const int t_end = min(pos + 1, t_begin + a.split_tokens);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = lane >> 5;
    const int li = lane & 31;
    const int d0 = 4 * li;
    const int d1 = 128 + 4 * li;

    const int n_tok = t_end - t_begin;
    const int n_hp = (n_tok + 7) / 8;
    /* every half-page is full except, in the split that holds `pos` (always
     * the sequence's last position), the last one: that one is handled after
     * the loop with per-row redirection */
    const bool has_tail = t_end == pos + 1;
    const int n_regular = has_tail ? n_hp - 1 : n_hp;
    const int lane_off = grp * Q38_ATTN_HEAD_DIM + d0;

    /* the split's page ids, loaded once: the streaming loop below then has
     * no global load whose address depends on another global load */
    const int32_t *pt = a.page_table + (size_t)seq * a.pt_stride;
    const int n_split_pages = (t_end - t_begin + Q38_PAGE_TOKENS - 1) / Q38_PAGE_TOKENS;
    Rows K, V;
    f32x4 q0[Q38_ATTN_GROUP], q1[Q38_ATTN_GROUP];
    /* the group's 6 query rows; with the pre step fused, raw q|gate rows
     * (each head's q followed by its gate) */
    const int q_stride = kPre ? 2 * Q38_ATTN_HEAD_DIM : Q38_ATTN_HEAD_DIM;
    const float *qb = a.q + ((size_t)b * Q38_ATTN_HEADS + j * Q38_ATTN_GROUP) * q_stride;
    if (kArgPages) {
        /* software pipeline start: wave w's half-page w lies in the split's
         * page 0 or 1, whose ids come with the launch, so these loads issue at
         * once.  A wave with no regular half-page loads page 0's rows (in the
         * pool, unused) so that no load sits under a branch.  The page-id load
         * is issued first and every thread stores its result (slots past the
         * split's pages are never read), so that store waits for it alone. */
        const int32_t my_page = pt[(t_begin >> 4) + min(tid, n_split_pages - 1)];
        __builtin_amdgcn_sched_barrier(0);
        const int hp0 = wave < n_regular ? wave : 0;
        const size_t base = ((size_t)a.head_pages[g][hp0 >> 1] * Q38_ATTN_KV_HEADS + j) * Q38_PAGE_TOKENS *
                                Q38_ATTN_HEAD_DIM + (size_t)(hp0 & 1) * 8 * Q38_ATTN_HEAD_DIM;
        load_rows(K, a.kpool, base, lane_off);
        load_rows(V, a.vpool, base, lane_off);
#pragma unroll
        for (int hh = 0; hh < Q38_ATTN_GROUP; ++hh) {
            q0[hh] = q38_ld4(qb + hh * q_stride + d0);
            q1[hh] = q38_ld4(qb + hh * q_stride + d1);
        }
        pages[tid] = my_page;
    } else {
#pragma unroll
        for (int hh = 0; hh < Q38_ATTN_GROUP; ++hh) {
            q0[hh] = q38_ld4(qb + hh * q_stride + d0);
            q1[hh] = q38_ld4(qb + hh * q_stride + d1);
        }
        if (tid < n_split_pages) pages[tid] = pt[(t_begin >> 4) + tid];
    }
    /* with the pre step fused, the split holding `pos` forms the new key row
     * (RMSNorm and RoPE of the raw key, ops.rs:844-856) in LDS; it is
     * appended below and scored from there */
    __shared__ __attribute__((aligned(16))) float k_formed[Q38_ATTN_HEAD_DIM];
    __shared__ float rope_cs[32][2];
    const bool holds_pos = pos >= t_begin && pos < t_end;
    if (kPre) {
        if (wave == NW - 1) q38_rope_table(rope_cs, lane, pos, a.theta_scale);
        __syncthreads();
        if (a.k_new != nullptr && holds_pos && wave == 0) {
            f32x4 x = q38_ld4(a.k_new + (size_t)b * Q38_ATTN_KV_DIM + j * Q38_ATTN_HEAD_DIM + 4 * lane);
            q38_norm_rope4_cs(x, q38_ld4(a.k_norm + 4 * lane), lane, rope_cs);
            q38_st4(&k_formed[4 * lane], x);
        }
    }
    __syncthreads();
    const float *k_new_row = nullptr;
    const float *v_new_row = nullptr;
    if (a.k_new != nullptr) {
        k_new_row = kPre ? k_formed : a.k_new + (size_t)b * Q38_ATTN_KV_DIM + j * Q38_ATTN_HEAD_DIM;
        v_new_row = a.v_new + (size_t)b * Q38_ATTN_KV_DIM + j * Q38_ATTN_HEAD_DIM;
        /* KV append (ops.rs:858-866): the split that holds `pos` stores the row. */
        if (pos >= t_begin && pos < t_end && wave == 0) {
            const int phys = pages[(pos - t_begin) >> 4];
            const size_t row = ((size_t)phys * Q38_ATTN_KV_HEADS + j) * Q38_PAGE_TOKENS * Q38_ATTN_HEAD_DIM +
                               (size_t)(pos & 15) * Q38_ATTN_HEAD_DIM;
            q38_st4(a.kpool + row + 4 * lane, q38_ld4(k_new_row + 4 * lane));
            q38_st4(a.vpool + row + 4 * lane, q38_ld4(v_new_row + 4 * lane));
        }
    }

    const bool all_valid[4] = {true, true, true, true};

    /* software pipeline: the K rows of the next half-page are in flight
     * while the current one is scored, and its V rows while the current one
     * is accumulated */
    if (!kArgPages && wave < n_regular) {
        const size_t base = half_page_base(pages, j, wave * 8);
        load_rows(K, a.kpool, base, lane_off);
        load_rows(V, a.vpool, base, lane_off);
    }

    if (kPre) {
        /* the group's query heads RMSNormed and rotated here (ops.rs:832-856;
         * the same arithmetic as q38_attn_pre), each half-wave holding a whole
         * head */
        const f32x4 w0 = q38_ld4(a.q_norm + d0), w1 = q38_ld4(a.q_norm + d1);
#pragma unroll
        for (int hh = 0; hh < Q38_ATTN_GROUP; ++hh) {
            q38_norm_rope8(q0[hh], q1[hh], w0, w1, li, rope_cs);
            q0[hh] *= Q38_SCORE_LOG2;
            q1[hh] *= Q38_SCORE_LOG2;
        }
    } else {
#pragma unroll
        for (int hh = 0; hh < Q38_ATTN_GROUP; ++hh) {
            q0[hh] *= Q38_SCORE_LOG2;
            q1[hh] *= Q38_SCORE_LOG2;
        }
    }

    DecodeState st;
#pragma unroll
    for (int hh = 0; hh < Q38_ATTN_GROUP; ++hh) {
        st.m[hh] = -INFINITY;
        st.l[hh] = 0.0f;
        st.o0[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
        st.o1[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    for (int hp = wave; hp < n_regular; hp += NW) {
        const bool has_next = hp + NW < n_regular;
        size_t nbase = 0;
        Rows Kn;
        if (has_next) {
            nbase = half_page_base(pages, j, (hp + NW) * 8);
            load_rows(Kn, a.kpool, nbase, lane_off);
        }
        decode_rows(st, q0, q1, K, V, all_valid);
        if (has_next) {
            load_rows(V, a.vpool, nbase, lane_off);
            K = Kn;
        }
    }

    if (has_tail && wave == (n_hp - 1) % NW) {
        const int tb = t_begin + (n_hp - 1) * 8;
        const size_t base = half_page_base(pages, j, tb - t_begin);
        TailRows tr;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int r = 2 * s + grp;
            const int t = tb + r;
            tr.valid[s] = t < t_end;
            tr.k[s] = a.kpool + base + r * Q38_ATTN_HEAD_DIM;
            tr.v[s] = a.vpool + base + r * Q38_ATTN_HEAD_DIM;
            if (k_new_row != nullptr && (t == pos || !tr.valid[s])) {
                tr.k[s] = k_new_row;
                tr.v[s] = v_new_row;
            } else if (!tr.valid[s]) {
                tr.k[s] = a.kpool + base;
                tr.v[s] = a.vpool + base;
            }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            K.x0[s] = q38_ld4_stream(tr.k[s] + d0);
            K.x1[s] = q38_ld4_stream(tr.k[s] + d1);
            V.x0[s] = q38_ld4_stream(tr.v[s] + d0);
            V.x1[s] = q38_ld4_stream(tr.v[s] + d1);
        }
        decode_rows(st, q0, q1, K, V, tr.valid);
    }

    /* merge the wave's two half-waves (lane i with lane i^32, same dims) */
#pragma unroll
    for (int hh = 0; hh < Q38_ATTN_GROUP; ++hh) {
        const q38_halves mh = q38_both_halves(st.m[hh]);
        const float M = fmaxf(mh.a, mh.b);
        const float fa = mh.a == -INFINITY ? 0.0f : q38_exp2(mh.a - M);
        const float fb = mh.b == -INFINITY ? 0.0f : q38_exp2(mh.b - M);
        const q38_halves lh = q38_both_halves(st.l[hh]);
        const float L = lh.a * fa + lh.b * fb;
        f32x4 o0, o1;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const q38_halves x0 = q38_both_halves(st.o0[hh][c]);
            const q38_halves x1 = q38_both_halves(st.o1[hh][c]);
            o0[c] = x0.a * fa + x0.b * fb;
            o1[c] = x1.a * fa + x1.b * fb;
        }
        if (grp == 0) {
            q38_st4(&red_o[wave][hh][d0], o0);
            q38_st4(&red_o[wave][hh][d1], o1);
        }
        if (lane == 0) {
            red_m[wave][hh] = M;
            red_l[wave][hh] = L;
        }
    }
    __syncthreads();

    if (tid >= Q38_ATTN_HEAD_DIM) return;
    const int d = tid; /* one output dim per thread */
#pragma unroll
    for (int hh = 0; hh < Q38_ATTN_GROUP; ++hh) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, red_m[w][hh]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float mw = red_m[w][hh];
            const float f = mw == -INFINITY ? 0.0f : q38_exp2(mw - M);
            L += red_l[w][hh] * f;
            O += red_o[w][hh][d] * f;
        }
        const int h = j * Q38_ATTN_GROUP + hh;
        if (nsplit == 1) {
            float r = O / L;
            if (a.gate != nullptr)
                r *= q38_sigmoid(a.gate[((size_t)b * Q38_ATTN_HEADS + h) * a.gate_head_stride + d]);
            a.out[(size_t)b * Q38_ATTN_Q_DIM + h * Q38_ATTN_HEAD_DIM + d] = r;
        } else {
            a.part_o[((size_t)g * Q38_ATTN_HEADS + h) * Q38_ATTN_HEAD_DIM + d] = O;
            if (d == 0) {
                a.part_ml[((size_t)g * Q38_ATTN_HEADS + h) * 2 + 0] = M;
                a.part_ml[((size_t)g * Q38_ATTN_HEADS + h) * 2 + 1] = L;
            }
        }
    }
}

/* Launches of at most Q38_HEAD_PAGE_SPLITS splits: the first two page ids of
 * every split come in a.head_pages. */
extern "C" __global__ __launch_bounds__(64 * Q38_DECODE_WAVES, Q38_DECODE_MIN_WGS) void q38_attn_decode_split(
    q38_decode_args a) {
    decode_split<false, true>(a);
}

/* One sequence of at most Q38_HEAD_PAGE_SPLITS splits (batch-1 decode). */
extern "C" __global__ __launch_bounds__(64 * Q38_DECODE_WAVES, Q38_DECODE_MIN_WGS) void q38_attn_decode_split_one(
    q38_decode_args a) {
    decode_split<false, true, true>(a);
}

/* Any number of splits: every page id read from the page table. */
extern "C" __global__ __launch_bounds__(64 * Q38_DECODE_WAVES, Q38_DECODE_MIN_WGS) void q38_attn_decode_split_many(
    q38_decode_args a) {
    decode_split<false, false>(a);
}

/* The same two with the pre step of full_core fused: q from the raw q|gate
 * rows and the appended key from the raw key, both RMSNormed and rotated in
 * the kernel; the gate read from q|gate. */
extern "C" __global__ __launch_bounds__(64 * Q38_DECODE_WAVES, Q38_DECODE_MIN_WGS) void q38_attn_decode_split_pre(
    q38_decode_args a) {
    decode_split<true, true>(a);
}

extern "C" __global__ __launch_bounds__(64 * Q38_DECODE_WAVES, Q38_DECODE_MIN_WGS) void q38_attn_decode_split_pre_one(
    q38_decode_args a) {
    decode_split<true, true, true>(a);
}

extern "C" __global__ __launch_bounds__(64 * Q38_DECODE_WAVES, Q38_DECODE_MIN_WGS) void q38_attn_decode_split_pre_many(
    q38_decode_args a) {
    decode_split<true, false>(a);
}

/* Combine the splits of each (sequence, head): rescale every partial to the
 * common max, sum, normalise, gate.  grid (n_seq, 24, 4): z picks 64 of the
 * 256 dims, so 96 workgroups share a sequence's merge.  Thread (sl, dl)
 * merges splits sl, sl + 16, ... of dims 4dl..4dl+3 online (running max,
 * sum and output in registers); up to 8 splits' (m, l, o) are loaded at
 * once, so a merge of up to 128 splits costs one memory round trip.  The 16
 * per-thread results of each dim quad then meet in LDS. */
extern "C" __global__ __launch_bounds__(256) void q38_attn_decode_merge(q38_merge_args a) {
    constexpr int kBatch = 8;
    __shared__ f32x4 red_o[16][16];
    __shared__ float red_m[16][16];
    __shared__ float red_l[16][16];
    const int b = blockIdx.x;
    const int h = blockIdx.y;
    const int dq = blockIdx.z;
    const int base = a.split_base[b];
    const int n = a.split_base[b + 1] - base;
    if (n <= 1) return;
    const int tid = threadIdx.x;
    const int dl = tid & 15;
    const int sl = tid >> 4;
    const int d = dq * 64 + 4 * dl;
    const size_t o_step = (size_t)Q38_ATTN_HEADS * Q38_ATTN_HEAD_DIM;
    const float *po = a.part_o + ((size_t)base * Q38_ATTN_HEADS + h) * Q38_ATTN_HEAD_DIM + d;
    const float *pml = a.part_ml + ((size_t)base * Q38_ATTN_HEADS + h) * 2;
    /* the gate of the 4 output dims this thread may store, loaded with the
     * partials rather than after them */
    const size_t off = (size_t)b * Q38_ATTN_Q_DIM + h * Q38_ATTN_HEAD_DIM + d;
    const bool gated = a.gate != nullptr;
    const f32x4 gt = gated && sl == 0 ? q38_ld4(a.gate + ((size_t)b * Q38_ATTN_HEADS + h) * a.gate_head_stride + d)
                                      : f32x4{0.f, 0.f, 0.f, 0.f};

    float M = -INFINITY, L = 0.0f;
    f32x4 O = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = sl; s0 < n; s0 += 16 * kBatch) {
        float m[kBatch], l[kBatch];
        f32x4 o[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const int s = s0 + 16 * k;
            const bool in = s < n;
            const int sc = in ? s : s0; /* a split known to exist */
            m[k] = in ? pml[(size_t)sc * Q38_ATTN_HEADS * 2] : -INFINITY;
            l[k] = pml[(size_t)sc * Q38_ATTN_HEADS * 2 + 1];
            o[k] = q38_ld4(po + (size_t)sc * o_step);
        }
        float mx = M;
#pragma unroll
        for (int k = 0; k < kBatch; ++k) mx = fmaxf(mx, m[k]);
        if (mx != -INFINITY) {
            const float f = q38_exp2(M - mx); /* 0 while M is -inf */
            L *= f;
            O *= f;
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const float w = q38_exp2(m[k] - mx); /* 0 for absent or empty splits */
                L = __builtin_fmaf(w, l[k], L);
                O = q38_fma4(w, o[k], O);
            }
            M = mx;
        }
    }
    red_o[sl][dl] = O;
    red_m[sl][dl] = M;
    red_l[sl][dl] = L;
    __syncthreads();
    if (sl == 0) {
        float Mt = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) Mt = fmaxf(Mt, red_m[i][dl]);
        float Lt = 0.0f;
        f32x4 Ot = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float mi = red_m[i][dl];
            const float w = mi == -INFINITY ? 0.0f : q38_exp2(mi - Mt);
            Lt = __builtin_fmaf(w, red_l[i][dl], Lt);
            Ot = q38_fma4(w, red_o[i][dl], Ot);
        }
        f32x4 r = Ot / Lt;
        if (gated) {
            r.x *= q38_sigmoid(gt.x);
            r.y *= q38_sigmoid(gt.y);
            r.z *= q38_sigmoid(gt.z);
            r.w *= q38_sigmoid(gt.w);
        }
        q38_st4(a.out + off, r);
    }
}

/* Rows <-> pages.  grid (n_tokens, 2), 256 threads x float4 = one 1024-float row. */
extern "C" __global__ __launch_bounds__(256) void q38_kv_copy(q38_kv_copy_args a) {
    const int t = blockIdx.x;
    const int which = blockIdx.y;
    const int p = a.pos0 + t;
    const int phys = a.page_table[(size_t)a.seq * a.pt_stride + (p >> 4)];
    float *pool = which ? a.vpool : a.kpool;
    float *rows = which ? a.v_rows : a.k_rows;
    const int e = 4 * threadIdx.x;
    const int head = e >> 8;
    const int d = e & 255;
    float *page_ptr = pool + ((size_t)phys * Q38_ATTN_KV_HEADS + head) * Q38_PAGE_TOKENS * Q38_ATTN_HEAD_DIM +
                      (size_t)(p & 15) * Q38_ATTN_HEAD_DIM + d;
    float *row_ptr = rows + (size_t)t * Q38_ATTN_KV_DIM + e;
    if (a.to_pages)
        q38_st4(page_ptr, q38_ld4(row_ptr));
    else
        q38_st4(row_ptr, q38_ld4(page_ptr));
}

/* q/gate split + q RMSNorm (ops.rs:832-843), k RMSNorm (ops.rs:844-850) and
 * RoPE on lanes (p, p+32), p < 32 (ops.rs:595-610, applied :851-856).
 * grid (n_tokens, 7), 256 threads: one wave per head (4 per workgroup), lane i
 * holds dims 4i..4i+3.  The token's 32 RoPE angles and their cosines and
 * sines are formed once per workgroup (wave 0, while every wave's loads are
 * in flight) and read from LDS by its 4 heads. */
extern "C" __global__ __launch_bounds__(256) void q38_attn_pre(q38_attn_pre_args a) {
    __shared__ float cs[32][2];
    const int t = blockIdx.x;
    const int hd = 4 * blockIdx.y + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int position = a.pos0 + t;
    const bool is_q = hd < Q38_ATTN_HEADS;
    const float *src;
    const float *w;
    float *dst;
    if (is_q) {
        src = a.q_and_gate + ((size_t)t * Q38_ATTN_HEADS + hd) * 2 * Q38_ATTN_HEAD_DIM;
        w = a.q_norm;
        dst = a.q_out + ((size_t)t * Q38_ATTN_HEADS + hd) * Q38_ATTN_HEAD_DIM;
    } else {
        const int kh = hd - Q38_ATTN_HEADS;
        src = a.key + ((size_t)t * Q38_ATTN_KV_HEADS + kh) * Q38_ATTN_HEAD_DIM;
        w = a.k_norm;
        dst = a.k_out + ((size_t)t * Q38_ATTN_KV_HEADS + kh) * Q38_ATTN_HEAD_DIM;
    }
    /* every load before the first store (the outputs may alias the inputs
     * as far as the compiler knows, and a load after a store waits for it) */
    f32x4 x = q38_ld4(src + 4 * lane);
    const f32x4 wv = q38_ld4(w + 4 * lane);
    const f32x4 gt = is_q ? q38_ld4(src + Q38_ATTN_HEAD_DIM + 4 * lane) : f32x4{0.f, 0.f, 0.f, 0.f};
    if (threadIdx.x < 64) q38_rope_table(cs, lane, position, a.theta_scale);
    if (is_q) q38_st4(a.gate_out + ((size_t)t * Q38_ATTN_HEADS + hd) * Q38_ATTN_HEAD_DIM + 4 * lane, gt);
    __syncthreads();
    q38_norm_rope4_cs(x, wv, lane, cs);
    q38_st4(dst + 4 * lane, x);
}
