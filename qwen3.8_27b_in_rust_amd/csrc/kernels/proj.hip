/*
 * Weight projections (gfx950, wave64): the Q8_K activation quantiser and the
 * K-quant x Q8_K row dots the reference runs for every projection of the
 * model (project, src/model/ops.rs:623-639).
 *
 * Reference semantics:
 *   quantize_q8_k      src/kernel/quant.rs:55-128 (quantize_block per 256 values)
 *   dot_q4_k_q8_k      src/kernel/tensor.rs:365-391
 *   dot_q5_k_q8_k      src/kernel/tensor.rs:393-428
 *   dot_q6_k_q8_k      src/kernel/tensor.rs:430-457
 *   tensor_gemv_q8_k / tensor_gemm_q8_k, tensor.rs:1131-1173, :1217-1270:
 *                      out[token * rows + row] = one row dot per element
 *
 * q38_quantize_q8k: one wave per 256-value block, 4 values per lane.  The
 * first element with the largest |x| (the reference's strict-greater scan)
 * comes out of a butterfly reduction on (|x|, index, x) that prefers the
 * lower index on ties; the inverse scale -127/max and the scale 1/inverse are
 * IEEE divisions; each quant is the reference's round-to-nearest-even by
 * adding 1.5 * 2^23 and reading the mantissa, clamped at 127.  Bit-exact.
 *
 * q38_gemv_q8k_*: one wave per weight row, 16 lanes per 256-weight block, so a
 * wave covers 4 blocks per step.  Each lane unpacks its share of the block's
 * 4-bit (plus fifth or fifth-and-sixth bit) weights into bytes and multiplies
 * them with the Q8_K quants on v_dot4_i32_i8; the block's integer sums meet
 * in a 16-lane reduction, exactly (integer arithmetic).  Each block's f32
 * term -- d * weighted - dmin * minimum, d and dmin the f16 scales times the
 * activation scale -- is formed with the reference's separate multiplies
 * and subtraction, and the terms are added to the row total in block order,
 * so the result equals the reference's bit for bit.  Up to 8 tokens reuse
 * the weights loaded for a step (the batched form's token loop).
 */
#include "q38_device.h"

namespace {

/* f16_to_f32 (quant.rs:22-47): subnormals are m * 2^-24 exactly. */
Q38_DEV float q38_f16(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0) return __uint_as_float(__float_as_uint((float)m * 5.9604644775390625e-8f) | sign);
    if (e == 31) return __uint_as_float(sign | 0x7f800000u | (m << 13));
    return __uint_as_float(sign | ((e + 112u) << 23) | (m << 13));
}

/* nearest_int (quant.rs:16-20) */
Q38_DEV int q38_nearest_int(float v) {
    const float shifted = v + 12582912.0f;
    return (int)(__float_as_uint(shifted) & 0x007fffffu) - 0x00400000;
}

Q38_DEV int q38_sdot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }

/* integer sum over the 16 lanes of a lane's group */
Q38_DEV int q38_isum16(int x) {
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) x += __shfl_xor(x, m, 64);
    return x;
}

/* Byte i (0..11) of the 12 packed scale bytes held in three words. */
Q38_DEV int q38_sbyte(uint32_t s0, uint32_t s1, uint32_t s2, int i) {
    const uint32_t w = i < 4 ? s0 : (i < 8 ? s1 : s2);
    return (int)((w >> (8 * (i & 3))) & 255u);
}

/* scale_min_k4 (tensor.rs:23-32) */
Q38_DEV void q38_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j, int &sc, int &mn) {
    if (j < 4) {
        sc = q38_sbyte(s0, s1, s2, j) & 63;
        mn = q38_sbyte(s0, s1, s2, j + 4) & 63;
    } else {
        sc = (q38_sbyte(s0, s1, s2, j + 4) & 15) | ((q38_sbyte(s0, s1, s2, j - 4) >> 6) << 4);
        mn = (q38_sbyte(s0, s1, s2, j + 4) >> 4) | ((q38_sbyte(s0, s1, s2, j) >> 6) << 4);
    }
}

/* A 32-bit word at a 2-byte-aligned address (Q6_K blocks are 210 bytes). */
Q38_DEV uint32_t q38_ld_u32_a2(const uint8_t *p) {
    const uint16_t *h = reinterpret_cast<const uint16_t *>(p);
    return (uint32_t)h[0] | ((uint32_t)h[1] << 16);
}

struct Q8kView {
    const int8_t *quants;  /* [T][W] */
    const int16_t *sums;   /* [T][B][16] */
    const float *scales;   /* [T][B] */
};

Q38_DEV Q8kView q8k_view(const void *q8k, int n_tokens, int width) {
    const int blocks = width / Q38_Q8K_BLOCK;
    Q8kView v;
    v.quants = static_cast<const int8_t *>(q8k);
    v.sums = reinterpret_cast<const int16_t *>(v.quants + (size_t)n_tokens * width);
    v.scales = reinterpret_cast<const float *>(v.sums + (size_t)n_tokens * blocks * 16);
    return v;
}

/* The weights of one block that one lane needs, loaded once per step. */
struct WLane {
    uint32_t h0, s0, s1, s2; /* Q4_K/Q5_K header: d | dmin << 16, 12 scale bytes; Q6_K: d in h0 */
    uint32_t q[2];           /* Q4_K/Q5_K: 8 bytes of 4-bit pairs; Q6_K: low quants of i0.. and i0+32.. */
    uint32_t x[2];           /* Q5_K: 8 bytes of fifth bits; Q6_K: x[0] high-bit byte quad */
    int sc6[4];              /* Q6_K: the lane's 4 signed scales */
};

template <int TYPE>
Q38_DEV WLane load_weights(const uint8_t *blk, int t) {
    WLane w{};
    if (TYPE == Q38_GGML_Q6_K) {
        const int h = t >> 3, i0 = 4 * (t & 7);
        w.q[0] = q38_ld_u32_a2(blk + 64 * h + i0);
        w.q[1] = q38_ld_u32_a2(blk + 64 * h + 32 + i0);
        w.x[0] = q38_ld_u32_a2(blk + 128 + 32 * h + i0);
        const int si = 8 * h + (t & 7) / 4;
#pragma unroll
        for (int k = 0; k < 4; ++k) w.sc6[k] = (int)(int8_t)blk[192 + si + 2 * k];
        w.h0 = *reinterpret_cast<const uint16_t *>(blk + 208);
    } else {
        const uint4 hdr = *reinterpret_cast<const uint4 *>(blk);
        w.h0 = hdr.x;
        w.s0 = hdr.y;
        w.s1 = hdr.z;
        w.s2 = hdr.w;
        const int c = t >> 2, sub = t & 3;
        const int qs_off = (TYPE == Q38_GGML_Q4_K ? 16 : 48) + 32 * c + 8 * sub;
        const uint2 qs = *reinterpret_cast<const uint2 *>(blk + qs_off);
        w.q[0] = qs.x;
        w.q[1] = qs.y;
        if (TYPE == Q38_GGML_Q5_K) {
            const uint2 qh = *reinterpret_cast<const uint2 *>(blk + 16 + 8 * sub);
            w.x[0] = qh.x;
            w.x[1] = qh.y;
        }
    }
    return w;
}

/* The f32 term of one block against one token (lane 0 of the block's 16
 * lanes holds it): dot_q4/q5/q6_k_q8_k's per-block update. */
template <int TYPE>
Q38_DEV float block_term(const WLane &w, const Q8kView &qv, int width, int blocks, int tok, int blk, int t) {
    const int8_t *qa = qv.quants + (size_t)tok * width + (size_t)blk * Q38_Q8K_BLOCK;
    const float a_scale = qv.scales[(size_t)tok * blocks + blk];
    if (TYPE == Q38_GGML_Q6_K) {
        const int h = t >> 3, i0 = 4 * (t & 7);
        const uint32_t lo = w.q[0], lo2 = w.q[1], hb = w.x[0];
        const uint32_t q[4] = {(lo & 0x0F0F0F0Fu) | ((hb & 0x03030303u) << 4),
                               (lo2 & 0x0F0F0F0Fu) | (((hb >> 2) & 0x03030303u) << 4),
                               ((lo >> 4) & 0x0F0F0F0Fu) | (((hb >> 4) & 0x03030303u) << 4),
                               ((lo2 >> 4) & 0x0F0F0F0Fu) | (((hb >> 6) & 0x03030303u) << 4)};
        int weighted = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t a4 = *reinterpret_cast<const uint32_t *>(qa + 128 * h + 32 * k + i0);
            /* sum of (q - 32) * a over the 4 bytes */
            const int dot = q38_sdot4(q[k], a4, 0) - 32 * q38_sdot4(0x01010101u, a4, 0);
            weighted += w.sc6[k] * dot;
        }
        weighted = q38_isum16(weighted);
        const float d = q38_f16(w.h0) * a_scale;
        return d * (float)weighted;
    } else {
        const int c = t >> 2, sub = t & 3;
        const uint2 alo = *reinterpret_cast<const uint2 *>(qa + 64 * c + 8 * sub);
        const uint2 ahi = *reinterpret_cast<const uint2 *>(qa + 64 * c + 32 + 8 * sub);
        uint32_t wl[2], wh[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            wl[k] = w.q[k] & 0x0F0F0F0Fu;
            wh[k] = (w.q[k] >> 4) & 0x0F0F0F0Fu;
            if (TYPE == Q38_GGML_Q5_K) {
                wl[k] |= ((w.x[k] >> (2 * c)) & 0x01010101u) << 4;
                wh[k] |= ((w.x[k] >> (2 * c + 1)) & 0x01010101u) << 4;
            }
        }
        const int dot0 = q38_sdot4(wl[1], alo.y, q38_sdot4(wl[0], alo.x, 0));
        const int dot1 = q38_sdot4(wh[1], ahi.y, q38_sdot4(wh[0], ahi.x, 0));
        int sc0, m0, sc1, m1;
        q38_scale_min(w.s0, w.s1, w.s2, 2 * c, sc0, m0);
        q38_scale_min(w.s0, w.s1, w.s2, 2 * c + 1, sc1, m1);
        int weighted = sc0 * dot0 + sc1 * dot1;
        int minimum = 0;
        if (sub == 0) {
            const int16_t *bs = qv.sums + ((size_t)tok * blocks + blk) * 16 + 4 * c;
            const uint2 b4 = *reinterpret_cast<const uint2 *>(bs);
            const int b0 = (int)(int16_t)(b4.x & 0xffffu), b1 = (int)(int16_t)(b4.x >> 16);
            const int b2 = (int)(int16_t)(b4.y & 0xffffu), b3 = (int)(int16_t)(b4.y >> 16);
            minimum = m0 * (b0 + b1) + m1 * (b2 + b3);
        }
        weighted = q38_isum16(weighted);
        minimum = q38_isum16(minimum);
        const float d = q38_f16(w.h0 & 0xffffu) * a_scale;
        const float dmin = q38_f16(w.h0 >> 16) * a_scale;
        return d * (float)weighted - dmin * (float)minimum;
    }
}

template <int TYPE>
Q38_DEV void gemv_q8k(const q38_gemv_args &a) {
    constexpr int kBlockBytes = TYPE == Q38_GGML_Q4_K ? 144 : (TYPE == Q38_GGML_Q5_K ? 176 : 210);
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + wave;
    if (row >= a.rows) return; /* the whole wave; the kernel has no barrier */
    const int tok0 = blockIdx.y * Q38_GEMV_TOKENS;
    const int ntok = min(Q38_GEMV_TOKENS, a.n_tokens - tok0);
    const int width = a.width;
    const int blocks = width / Q38_Q8K_BLOCK;
    const int grp = lane >> 4;
    const int t = lane & 15;
    const Q8kView qv = q8k_view(a.q8k, a.n_tokens, width);
    const uint8_t *wrow = a.weights + (size_t)row * blocks * kBlockBytes;
    float total[Q38_GEMV_TOKENS];
#pragma unroll
    for (int k = 0; k < Q38_GEMV_TOKENS; ++k) total[k] = 0.0f;

    for (int b0 = 0; b0 < blocks; b0 += 4) {
        const int blk = b0 + grp;
        const int blkc = blk < blocks ? blk : b0; /* a block that exists; its term is not added */
        const WLane w = load_weights<TYPE>(wrow + (size_t)blkc * kBlockBytes, t);
        const int n_here = min(4, blocks - b0);
#pragma unroll
        for (int k = 0; k < Q38_GEMV_TOKENS; ++k) {
            if (k >= ntok) break;
            const float term = block_term<TYPE>(w, qv, width, blocks, tok0 + k, blkc, t);
            /* the row total in block order: blocks b0, b0+1, ... */
#pragma unroll
            for (int g = 0; g < 4; ++g)
                if (g < n_here)
                    total[k] += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(term), 16 * g));
        }
    }
#pragma unroll
    for (int k = 0; k < Q38_GEMV_TOKENS; ++k)
        if (k < ntok && lane == k) a.out[(size_t)(tok0 + k) * a.rows + row] = total[k];
}

}  // namespace

extern "C" __global__ __launch_bounds__(64) void q38_quantize_q8k(q38_quantize_args a) {
    const int b = blockIdx.x;
    const int tok = blockIdx.y;
    const int lane = threadIdx.x;
    const int width = a.width;
    const int blocks = width / Q38_Q8K_BLOCK;
    int8_t *quants = static_cast<int8_t *>(a.q8k);
    int16_t *sums = reinterpret_cast<int16_t *>(quants + (size_t)a.n_tokens * width);
    float *scales = reinterpret_cast<float *>(sums + (size_t)a.n_tokens * blocks * 16);
    const size_t k = (size_t)tok * blocks + b;
    const f32x4 v = q38_ld4(a.x + (size_t)tok * width + (size_t)b * Q38_Q8K_BLOCK + 4 * lane);

    /* the first element of the block with the largest |x| */
    float best = fabsf(v.x), val = v.x;
    int idx = 4 * lane;
#pragma unroll
    for (int c = 1; c < 4; ++c) {
        if (fabsf(v[c]) > best) {
            best = fabsf(v[c]);
            val = v[c];
            idx = 4 * lane + c;
        }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float ob = __shfl_xor(best, m, 64);
        const float ov = __shfl_xor(val, m, 64);
        const int oi = __shfl_xor(idx, m, 64);
        if (ob > best || (ob == best && oi < idx)) {
            best = ob;
            val = ov;
            idx = oi;
        }
    }
    int8_t *qo = quants + k * Q38_Q8K_BLOCK;
    if (best == 0.0f) {
        reinterpret_cast<uint32_t *>(qo)[lane] = 0u;
        if (lane < 16) sums[k * 16 + lane] = 0;
        if (lane == 0) scales[k] = 0.0f;
        return;
    }
    const float inverse_scale = -127.0f / val;
    int q[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) q[c] = min(q38_nearest_int(inverse_scale * v[c]), 127);
    reinterpret_cast<uint32_t *>(qo)[lane] = (uint32_t)(q[0] & 255) | ((uint32_t)(q[1] & 255) << 8) |
                                             ((uint32_t)(q[2] & 255) << 16) | ((uint32_t)(q[3] & 255) << 24);
    int s = q[0] + q[1] + q[2] + q[3];
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    if ((lane & 3) == 0) sums[k * 16 + lane / 4] = (int16_t)s;
    if (lane == 0) scales[k] = 1.0f / inverse_scale;
}

extern "C" __global__ __launch_bounds__(256) void q38_gemv_q8k_q4k(q38_gemv_args a) { gemv_q8k<Q38_GGML_Q4_K>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemv_q8k_q5k(q38_gemv_args a) { gemv_q8k<Q38_GGML_Q5_K>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemv_q8k_q6k(q38_gemv_args a) { gemv_q8k<Q38_GGML_Q6_K>(a); }
