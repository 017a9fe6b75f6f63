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
 *   dot_q2_k_q8_k      src/kernel/tensor.rs:301-333
 *   dot_q3_k_q8_k      src/kernel/tensor.rs:335-363 (unpack_q3_scales :34-44)
 *   dot_iq4_nl_q8_k    src/kernel/iq.rs:355-377 (eight per-group terms per block)
 *   dot_iq4_xs_q8_k    src/kernel/iq.rs:379-405 (code book iq_tables.rs:53-56)
 *   dot_iq2_xxs/_iq2_xs/_iq2_s/_iq3_xxs/_iq3_s/_iq1_s/_iq1_m_q8_k
 *                      src/kernel/iq.rs:407-667 (lattice grids: ggml's
 *                      tables, q38_iq_grids.h, copied into LDS)
 *   dot_f32/f16/bf16/q8_0 (f32 input), tensor.rs:79-117, through
 *                      tensor_gemv_f32 / tensor_gemm_f32, tensor.rs:1095-1129,
 *                      :1175-1215
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
 * q38_gemv_q8k_*: one lane per 256-weight block of one row (a "unit"): the
 * lane loads the block whole (rows are contiguous, so a wave's loads cover a
 * contiguous stretch of the matrix), unpacks its 4-bit (plus fifth, or fifth
 * and sixth, bit) weights into bytes and multiplies them with the token's
 * Q8_K quants, staged in LDS, on v_dot4_i32_i8.  The block's integer sums are
 * exact; its f32 term -- d * weighted - dmin * minimum, d and dmin the f16
 * scales times the activation scale -- is formed with the reference's
 * separate multiplies and subtraction, and one lane per row adds the terms
 * in block order, so the result equals the reference's bit for bit.  Up to
 * 8 tokens reuse the weights a lane holds (the batched form's token loop).
 */
#include "q38_device.h"
#include "../q38_iq_grids.h"

namespace {

/* f16_to_f32 (quant.rs:22-47): the hardware conversion is exact for every
 * half (subnormals included; f16 denormals are not flushed). */
Q38_DEV float q38_f16(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xffffu)); }

/* nearest_int (quant.rs:16-20) */
Q38_DEV int q38_nearest_int(float v) {
    const float shifted = v + 12582912.0f;
    return (int)(__float_as_uint(shifted) & 0x007fffffu) - 0x00400000;
}

Q38_DEV int q38_sdot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }

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

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

/* LDS bytes of one block's 256 int8 quants, padded to 272 (68 dwords) so that
 * 16 lanes reading consecutive blocks with 16-byte reads touch distinct
 * banks. */
constexpr int kRec = 272;

template <int TYPE> struct KQuant;
template <> struct KQuant<Q38_GGML_Q4_K> { static constexpr int bytes = 144, words = 36; };
template <> struct KQuant<Q38_GGML_Q5_K> { static constexpr int bytes = 176, words = 44; };
template <> struct KQuant<Q38_GGML_Q6_K> { static constexpr int bytes = 210, words = 52; };
template <> struct KQuant<Q38_GGML_Q3_K> { static constexpr int bytes = 110, words = 27; };
template <> struct KQuant<Q38_GGML_IQ4_XS> { static constexpr int bytes = 136, words = 34; };
template <> struct KQuant<Q38_GGML_Q2_K> { static constexpr int bytes = 84, words = 21; };
template <> struct KQuant<Q38_GGML_IQ4_NL> { static constexpr int bytes = 144, words = 36; };
template <> struct KQuant<Q38_GGML_IQ2_XXS> { static constexpr int bytes = 66, words = 17; };
template <> struct KQuant<Q38_GGML_IQ2_XS> { static constexpr int bytes = 74, words = 19; };
template <> struct KQuant<Q38_GGML_IQ2_S> { static constexpr int bytes = 82, words = 21; };
template <> struct KQuant<Q38_GGML_IQ3_XXS> { static constexpr int bytes = 98, words = 25; };
template <> struct KQuant<Q38_GGML_IQ3_S> { static constexpr int bytes = 110, words = 28; };
template <> struct KQuant<Q38_GGML_IQ1_S> { static constexpr int bytes = 50, words = 13; };
template <> struct KQuant<Q38_GGML_IQ1_M> { static constexpr int bytes = 56, words = 14; };

/* The IQ lattice grids (format data) and the bytes a workgroup copies into
 * LDS: 8-byte entries (IQ2, IQ1: 8 weights) or 4-byte ones (IQ3: 4). */
__device__ __attribute__((aligned(16))) const uint64_t kIq2xxsGrid[256] = Q38_IQ2XXS_GRID;
__device__ __attribute__((aligned(16))) const uint64_t kIq2xsGrid[512] = Q38_IQ2XS_GRID;
__device__ __attribute__((aligned(16))) const uint64_t kIq2sGrid[1024] = Q38_IQ2S_GRID;
__device__ __attribute__((aligned(16))) const uint32_t kIq3xxsGrid[256] = Q38_IQ3XXS_GRID;
__device__ __attribute__((aligned(16))) const uint32_t kIq3sGrid[512] = Q38_IQ3S_GRID;
__device__ __attribute__((aligned(16))) const uint64_t kIq1sGrid[2048] = Q38_IQ1S_GRID;
template <int TYPE> struct IqGrid { static constexpr int bytes = 0; };
template <> struct IqGrid<Q38_GGML_IQ2_XXS> { static constexpr int bytes = sizeof(kIq2xxsGrid); };
template <> struct IqGrid<Q38_GGML_IQ2_XS> { static constexpr int bytes = sizeof(kIq2xsGrid); };
template <> struct IqGrid<Q38_GGML_IQ2_S> { static constexpr int bytes = sizeof(kIq2sGrid); };
template <> struct IqGrid<Q38_GGML_IQ3_XXS> { static constexpr int bytes = sizeof(kIq3xxsGrid); };
template <> struct IqGrid<Q38_GGML_IQ3_S> { static constexpr int bytes = sizeof(kIq3sGrid); };
template <> struct IqGrid<Q38_GGML_IQ1_S> { static constexpr int bytes = sizeof(kIq1sGrid); };
template <> struct IqGrid<Q38_GGML_IQ1_M> { static constexpr int bytes = sizeof(kIq1sGrid); };
template <int TYPE> Q38_DEV const void *iq_grid_table() {
    if (TYPE == Q38_GGML_IQ2_XXS) return kIq2xxsGrid;
    if (TYPE == Q38_GGML_IQ2_XS) return kIq2xsGrid;
    if (TYPE == Q38_GGML_IQ2_S) return kIq2sGrid;
    if (TYPE == Q38_GGML_IQ3_XXS) return kIq3xxsGrid;
    if (TYPE == Q38_GGML_IQ3_S) return kIq3sGrid;
    return kIq1sGrid;
}

/* Bytes of a block held as little-endian words from its start (the indices
 * are constants once the loops over groups and sections are unrolled). */
Q38_DEV uint32_t wbyte(const uint32_t *w, int b) { return (w[b >> 2] >> (8 * (b & 3))) & 255u; }
Q38_DEV uint32_t whalf(const uint32_t *w, int b) { return (w[b >> 2] >> (8 * (b & 3))) & 0xffffu; } /* b even */
Q38_DEV uint32_t wword(const uint32_t *w, int b) {                                                  /* b even */
    return (b & 3) ? (w[b >> 2] >> 16) | (w[(b >> 2) + 1] << 16) : w[b >> 2];
}

/* ksigns_iq2xs[i]: the 7 stored sign bits and an eighth that makes the
 * count of minus signs even */
Q38_DEV uint32_t iq_ksigns(uint32_t i) { return i | ((uint32_t)(__builtin_popcount(i) & 1) << 7); }

/* The 4 grid bytes of x (each 1..127) negated where bit j of m (j < 4) is
 * set: (x ^ 0xFF) + 1 per byte, no carry since no byte is 0. */
Q38_DEV uint32_t iq_signed4(uint32_t x, uint32_t m) {
    const uint32_t t = ((m & 15u) * 0x00204081u) & 0x01010101u;
    return (x ^ (t * 0xFFu)) + t;
}

/* f32 terms a block adds to its row's total, in order: one (d * weighted
 * [- dmin * minimum]) for the K-quants and IQ4_XS, one per 32-weight group
 * for IQ4_NL (its groups carry their own f16 scales) */
template <int TYPE> struct BlockTerms { static constexpr int n = 1; };
template <> struct BlockTerms<Q38_GGML_IQ4_NL> { static constexpr int n = 8; };

/* ggml's IQ4_NL / IQ4_XS code book as int8 bytes, 4 per word:
 * -127 -104 -83 -65 | -49 -35 -22 -10 | 1 13 25 38 | 53 69 89 113 */
constexpr uint32_t kIq4Lut[4] = {0xBFAD9881u, 0xF6EADDCFu, 0x26190D01u, 0x71594535u};

/* The code-book values of 4 nibbles (one per byte, 0..15) as 4 int8 bytes:
 * v_perm_b32 picks byte n & 7 of the low or high half of the book, and
 * bit 3 of each nibble chooses between the two. */
Q38_DEV uint32_t q38_iq4_lookup(uint32_t nib) {
    const uint32_t sel = nib & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(kIq4Lut[1], kIq4Lut[0], sel);
    const uint32_t hi = __builtin_amdgcn_perm(kIq4Lut[3], kIq4Lut[2], sel);
    const uint32_t mask = ((nib >> 3) & 0x01010101u) * 0xFFu;
    return (hi & mask) | (lo & ~mask);
}

/* One 256-weight block of one row (a "unit"), held by one lane. */
template <int TYPE> struct Unit {
    uint32_t w[KQuant<TYPE>::words];
    uint32_t dh; /* Q6_K: the f16 scale (bytes 208-209) */
};

/* Unit g of the matrix (row-major: g = row * B + block).  Q4_K and Q5_K
 * blocks are multiples of 16 bytes and start 16-byte aligned.  Q6_K blocks
 * are 210 bytes and start 2-byte aligned: the 208 bytes before the scale are
 * read as 52 dwords from the dword boundary at or below the start (16-byte
 * reads need dword alignment only) plus the halfword at 206, and shifted into
 * place; the scale is its own halfword.  Every byte read lies in the block. */
/* IQ blocks of S bytes, S = 2 (mod 4), start 2-byte aligned: the block as
 * (S + 2) / 4 words from its start.  (S - 2) / 4 whole words are read from
 * the dword boundary at or below the start, then the block's last bytes --
 * the halfword that ends it when the start is dword aligned, else the
 * dword that ends it -- and the window is shifted into place.  Every byte
 * read lies in the block or, for a start 2 bytes past a dword boundary, in
 * the 2 bytes before it (block 0 starts dword aligned). */
template <int S>
Q38_DEV void load_block_2aligned(const uint8_t *weights, size_t g, uint32_t *w) {
    constexpr int n = (S - 2) / 4;
    const size_t s = g * S;
    const uint32_t o = (uint32_t)(s & 3); /* 0 or 2 */
    const uint32_t *base = reinterpret_cast<const uint32_t *>(weights + (s - o));
    uint32_t win[n + 2];
#pragma unroll
    for (int i = 0; i < n / 4; ++i) {
        u32x4 v;
        __builtin_memcpy(&v, base + 4 * i, 16);
        win[4 * i] = v.x;
        win[4 * i + 1] = v.y;
        win[4 * i + 2] = v.z;
        win[4 * i + 3] = v.w;
    }
#pragma unroll
    for (int i = (n / 4) * 4; i < n; ++i) win[i] = base[i];
    const uint32_t tail_dword = base[o ? n : n - 1]; /* o == 0: an inner word, not used */
    const uint32_t tail_half = *reinterpret_cast<const uint16_t *>(weights + s + S - 2);
    win[n] = o ? tail_dword : tail_half;
    win[n + 1] = 0;
#pragma unroll
    for (int j = 0; j <= n; ++j) w[j] = __builtin_amdgcn_alignbyte(win[j + 1], win[j], o);
}

template <int TYPE>
Q38_DEV void load_unit(const uint8_t *weights, size_t g, Unit<TYPE> &u) {
    if constexpr (TYPE == Q38_GGML_IQ2_XXS || TYPE == Q38_GGML_IQ2_XS || TYPE == Q38_GGML_IQ2_S ||
                  TYPE == Q38_GGML_IQ3_XXS || TYPE == Q38_GGML_IQ3_S || TYPE == Q38_GGML_IQ1_S) {
        static_assert(KQuant<TYPE>::bytes % 4 == 2 && KQuant<TYPE>::words == (KQuant<TYPE>::bytes + 2) / 4,
                      "a 2-byte aligned IQ block");
        load_block_2aligned<KQuant<TYPE>::bytes>(weights, g, u.w);
        u.dh = 0;
    } else if constexpr (TYPE == Q38_GGML_IQ1_M) {
        /* 56-byte blocks start 8-byte aligned */
        const uint32_t *p = reinterpret_cast<const uint32_t *>(weights + g * KQuant<TYPE>::bytes);
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            u32x4 v;
            __builtin_memcpy(&v, p + 4 * i, 16);
            u.w[4 * i] = v.x;
            u.w[4 * i + 1] = v.y;
            u.w[4 * i + 2] = v.z;
            u.w[4 * i + 3] = v.w;
        }
        u.w[12] = p[12];
        u.w[13] = p[13];
        u.dh = 0;
    } else if (TYPE == Q38_GGML_Q3_K) {
        /* 110-byte blocks start 2-byte aligned: the 108 bytes before the
         * scale are read as 27 dwords from the dword boundary at or below
         * the start plus the halfword at 106, and shifted into place; the
         * f16 scale is its own halfword.  Every byte read lies in the block
         * or (the 2 bytes below an odd start) in the one before it. */
        const size_t s = g * 110;
        const uint32_t o = (uint32_t)(s & 3); /* 0 or 2 */
        const uint32_t *base = reinterpret_cast<const uint32_t *>(weights + (s - o));
        uint32_t win[28];
#pragma unroll
        for (int i = 0; i < 6; ++i) {
            u32x4 v;
            __builtin_memcpy(&v, base + 4 * i, 16);
            win[4 * i] = v.x;
            win[4 * i + 1] = v.y;
            win[4 * i + 2] = v.z;
            win[4 * i + 3] = v.w;
        }
        win[24] = base[24];
        win[25] = base[25];
        win[26] = base[26];
        win[27] = *reinterpret_cast<const uint16_t *>(weights + s + 106);
        u.dh = *reinterpret_cast<const uint16_t *>(weights + s + 108);
#pragma unroll
        for (int j = 0; j < 27; ++j) u.w[j] = __builtin_amdgcn_alignbyte(win[j + 1], win[j], o);
    } else if (TYPE == Q38_GGML_Q2_K) {
        /* 84-byte blocks start 4-byte aligned */
        const uint32_t *p = reinterpret_cast<const uint32_t *>(weights + g * 84);
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            u32x4 v;
            __builtin_memcpy(&v, p + 4 * i, 16);
            u.w[4 * i] = v.x;
            u.w[4 * i + 1] = v.y;
            u.w[4 * i + 2] = v.z;
            u.w[4 * i + 3] = v.w;
        }
        u.w[20] = p[20];
        u.dh = 0;
    } else if (TYPE == Q38_GGML_IQ4_XS) {
        /* 136-byte blocks start 8-byte aligned */
        const uint32_t *p = reinterpret_cast<const uint32_t *>(weights + g * 136);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            u32x4 v;
            __builtin_memcpy(&v, p + 4 * i, 16);
            u.w[4 * i] = v.x;
            u.w[4 * i + 1] = v.y;
            u.w[4 * i + 2] = v.z;
            u.w[4 * i + 3] = v.w;
        }
        u.w[32] = p[32];
        u.w[33] = p[33];
        u.dh = 0;
    } else if (TYPE == Q38_GGML_Q6_K) {
        const size_t s = g * 210;
        const uint32_t o = (uint32_t)(s & 3); /* 0 or 2 */
        const uint32_t *base = reinterpret_cast<const uint32_t *>(weights + (s - o));
        uint32_t win[53];
#pragma unroll
        for (int i = 0; i < 13; ++i) {
            u32x4 v;
            __builtin_memcpy(&v, base + 4 * i, 16);
            win[4 * i] = v.x;
            win[4 * i + 1] = v.y;
            win[4 * i + 2] = v.z;
            win[4 * i + 3] = v.w;
        }
        win[52] = *reinterpret_cast<const uint16_t *>(weights + s + 206);
        u.dh = *reinterpret_cast<const uint16_t *>(weights + s + 208);
#pragma unroll
        for (int j = 0; j < 52; ++j) u.w[j] = __builtin_amdgcn_alignbyte(win[j + 1], win[j], o);
    } else {
        const uint4 *p = reinterpret_cast<const uint4 *>(weights + g * KQuant<TYPE>::bytes);
#pragma unroll
        for (int i = 0; i < KQuant<TYPE>::words / 4; ++i) {
            const uint4 v = p[i];
            u.w[4 * i] = v.x;
            u.w[4 * i + 1] = v.y;
            u.w[4 * i + 2] = v.z;
            u.w[4 * i + 3] = v.w;
        }
        u.dh = 0;
    }
}

/* Per-unit constants: the 8 (Q4_K/Q5_K: scale, min) pairs or the 16 signed
 * Q6_K scales, and the f16 scales as f32. */
template <int TYPE> struct UnitScales {
    int sc[16];
    int mn[8];
    float gd[8]; /* IQ4_NL: the groups' scales */
    float d, dmin;
};

template <int TYPE>
Q38_DEV void unit_scales(const Unit<TYPE> &u, UnitScales<TYPE> &s) {
    s.dmin = 0.0f;
    if constexpr (TYPE == Q38_GGML_IQ2_XXS) {
        /* group g: 4 grid indices at 2 + 8g, then a word of 4 x 7 sign bits
         * and the scale in bits 28-31; d = IQ1_DELTA * d (iq.rs:489) */
#pragma unroll
        for (int g = 0; g < 8; ++g) s.sc[g] = 1 + 2 * (int)(wword(u.w, 6 + 8 * g) >> 28);
        s.d = 0.125f * q38_f16(u.w[0]);
    } else if constexpr (TYPE == Q38_GGML_IQ2_XS || TYPE == Q38_GGML_IQ2_S) {
        /* one scale byte per group (sections 0-1: low nibble, 2-3: high) */
        constexpr int at = TYPE == Q38_GGML_IQ2_XS ? 66 : 74;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint32_t b = wbyte(u.w, at + g);
            s.sc[2 * g] = 1 + 2 * (int)(b & 15u);
            s.sc[2 * g + 1] = 1 + 2 * (int)(b >> 4);
        }
        s.d = 0.125f * q38_f16(u.w[0]);
    } else if constexpr (TYPE == Q38_GGML_IQ3_XXS) {
        /* group g's word at 66 + 4g: 4 x 7 sign bits, the scale in 28-31;
         * d = 0.25 * d (iq.rs:453) */
#pragma unroll
        for (int g = 0; g < 8; ++g) s.sc[g] = 1 + 2 * (int)(wword(u.w, 66 + 4 * g) >> 28);
        s.d = 0.25f * q38_f16(u.w[0]);
    } else if constexpr (TYPE == Q38_GGML_IQ3_S) {
        /* group g: nibble g % 2 of scale byte 106 + g / 2 */
#pragma unroll
        for (int g = 0; g < 8; ++g) s.sc[g] = 1 + 2 * (int)((wbyte(u.w, 106 + g / 2) >> (4 * (g % 2))) & 15u);
        s.d = q38_f16(u.w[0]);
    } else if constexpr (TYPE == Q38_GGML_IQ1_S) {
        /* group g's halfword at 34 + 2g: 3 index bits per section, the
         * scale in bits 12-14, the delta's sign in bit 15 */
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint32_t qh = whalf(u.w, 34 + 2 * g);
            s.sc[g] = 1 + 2 * (int)((qh >> 12) & 7u);
            s.mn[g] = (qh & 0x8000u) ? -1 : 1;
        }
        s.d = q38_f16(u.w[0]);
    } else if constexpr (TYPE == Q38_GGML_IQ1_M) {
        /* 3-bit scales in the halfwords at 48..55 (group g: halfword g / 2,
         * bits 6 (g % 2) .. +5); d is their four top nibbles */
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint32_t sc = whalf(u.w, 48 + 2 * (g / 2));
            const int shift = 6 * (g % 2);
            s.sc[2 * g] = 1 + 2 * (int)((sc >> shift) & 7u);
            s.sc[2 * g + 1] = 1 + 2 * (int)((sc >> (shift + 3)) & 7u);
        }
        const uint32_t bits = (whalf(u.w, 48) >> 12) | ((whalf(u.w, 50) >> 8) & 0x00f0u) |
                              ((whalf(u.w, 52) >> 4) & 0x0f00u) | (whalf(u.w, 54) & 0xf000u);
        s.d = q38_f16(bits);
    } else if (TYPE == Q38_GGML_Q3_K) {
        /* unpack_q3_scales: low nibble from byte i (i < 8) or the high
         * nibble of byte i - 8, high 2 bits from byte 8 + i % 4 at 2 (i / 4);
         * the 12 scale bytes are block bytes 96..107, words 24..26 */
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int low = i < 8 ? q38_sbyte(u.w[24], u.w[25], u.w[26], i) & 15
                                  : q38_sbyte(u.w[24], u.w[25], u.w[26], i - 8) >> 4;
            const int high = (q38_sbyte(u.w[24], u.w[25], u.w[26], 8 + i % 4) >> (2 * (i / 4))) & 3;
            s.sc[i] = (low | (high << 4)) - 32;
        }
        s.d = q38_f16(u.dh);
        s.dmin = 0.0f;
    } else if (TYPE == Q38_GGML_Q2_K) {
        /* the 16 scale bytes (low nibble scale, high nibble minimum) */
#pragma unroll
        for (int g = 0; g < 16; ++g) s.sc[g] = (int)((u.w[g >> 2] >> (8 * (g & 3))) & 255u);
        s.d = q38_f16(u.w[20]);
        s.dmin = q38_f16(u.w[20] >> 16);
    } else if (TYPE == Q38_GGML_IQ4_NL) {
        /* group g's f16 scale is the halfword at byte 18 g */
#pragma unroll
        for (int g = 0; g < 8; ++g) s.gd[g] = q38_f16(u.w[(18 * g) >> 2] >> (8 * ((18 * g) & 3)));
        s.d = 0.0f;
        s.dmin = 0.0f;
    } else if (TYPE == Q38_GGML_IQ4_XS) {
        /* group g: low 4 bits from scales_l[g / 2] (nibble g % 2), high 2
         * bits from scales_h at 2g; offset 32 */
        const uint32_t sh = u.w[0] >> 16, sl = u.w[1];
#pragma unroll
        for (int g = 0; g < 8; ++g) s.sc[g] = (int)(((sl >> (4 * g)) & 15u) | (((sh >> (2 * g)) & 3u) << 4)) - 32;
        s.d = q38_f16(u.w[0]);
        s.dmin = 0.0f;
    } else if (TYPE == Q38_GGML_Q6_K) {
#pragma unroll
        for (int g = 0; g < 16; ++g) s.sc[g] = (int)(int8_t)((u.w[48 + g / 4] >> (8 * (g & 3))) & 255u);
        s.d = q38_f16(u.dh);
        s.dmin = 0.0f;
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) q38_scale_min(u.w[1], u.w[2], u.w[3], j, s.sc[j], s.mn[j]);
        s.d = q38_f16(u.w[0]);
        s.dmin = q38_f16(u.w[0] >> 16);
    }
}

/* The f32 term of one unit against one token's activation block `rec`:
 * dot_q4_k_q8_k / dot_q5_k_q8_k / dot_q6_k_q8_k's per-block update
 * (tensor.rs:365-457).  The integer sums are exact in any order; the f32
 * part is the reference's: d = f16(d) * a.d, then d * weighted - dmin *
 * minimum (Q6_K: d * weighted). */
template <int TYPE>
Q38_DEV float unit_term(const Unit<TYPE> &u, const UnitScales<TYPE> &s, const uint8_t *rec, const int16_t *gsums,
                        float a_scale, const uint8_t *grid) {
    const u32x4 *aq = reinterpret_cast<const u32x4 *>(rec);
    /* 4 activations 4j .. 4j+3 */
    auto a4 = [&](int j) { return aq[j >> 2][j & 3]; };
    auto grid8 = [&](uint32_t idx) { return *reinterpret_cast<const uint2 *>(grid + 8 * idx); };
    auto grid4 = [&](uint32_t idx) { return *reinterpret_cast<const uint32_t *>(grid + 4 * idx); };
    if constexpr (TYPE == Q38_GGML_IQ2_XXS || TYPE == Q38_GGML_IQ2_XS || TYPE == Q38_GGML_IQ2_S ||
                  TYPE == Q38_GGML_IQ3_XXS || TYPE == Q38_GGML_IQ3_S) {
        /* dot_iq2_xxs / _iq2_xs / _iq2_s / _iq3_xxs / _iq3_s_q8_k (iq.rs:407-578):
         * section s of group g is values 32g + 8s .. +7, grid bytes with
         * the section's 8 signs against the activations; the scale weights
         * a group (IQ2_XS, IQ2_S: a pair of sections) */
        int weighted = 0;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            int sub[2] = {0, 0};
#pragma unroll
            for (int sec = 0; sec < 4; ++sec) {
                uint32_t lo, hi, signs;
                if constexpr (TYPE == Q38_GGML_IQ2_XXS) {
                    const uint2 e = grid8(wbyte(u.w, 2 + 8 * g + sec));
                    lo = e.x, hi = e.y;
                    signs = iq_ksigns((wword(u.w, 6 + 8 * g) >> (7 * sec)) & 127u);
                } else if constexpr (TYPE == Q38_GGML_IQ2_XS) {
                    const uint32_t code = whalf(u.w, 2 + 8 * g + 2 * sec);
                    const uint2 e = grid8(code & 511u);
                    lo = e.x, hi = e.y;
                    signs = iq_ksigns(code >> 9);
                } else if constexpr (TYPE == Q38_GGML_IQ2_S) {
                    const uint32_t idx = wbyte(u.w, 2 + 4 * g + sec) | ((wbyte(u.w, 66 + g) << (8 - 2 * sec)) & 0x300u);
                    const uint2 e = grid8(idx);
                    lo = e.x, hi = e.y;
                    signs = wbyte(u.w, 34 + 4 * g + sec);
                } else if constexpr (TYPE == Q38_GGML_IQ3_XXS) {
                    lo = grid4(wbyte(u.w, 2 + 8 * g + 2 * sec));
                    hi = grid4(wbyte(u.w, 3 + 8 * g + 2 * sec));
                    signs = iq_ksigns((wword(u.w, 66 + 4 * g) >> (7 * sec)) & 127u);
                } else {
                    const uint32_t qh = wbyte(u.w, 66 + g);
                    lo = grid4(wbyte(u.w, 2 + 8 * g + 2 * sec) | ((qh << (8 - 2 * sec)) & 0x100u));
                    hi = grid4(wbyte(u.w, 3 + 8 * g + 2 * sec) | ((qh << (7 - 2 * sec)) & 0x100u));
                    signs = wbyte(u.w, 74 + 4 * g + sec);
                }
                int t = q38_sdot4(iq_signed4(lo, signs), a4(8 * g + 2 * sec), 0);
                t = q38_sdot4(iq_signed4(hi, signs >> 4), a4(8 * g + 2 * sec + 1), t);
                sub[sec / 2] += t;
            }
            if constexpr (TYPE == Q38_GGML_IQ2_XS || TYPE == Q38_GGML_IQ2_S)
                weighted += s.sc[2 * g] * sub[0] + s.sc[2 * g + 1] * sub[1];
            else
                weighted += s.sc[g] * (sub[0] + sub[1]);
            /* IQ2: one group's grid loads at a time (215-226 registers, two
             * waves per SIMD); scheduled freely the unrolled groups' loads
             * need 260 registers, and capped at 256 they spill (6% slower) */
            if constexpr (TYPE == Q38_GGML_IQ2_XXS || TYPE == Q38_GGML_IQ2_XS || TYPE == Q38_GGML_IQ2_S)
                __builtin_amdgcn_sched_barrier(0);
        }
        return s.d * a_scale * (float)weighted;
    }
    if constexpr (TYPE == Q38_GGML_IQ1_S || TYPE == Q38_GGML_IQ1_M) {
        /* dot_iq1_s_q8_k / dot_iq1_m_q8_k (iq.rs:580-667): signed grid bytes
         * (-1, 0, 1) plus a delta of +-1/8 per group (IQ1_S, through the
         * activations' group sums) or per section (IQ1_M) */
        int weighted = 0, correction = 0;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            int dot[2] = {0, 0}, cdot[2] = {0, 0};
#pragma unroll
            for (int sec = 0; sec < 4; ++sec) {
                uint32_t idx;
                int delta = 1;
                if constexpr (TYPE == Q38_GGML_IQ1_S) {
                    idx = wbyte(u.w, 2 + 4 * g + sec) | (((whalf(u.w, 34 + 2 * g) >> (3 * sec)) & 7u) << 8);
                } else {
                    const uint32_t hb = wbyte(u.w, 32 + 2 * g + sec / 2);
                    idx = wbyte(u.w, 4 * g + sec) | ((hb << (sec % 2 ? 4 : 8)) & 0x700u);
                    delta = (hb & (sec % 2 ? 0x80u : 0x08u)) ? -1 : 1;
                }
                const uint2 e = grid8(idx);
                const uint32_t a0 = a4(8 * g + 2 * sec), a1 = a4(8 * g + 2 * sec + 1);
                dot[sec / 2] += q38_sdot4(e.y, a1, q38_sdot4(e.x, a0, 0));
                if constexpr (TYPE == Q38_GGML_IQ1_M)
                    cdot[sec / 2] += delta * q38_sdot4(0x01010101u, a1, q38_sdot4(0x01010101u, a0, 0));
            }
            if constexpr (TYPE == Q38_GGML_IQ1_S) {
                weighted += s.sc[g] * (dot[0] + dot[1]);
                correction += s.sc[g] * s.mn[g] * ((int)gsums[2 * g] + (int)gsums[2 * g + 1]);
            } else {
                weighted += s.sc[2 * g] * dot[0] + s.sc[2 * g + 1] * dot[1];
                correction += s.sc[2 * g] * cdot[0] + s.sc[2 * g + 1] * cdot[1];
            }
        }
        return s.d * a_scale * ((float)weighted + 0.125f * (float)correction);
    }
    const u32x4 bs4[2] = {reinterpret_cast<const u32x4 *>(gsums)[0], reinterpret_cast<const u32x4 *>(gsums)[1]};
    int bsum[16];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t v = bs4[k / 4][k & 3];
        bsum[2 * k] = (int)(int16_t)(v & 0xffffu);
        bsum[2 * k + 1] = (int)(int16_t)(v >> 16);
    }
    if (TYPE == Q38_GGML_Q2_K) {
        /* group s (16 values 16s..16s+15: half s / 8, field (s % 8) / 2,
         * lanes 16 (s % 2)..+15): 2-bit quants times the low nibble of
         * scale byte s, minus the high nibble times the group's sum */
        int weighted = 0, minimum = 0;
#pragma unroll
        for (int g = 0; g < 16; ++g) {
            const int half = g >> 3, field = (g >> 1) & 3, part = g & 1;
            const u32x4 av = aq[g];
            int dot = 0;
#pragma unroll
            for (int c = 0; c < 4; ++c)
                dot = q38_sdot4((u.w[4 + 8 * half + 4 * part + c] >> (2 * field)) & 0x03030303u, av[c], dot);
            weighted += (s.sc[g] & 15) * dot;
            minimum += (s.sc[g] >> 4) * bsum[g];
        }
        const float d = s.d * a_scale;
        const float dmin = s.dmin * a_scale;
        return d * (float)weighted - dmin * (float)minimum;
    } else if (TYPE == Q38_GGML_Q3_K) {
        /* group s (16 values 16s..16s+15: half s / 8, field (s % 8) / 2,
         * lanes 16 (s % 2)..+15): q = 2 low bits + 4 * high bit in 0..7 is
         * the reference's qv + 4, so sum qv a = dot(q, a) - 4 * bsum[s] */
        int weighted = 0;
#pragma unroll
        for (int g = 0; g < 16; ++g) {
            const int half = g >> 3, field = (g >> 1) & 3, part = g & 1;
            const u32x4 av = aq[g];
            int dot = 0;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint32_t low = (u.w[8 + 8 * half + 4 * part + c] >> (2 * field)) & 0x03030303u;
                const uint32_t hb = (u.w[4 * part + c] >> (4 * half + field)) & 0x01010101u;
                dot = q38_sdot4(low | (hb << 2), av[c], dot);
            }
            weighted += s.sc[g] * (dot - 4 * bsum[g]);
        }
        const float d = s.d * a_scale;
        return d * (float)weighted;
    } else if (TYPE == Q38_GGML_IQ4_XS) {
        /* group g: its 16 quant bytes hold values 32g..32g+15 in the low
         * nibbles and 32g+16.. in the high ones */
        int weighted = 0;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const u32x4 alo = aq[2 * g], ahi = aq[2 * g + 1];
            int sub = 0;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint32_t x = u.w[2 + 4 * g + c];
                sub = q38_sdot4(q38_iq4_lookup(x & 0x0F0F0F0Fu), alo[c], sub);
                sub = q38_sdot4(q38_iq4_lookup((x >> 4) & 0x0F0F0F0Fu), ahi[c], sub);
            }
            weighted += s.sc[g] * sub;
        }
        const float d = s.d * a_scale;
        return d * (float)weighted;
    } else if (TYPE == Q38_GGML_Q6_K) {
        int dg[16];
#pragma unroll
        for (int g = 0; g < 16; ++g) dg[g] = 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i4 = 0; i4 < 8; i4 += 4) {
                /* activation dwords of values 128h + 32k + 4i4 .. +15, k = 0..3 */
                u32x4 av[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) av[k] = aq[(128 * h + 32 * k + 4 * i4) / 16];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const uint32_t lo = u.w[16 * h + i4 + c], hi = u.w[16 * h + 8 + i4 + c];
                    const uint32_t qh = u.w[32 + 8 * h + i4 + c];
                    const uint32_t q0 = (lo & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u);
                    const uint32_t q1 = (hi & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u);
                    const uint32_t q2 = ((lo >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u);
                    const uint32_t q3 = ((hi >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u);
                    const int g = 8 * h + i4 / 4;
                    dg[g] = q38_sdot4(q0, av[0][c], dg[g]);
                    dg[g + 2] = q38_sdot4(q1, av[1][c], dg[g + 2]);
                    dg[g + 4] = q38_sdot4(q2, av[2][c], dg[g + 4]);
                    dg[g + 6] = q38_sdot4(q3, av[3][c], dg[g + 6]);
                }
            }
        }
        int weighted = 0;
#pragma unroll
        for (int g = 0; g < 16; ++g) weighted += s.sc[g] * (dg[g] - 32 * bsum[g]);
        const float d = s.d * a_scale;
        return d * (float)weighted;
    } else {
        int weighted = 0, minimum = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int dot0 = 0, dot1 = 0;
#pragma unroll
            for (int i4 = 0; i4 < 8; i4 += 4) {
                const u32x4 alo = aq[(64 * j + 4 * i4) / 16];
                const u32x4 ahi = aq[(64 * j + 32 + 4 * i4) / 16];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int i = i4 + c;
                    uint32_t ql, qh;
                    if (TYPE == Q38_GGML_Q4_K) {
                        const uint32_t q = u.w[4 + 8 * j + i];
                        ql = q & 0x0F0F0F0Fu;
                        qh = (q >> 4) & 0x0F0F0F0Fu;
                    } else {
                        const uint32_t q = u.w[12 + 8 * j + i], hb = u.w[4 + i];
                        ql = (q & 0x0F0F0F0Fu) | (((hb >> (2 * j)) & 0x01010101u) << 4);
                        qh = ((q >> 4) & 0x0F0F0F0Fu) | (((hb >> (2 * j + 1)) & 0x01010101u) << 4);
                    }
                    dot0 = q38_sdot4(ql, alo[c], dot0);
                    dot1 = q38_sdot4(qh, ahi[c], dot1);
                }
            }
            weighted += s.sc[2 * j] * dot0 + s.sc[2 * j + 1] * dot1;
            minimum += s.mn[2 * j] * (bsum[4 * j] + bsum[4 * j + 1]) + s.mn[2 * j + 1] * (bsum[4 * j + 2] + bsum[4 * j + 3]);
        }
        const float d = s.d * a_scale;
        const float dmin = s.dmin * a_scale;
        return d * (float)weighted - dmin * (float)minimum;
    }
}

/* IQ4_NL's eight group terms of one unit against one token's activation
 * block (dot_iq4_nl_q8_k's per-group update, iq.rs:363-374): group g's 16
 * quant bytes start at byte 18 g + 2 (2 bytes off a dword for even g). */
Q38_DEV void unit_terms_iq4nl(const Unit<Q38_GGML_IQ4_NL> &u, const UnitScales<Q38_GGML_IQ4_NL> &s,
                              const uint8_t *rec, float a_scale, float *out) {
    const u32x4 *aq = reinterpret_cast<const u32x4 *>(rec);
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        const int base = (18 * g + 2) >> 2;
        const uint32_t o = (uint32_t)((18 * g + 2) & 3);
        const u32x4 alo = aq[2 * g], ahi = aq[2 * g + 1];
        int sub = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t x = o ? __builtin_amdgcn_alignbyte(u.w[base + c + 1], u.w[base + c], o) : u.w[base + c];
            sub = q38_sdot4(q38_iq4_lookup(x & 0x0F0F0F0Fu), alo[c], sub);
            sub = q38_sdot4(q38_iq4_lookup((x >> 4) & 0x0F0F0F0Fu), ahi[c], sub);
        }
        const float d = s.gd[g] * a_scale;
        out[g] = d * (float)sub;
    }
}

/* The (|x|, first index) maximum of a row of 16 lanes: each lane offers its
 * candidate (best = |x|, val = x, idx = position in the block); a larger
 * |x| wins, equal ones go to the lower index, so the order of the
 * exchanges does not matter.  Four DPP steps (quad swaps, half-row and row
 * mirrors) leave the row's winner in all 16 lanes. */
Q38_DEV void row16_argmax(float &best, float &val, int &idx) {
    auto step = [&](auto ctrl_tag) {
        constexpr int ctrl = decltype(ctrl_tag)::value;
        const float ob = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, best), ctrl,
                                                                                0xF, 0xF, false));
        const float ov = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, val), ctrl,
                                                                                0xF, 0xF, false));
        const int oi = __builtin_amdgcn_update_dpp(0, idx, ctrl, 0xF, 0xF, false);
        if (ob > best || (ob == best && oi < idx)) {
            best = ob;
            val = ov;
            idx = oi;
        }
    };
    step(std::integral_constant<int, 0xB1>{});  /* quad_perm 1,0,3,2 */
    step(std::integral_constant<int, 0x4E>{});  /* quad_perm 2,3,0,1 */
    step(std::integral_constant<int, 0x141>{}); /* row_half_mirror */
    step(std::integral_constant<int, 0x140>{}); /* row_mirror */
}

/* quantize_q8_k of one 256-value block (src/kernel/quant.rs:97-128) by a
 * row of 16 lanes, lane g holding values 16 g .. 16 g + 15 in v: the value
 * of largest |x| (the first such, as the reference's scan keeps it) sets
 * inverse_scale = -127 / x; each value becomes min(nearest(inverse_scale
 * x), 127).
 * qw: the lane's 16 quants packed 4 per word; gsum: their sum (the block's
 * group sum g); scale: 1 / inverse_scale.  An all-zero block gives zeros. */
Q38_DEV void q8k_quantize_group16(const f32x4 (&v)[4], int g, uint32_t (&qw)[4], int &gsum, float &scale) {
    float best = fabsf(v[0].x), val = v[0].x;
    int idx = 16 * g;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (c == 0 && e == 0) continue;
            if (fabsf(v[c][e]) > best) {
                best = fabsf(v[c][e]);
                val = v[c][e];
                idx = 16 * g + 4 * c + e;
            }
        }
    row16_argmax(best, val, idx);
    if (best == 0.0f) {
#pragma unroll
        for (int c = 0; c < 4; ++c) qw[c] = 0u;
        gsum = 0;
        scale = 0.0f;
        return;
    }
    const float inverse_scale = -127.0f / val;
    int sum = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        int q[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) q[e] = min(q38_nearest_int(inverse_scale * v[c][e]), 127);
        sum += q[0] + q[1] + q[2] + q[3];
        qw[c] = (uint32_t)(q[0] & 255) | ((uint32_t)(q[1] & 255) << 8) | ((uint32_t)(q[2] & 255) << 16) |
                ((uint32_t)(q[3] & 255) << 24);
    }
    gsum = sum;
    scale = 1.0f / inverse_scale;
}

/*
 * A workgroup owns rows [row0, row0 + R) of one of up to Q38_GEMV_MAX_MATS
 * matrices that read the same activations, and the tokens [tok0, tok0 + tp);
 * its R * B units (at most Q38_GEMV_UNITS_MAX) are taken by the 256 lanes in
 * steps of 256:
 *   1. each lane issues the loads of its first unit, then the workgroup
 *      copies the tp tokens' Q8_K blocks into LDS (quants [t][b] in
 *      kRec-byte records, group sums [t][b][16], scales [t][b]);
 *   2. at each step a lane issues the loads of its next unit before it
 *      computes the current one (past the workgroup's last unit it loads
 *      that unit again, a cache hit, so the wait counts are static), and
 *      writes the unit's f32 term per token into LDS;
 *   3. one lane per (row, token) adds the row's B terms in block order, the
 *      reference's `total += ...` sequence, and stores the result.
 * The host sizes R and tp (LDS: tp * B * Q38_GEMV_REC_BYTES + tp * R * B * 4).
 * When the tokens take several passes, the passes of one row group are
 * workgroups 8 ids apart: they start together on one XCD, and all but the
 * first find the rows' weights in its L2 rather than in HBM.
 */
template <int TYPE>
Q38_DEV void gemv_q8k(const q38_gemv_args &a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x;
    const int width = a.width;
    const int B = width / Q38_Q8K_BLOCK;
    /* (row group, token pass) of this workgroup */
    int grp = (int)blockIdx.x, pass = 0;
    if (a.tok_groups > 1) {
        const int q = (int)(blockIdx.x >> 3);
        pass = q % a.tok_groups;
        grp = (q / a.tok_groups) * 8 + (int)(blockIdx.x & 7);
        if (grp >= a.wg_begin[a.n_mats]) return; /* the grid's round-up to 8 row groups */
    }
    /* the matrix of this row group: matrices share the activations and
     * take consecutive ranges of row groups */
    int mat = 0;
#pragma unroll
    for (int i = 1; i < Q38_GEMV_MAX_MATS; ++i) mat += (i < a.n_mats && grp >= a.wg_begin[i]) ? 1 : 0;
    const uint8_t *weights = a.weights[mat];
    float *out = a.out[mat];
    const int rows = a.rows[mat];
    const int R = a.rows_per_wg[mat];
    const int row0 = (grp - a.wg_begin[mat]) * R;
    const int rows_here = min(R, rows - row0);
    const int units = rows_here * B;
    const int steps = (units + 255) >> 8;
    const int tok0 = pass * a.tok_pass;
    const int tp = min(a.tok_pass, a.n_tokens - tok0);
    const int nrec = a.tok_pass * B;
    /* an IQ format's lattice grid first, then the staged activations */
    constexpr int kGridBytes = IqGrid<TYPE>::bytes;
    uint8_t *grid = lds;
    if (kGridBytes > 0) {
        const u32x4 *src = static_cast<const u32x4 *>(iq_grid_table<TYPE>());
        for (int i = tid; i < kGridBytes / 16; i += 256) reinterpret_cast<u32x4 *>(grid)[i] = src[i];
    }
    uint8_t *recs = lds + kGridBytes;                                        /* [tp][B] x kRec */
    int16_t *lsums = reinterpret_cast<int16_t *>(recs + (size_t)nrec * kRec); /* [tp][B][16] */
    float *lscales = reinterpret_cast<float *>(lsums + (size_t)nrec * 16);   /* [tp][B] */
    constexpr int NT = BlockTerms<TYPE>::n;
    float *terms = lscales + nrec;                                           /* [tp][units][NT] */
    const size_t g0 = (size_t)row0 * B;

    /* the tokens' blocks are contiguous from token tok0 in each of the three
     * planes: quants [T][W], sums [T][B][16], scales [T][B] */
    const int8_t *quants = static_cast<const int8_t *>(a.q8k) + (size_t)tok0 * width;
    const int16_t *sums = reinterpret_cast<const int16_t *>(quants - (size_t)tok0 * width + (size_t)a.n_tokens * width);
    const float *scales = reinterpret_cast<const float *>(sums + (size_t)a.n_tokens * B * 16) + (size_t)tok0 * B;
    sums += (size_t)tok0 * B * 16;
    const int nblk = tp * B;
    const int nq16 = nblk * 16, ns16 = nblk * 2; /* 16-byte pieces of quants and of sums */
    const bool from_x = a.x != nullptr;
    const int g = tid & 15;
    const float *xs = a.x + (size_t)tok0 * width;
    /* the activations' first loads go out before the weights' (loads return
     * in order): with the f32 input, the first two rounds of 16 blocks (see
     * below); else the first 4 quant pieces, one sums piece and one scale of
     * every thread (indices past the end reload the last piece and are not
     * written) */
    f32x4 v0[2][4];
    u32x4 qv[4], sv;
    float sc;
    if (from_x) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int i = min(16 * r + (tid >> 4), nblk - 1);
#pragma unroll
            for (int c = 0; c < 4; ++c) v0[r][c] = q38_ld4(xs + (size_t)i * 256 + 16 * g + 4 * c);
        }
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k)
            qv[k] = *reinterpret_cast<const u32x4 *>(quants + (size_t)min(256 * k + tid, nq16 - 1) * 16);
        sv = *reinterpret_cast<const u32x4 *>(sums + (size_t)min(tid, ns16 - 1) * 8);
        sc = scales[min(tid, nblk - 1)];
    }
    Unit<TYPE> w[2];
    load_unit<TYPE>(weights, g0 + min(tid, units - 1), w[0]);

    if (from_x) {
        /* quantise the pass's tokens from the f32 input: block i (token
         * tok0 + i / B, block i % B, values x[tok0 * W + 256 i ..]) by the
         * 16 threads 16 (i % 16) .. + 15 of a round of 16 blocks, thread
         * 16 b + g holding values 16 g .. 16 g + 15, two rounds' loads at a
         * time.  The first row group of the pass also stores them to q8k. */
        const bool store = grp == 0;
        int8_t *gq = const_cast<int8_t *>(quants);
        int16_t *gs = const_cast<int16_t *>(sums);
        float *gsc = const_cast<float *>(scales);
        for (int i0 = 0; i0 < nblk; i0 += 32) {
            f32x4 v[2][4];
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const int i = min(i0 + 16 * r + (tid >> 4), nblk - 1);
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    v[r][c] = i0 == 0 ? v0[r][c] : q38_ld4(xs + (size_t)i * 256 + 16 * g + 4 * c);
            }
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const int i = i0 + 16 * r + (tid >> 4);
                uint32_t qw[4];
                int gsum;
                float scale;
                q8k_quantize_group16(v[r], g, qw, gsum, scale);
                if (i < nblk) {
                    *reinterpret_cast<u32x4 *>(recs + i * kRec + 16 * g) = u32x4{qw[0], qw[1], qw[2], qw[3]};
                    lsums[i * 16 + g] = (int16_t)gsum;
                    if (g == 0) lscales[i] = scale;
                    if (store) {
                        *reinterpret_cast<u32x4 *>(gq + (size_t)i * 256 + 16 * g) = u32x4{qw[0], qw[1], qw[2], qw[3]};
                        gs[(size_t)i * 16 + g] = (int16_t)gsum;
                        if (g == 0) gsc[i] = scale;
                    }
                }
            }
        }
    } else {
        {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int p = 256 * k + tid;
                if (p < nq16) *reinterpret_cast<u32x4 *>(recs + (p >> 4) * kRec + (p & 15) * 16) = qv[k];
            }
            if (tid < ns16) *reinterpret_cast<u32x4 *>(lsums + tid * 8) = sv;
            if (tid < nblk) lscales[tid] = sc;
        }
        for (int p = 1024 + tid; p < nq16; p += 256)
            *reinterpret_cast<u32x4 *>(recs + (p >> 4) * kRec + (p & 15) * 16) =
                *reinterpret_cast<const u32x4 *>(quants + (size_t)p * 16);
        for (int p = 256 + tid; p < ns16; p += 256)
            *reinterpret_cast<u32x4 *>(lsums + p * 8) = *reinterpret_cast<const u32x4 *>(sums + (size_t)p * 8);
        for (int p = 256 + tid; p < nblk; p += 256) lscales[p] = scales[p];
    }
    __syncthreads();

#pragma unroll
    for (int k = 0; k < Q38_GEMV_UNITS_MAX / 256; ++k) {
        if (k >= steps) break;
        const int u = tid + 256 * k;
        load_unit<TYPE>(weights, g0 + min(u + 256, units - 1), w[(k + 1) & 1]);
        if (u < units) {
            UnitScales<TYPE> s;
            unit_scales<TYPE>(w[k & 1], s);
            const int b = u % B;
            for (int t = 0; t < tp; ++t) {
                const int r = t * B + b;
                if constexpr (NT == 1)
                    terms[t * units + u] =
                        unit_term<TYPE>(w[k & 1], s, recs + r * kRec, lsums + r * 16, lscales[r], grid);
                else
                    unit_terms_iq4nl(w[k & 1], s, recs + r * kRec, lscales[r], terms + ((size_t)t * units + u) * NT);
            }
        }
    }
    __syncthreads();

    for (int i = tid; i < tp * rows_here; i += 256) {
        const int t = i / rows_here, r = i - t * rows_here;
        const float *tr = terms + ((size_t)t * units + r * B) * NT;
        float total = 0.0f;
        for (int b = 0; b < B * NT; ++b) total += tr[b];
        out[(size_t)(tok0 + t) * rows + row0 + r] = total;
    }
}

/*
 * The batched form for many tokens (tensor_gemm_q8_k, tensor.rs:1217-1270):
 * the same per-block integer sums and f32 block terms, with the integer
 * dot products on the int8 matrix unit (v_mfma_i32_32x32x32_i8, exact).
 * A workgroup of 4 waves owns 128 rows x 64 tokens; wave w owns rows
 * 128 bx + 32 w .. + 31 (lane l: row l % 32, k half l / 32 of each 32-value
 * step) and both 32-token tiles.  The activations are the MFMA's first
 * operand (tokens x k, from LDS), the weights its second (k x rows, unpacked
 * in registers from the lane's own copy of its row's block), so every
 * lane's accumulator column is its own row: element 4J+i of a tile is token
 * 8J + 4(l/32) + i.  A block's weights and activations are loaded, then
 * computed, without prefetch: at 160-220 registers (accumulators in
 * ordinary VGPRs, the file built with -amdgpu-mfma-vgpr-form) two or three
 * workgroups share a CU and cover each other's loads, where a prefetching
 * form held 300-400 registers and one.
 *  - the sub-block scale goes into the weights, split into two byte planes
 *    accumulated over the block: Q4_K w = sc q with sc = 8 sh + sl, planes
 *    q sh and q sl (packed 16-bit products, weighted = 8 C_hi + C_lo);
 *    Q5_K w = sc q and Q6_K w = sc (q - 32) (a k step holds two 16-value
 *    groups, one per lane half), |w| <= 4096, planes w = 128 hi + lo (hi
 *    signed, lo in 0..127, weighted = 128 C_hi + C_lo);
 *  - Q4_K / Q5_K's minimum term sum_j m_j bsum_j is a third MFMA, of the
 *    activations against m_j splatted over its sub-block (sum_i m_j(i) a_i);
 *  - the other formats take the same form (gemm_step_bytes): Q3_K w = sc
 *    (q - 4) and Q2_K w = sc q per 16-value group with Q2_K's minimum as the
 *    third MFMA; IQ4_XS the code book's values biased by 128; the lattice
 *    formats their grid bytes (from LDS) with signs, biased by 64 (IQ2, IQ3)
 *    or 1 (IQ1), IQ1's delta correction as the third MFMA against scale x
 *    delta.  IQ4_NL, whose eight groups each end in their own f32 term,
 *    has a kernel of its own (q38_gemm_q8k_iq4nl).
 * Every integer is exact; the f32 block term and the row total follow the
 * reference's operation order, so the result equals q38_gemv_q8_k's (and
 * the reference's) bit for bit.
 */
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
constexpr int kGemmRows = 128;
constexpr int kGemmTokens = Q38_GEMM_TOKENS; /* tiles of 32 */
constexpr int kGemmTiles = kGemmTokens / 32;
constexpr int kStagePieces = kGemmTokens * 16 / 256; /* 16-byte activation pieces per thread and block */
constexpr int kActRow = 272; /* LDS bytes of one token's 256 quants: 16-byte pad, conflict-free reads */

Q38_DEV i32x16 mfma_i8(i32x4 a, i32x4 b, i32x16 c) { return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0); }

/* Four weights w = sc * (q - off) (q the unpacked bytes, |w| <= 4096) split
 * into byte planes w = 128 hi + lo, hi signed, lo in 0..127; the arithmetic
 * runs on packed 16-bit lanes (even and odd bytes, w = q sc - off sc in one
 * multiply-add), and a byte permute gathers each plane's low bytes. */
Q38_DEV void split_weights(uint32_t q, int sc, short off, uint32_t &hi, uint32_t &lo) {
    const s16x2 s2 = {(short)sc, (short)sc};
    const short c = (short)(-off * sc);
    const s16x2 c2 = {c, c};
    const s16x2 ve = __builtin_bit_cast(s16x2, q & 0x00FF00FFu) * s2 + c2;
    const s16x2 vo = __builtin_bit_cast(s16x2, (q >> 8) & 0x00FF00FFu) * s2 + c2;
    const s16x2 sh = {7, 7};
    /* bytes 0 and 2 of the even lanes, interleaved with those of the odd */
    hi = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, vo >> sh), __builtin_bit_cast(uint32_t, ve >> sh), 0x06020400u);
    lo = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, vo), __builtin_bit_cast(uint32_t, ve), 0x06020400u) & 0x7F7F7F7Fu;
}

/* Formats whose block term has a second integer sum over the activations:
 * a minimum (Q2_K, Q4_K, Q5_K) or the IQ1 delta correction. */
template <int TYPE> constexpr bool kGemmSecond =
    TYPE == Q38_GGML_Q2_K || TYPE == Q38_GGML_Q4_K || TYPE == Q38_GGML_Q5_K || TYPE == Q38_GGML_IQ1_S ||
    TYPE == Q38_GGML_IQ1_M;

/* Grid bytes g (1..62) with their signs (bit j of m set: byte j negative),
 * biased by 64: every byte 64 +- g, no carry or borrow between bytes. */
Q38_DEV uint32_t iq_biased4(uint32_t g, uint32_t m) {
    const uint32_t t = ((m & 15u) * 0x00204081u) & 0x01010101u;
    const uint32_t neg = t * 0xFFu;
    return (0x40404040u + (g & ~neg)) - (g & neg);
}

/* Q4_K, Q5_K and Q6_K in the matrix-unit form: a lane reads only its half
 * of the block (load_unit_half) */
template <int TYPE> constexpr bool kGemmHalfUnit =
    TYPE == Q38_GGML_Q4_K || TYPE == Q38_GGML_Q5_K || TYPE == Q38_GGML_Q6_K;

/* 16 bytes at offset r (a multiple of 4) of a block that starts 2 bytes
 * past a dword boundary (o = 2) or on one (o = 0): the dwords from the
 * boundary at or below, shifted into place.  The fifth dword is read only
 * where it lies in the block: at_end (the 16 bytes end 2 bytes before the
 * block does) reads it only for o = 2. */
Q38_DEV u32x4 load16_2aligned(const uint8_t *blk, uint32_t o, int r, bool at_end) {
    const uint32_t *p = reinterpret_cast<const uint32_t *>(blk + r - o);
    u32x4 v;
    __builtin_memcpy(&v, p, 16);
    const uint32_t t = at_end ? p[o ? 4 : 3] : p[4];
    return u32x4{__builtin_amdgcn_alignbyte(v.y, v.x, o), __builtin_amdgcn_alignbyte(v.z, v.y, o),
                 __builtin_amdgcn_alignbyte(v.w, v.z, o), __builtin_amdgcn_alignbyte(t, v.w, o)};
}

/* The words of a Q4_K / Q5_K block that lane half h uses in the matrix-unit
 * form, at the positions where the h = 0 lanes find theirs: the 16-byte
 * header (d, dmin, the 12 scale bytes) in words 0-3; Q5_K's high bits of
 * values 16 h .. + 15 of every sub-block (bytes 16 + 16 h ..) in words 4-7;
 * of each 32-byte quant chunk c the 16 bytes 16 h .. + 15 in words
 * q0 + 8 c .. + 3 (q0 = 4 for Q4_K, 12 for Q5_K).  Blocks start 16-byte
 * aligned; every load is 16 bytes inside the block. */
/* Q6_K blocks (210 bytes, 2-byte aligned; load16_2aligned): of each
 * 32-byte piece of ql (bytes 0-127) and qh (128-191) the 16 bytes 16 h ..
 * + 15 in words 8 p .. + 3 (piece p), the 16 scale bytes in words 48-51
 * and the f16 scale as dh.  Every byte read lies in the block or, for a
 * start 2 bytes past a dword boundary, in the 2 bytes before it (block 0
 * starts dword aligned). */
template <int TYPE>
Q38_DEV void load_unit_half(const uint8_t *weights, size_t g, int h, Unit<TYPE> &u) {
    const uint8_t *blk = weights + g * KQuant<TYPE>::bytes;
    auto put = [&](int at, const u32x4 v) {
        u.w[at] = v.x;
        u.w[at + 1] = v.y;
        u.w[at + 2] = v.z;
        u.w[at + 3] = v.w;
    };
    if constexpr (TYPE == Q38_GGML_Q6_K) {
        const uint32_t o = (uint32_t)((g * 210) & 3); /* 0 or 2 */
#pragma unroll
        for (int i = 0; i < 52; ++i) u.w[i] = 0; /* the other half's words: not read */
#pragma unroll
        for (int p = 0; p < 6; ++p) put(8 * p, load16_2aligned(blk, o, 32 * p + 16 * h, false));
        put(48, load16_2aligned(blk, o, 192, true));
        u.dh = *reinterpret_cast<const uint16_t *>(blk + 208);
        return;
    }
    put(0, *reinterpret_cast<const u32x4 *>(blk));
    constexpr int q0 = TYPE == Q38_GGML_Q5_K ? 12 : 4;
    if constexpr (TYPE == Q38_GGML_Q5_K) put(4, *reinterpret_cast<const u32x4 *>(blk + 16 + 16 * h));
#pragma unroll
    for (int c = 0; c < 4; ++c) put(q0 + 8 * c, *reinterpret_cast<const u32x4 *>(blk + 4 * q0 + 32 * c + 16 * h));
#pragma unroll
    for (int i = 0; i < KQuant<TYPE>::words; ++i)
        if (i >= q0 && ((i - q0) & 7) >= 4) u.w[i] = 0; /* the other half's words: not read */
    if constexpr (TYPE == Q38_GGML_Q5_K) {
#pragma unroll
        for (int i = 8; i < 12; ++i) u.w[i] = 0;
    }
    u.dh = 0;
}

/* 0 for the lane half h = 0, all ones for h = 1, hidden from the optimizer:
 * a choice between two register values made with it stays a bit select and
 * never becomes an index into a register array (which would place the array
 * in scratch memory) */
Q38_DEV uint32_t lane_half_mask(int h) {
    uint32_t m = 0u - (uint32_t)h;
    asm volatile("" : "+v"(m));
    return m;
}

/* The lane's 16 weights of k step st (values 32 st + 16 h .. + 15 of the
 * block) for the formats beyond Q4_K..Q6_K, as unsigned bytes q with the
 * scale sc and offset off of w = sc (q - off), and (kGemmSecond) the bytes
 * the activations meet in the second sum.  hm (lane_half_mask) picks between
 * values computed for both halves, so no register index depends on the lane. */
template <int TYPE>
Q38_DEV void gemm_step_bytes(const Unit<TYPE> &u, const UnitScales<TYPE> &s, int st, uint32_t hm, const uint8_t *grid,
                             uint32_t (&q)[4], int &sc, short &off, uint32_t (&second)[4]) {
    auto sel = [&](uint32_t a0, uint32_t a1) { return (a0 & ~hm) | (a1 & hm); };
    auto seli = [&](int a0, int a1) { return (int)sel((uint32_t)a0, (uint32_t)a1); };
    auto grid8 = [&](uint32_t idx) { return *reinterpret_cast<const uint2 *>(grid + 8 * idx); };
    auto grid4 = [&](uint32_t idx) { return *reinterpret_cast<const uint32_t *>(grid + 4 * idx); };
#pragma unroll
    for (int j = 0; j < 4; ++j) second[j] = 0;
    if constexpr (TYPE == Q38_GGML_Q3_K || TYPE == Q38_GGML_Q2_K) {
        /* the step is 2 bits at shift 2 (st % 4) of the quant bytes of half
         * st / 4, one 16-value group (2 st + h) per lane half; Q3_K adds the
         * high bit from hmask bit st (value q + 4 hbit - 4) */
        const int n = st >> 2, sh = 2 * (st & 3);
        const int sg = seli(s.sc[2 * st], s.sc[2 * st + 1]); /* group 2 st + h */
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if constexpr (TYPE == Q38_GGML_Q3_K) {
                const uint32_t qs = sel(u.w[8 + 8 * n + j], u.w[12 + 8 * n + j]);
                const uint32_t hm = sel(u.w[j], u.w[4 + j]);
                q[j] = ((qs >> sh) & 0x03030303u) | (((hm >> st) & 0x01010101u) << 2);
            } else {
                const uint32_t qs = sel(u.w[4 + 8 * n + j], u.w[8 + 8 * n + j]);
                q[j] = (qs >> sh) & 0x03030303u;
                second[j] = (uint32_t)(sg >> 4) * 0x01010101u;
            }
        }
        sc = TYPE == Q38_GGML_Q3_K ? sg : (sg & 15);
        off = TYPE == Q38_GGML_Q3_K ? (short)4 : (short)0;
    } else if constexpr (TYPE == Q38_GGML_IQ4_XS) {
        /* group st's 16 quant bytes: low nibbles are values 0..15, high
         * nibbles 16..31; the code book's int8 values biased by 128 */
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t b = u.w[2 + 4 * st + j];
            q[j] = q38_iq4_lookup(sel(b, b >> 4) & 0x0F0F0F0Fu) ^ 0x80808080u;
        }
        sc = s.sc[st];
        off = 128;
    } else if constexpr (TYPE == Q38_GGML_IQ1_S || TYPE == Q38_GGML_IQ1_M) {
        /* sections 2h and 2h + 1 of group st: signed grid bytes (-1, 0, 1)
         * biased by 1; the second sum's bytes are scale x delta */
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            uint32_t idx0, idx1;
            int d0 = 1, d1 = 1;
            if constexpr (TYPE == Q38_GGML_IQ1_S) {
                const uint32_t qh = whalf(u.w, 34 + 2 * st);
                idx0 = wbyte(u.w, 2 + 4 * st + k) | (((qh >> (3 * k)) & 7u) << 8);
                idx1 = wbyte(u.w, 2 + 4 * st + 2 + k) | (((qh >> (3 * (2 + k))) & 7u) << 8);
            } else {
                const uint32_t hb0 = wbyte(u.w, 32 + 2 * st), hb1 = wbyte(u.w, 33 + 2 * st);
                idx0 = wbyte(u.w, 4 * st + k) | ((hb0 << (k ? 4 : 8)) & 0x700u);
                idx1 = wbyte(u.w, 4 * st + 2 + k) | ((hb1 << (k ? 4 : 8)) & 0x700u);
                d0 = (hb0 & (k ? 0x80u : 0x08u)) ? -1 : 1;
                d1 = (hb1 & (k ? 0x80u : 0x08u)) ? -1 : 1;
            }
            const uint2 e = grid8(sel(idx0, idx1));
            q[2 * k] = ((e.x ^ 0x80808080u) + 0x01010101u) ^ 0x80808080u;
            q[2 * k + 1] = ((e.y ^ 0x80808080u) + 0x01010101u) ^ 0x80808080u;
            const int scale = TYPE == Q38_GGML_IQ1_S ? s.sc[st] : seli(s.sc[2 * st], s.sc[2 * st + 1]);
            const int delta = TYPE == Q38_GGML_IQ1_S ? s.mn[st] : seli(d0, d1);
            const uint32_t m = (uint32_t)(uint8_t)(int8_t)(scale * delta) * 0x01010101u;
            second[2 * k] = m;
            second[2 * k + 1] = m;
        }
        sc = TYPE == Q38_GGML_IQ1_S ? s.sc[st] : seli(s.sc[2 * st], s.sc[2 * st + 1]);
        off = 1;
    } else {
        /* IQ2 / IQ3: sections 2h and 2h + 1 of group st, grid bytes with
         * their signs, biased by 64 */
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int sa = k, sb = 2 + k; /* the section for h = 0 and for h = 1 */
            uint32_t lo, hi;
            if constexpr (TYPE == Q38_GGML_IQ2_XXS) {
                const uint32_t meta = wword(u.w, 6 + 8 * st);
                const uint2 e = grid8(sel(wbyte(u.w, 2 + 8 * st + sa), wbyte(u.w, 2 + 8 * st + sb)));
                const uint32_t sg = iq_ksigns(sel((meta >> (7 * sa)) & 127u, (meta >> (7 * sb)) & 127u));
                lo = iq_biased4(e.x, sg), hi = iq_biased4(e.y, sg >> 4);
            } else if constexpr (TYPE == Q38_GGML_IQ2_XS) {
                const uint32_t code = sel(whalf(u.w, 2 + 8 * st + 2 * sa), whalf(u.w, 2 + 8 * st + 2 * sb));
                const uint2 e = grid8(code & 511u);
                const uint32_t sg = iq_ksigns(code >> 9);
                lo = iq_biased4(e.x, sg), hi = iq_biased4(e.y, sg >> 4);
            } else if constexpr (TYPE == Q38_GGML_IQ2_S) {
                const uint32_t qh = wbyte(u.w, 66 + st);
                const uint32_t i0 = wbyte(u.w, 2 + 4 * st + sa) | ((qh << (8 - 2 * sa)) & 0x300u);
                const uint32_t i1 = wbyte(u.w, 2 + 4 * st + sb) | ((qh << (8 - 2 * sb)) & 0x300u);
                const uint2 e = grid8(sel(i0, i1));
                const uint32_t sg = sel(wbyte(u.w, 34 + 4 * st + sa), wbyte(u.w, 34 + 4 * st + sb));
                lo = iq_biased4(e.x, sg), hi = iq_biased4(e.y, sg >> 4);
            } else if constexpr (TYPE == Q38_GGML_IQ3_XXS) {
                const uint32_t meta = wword(u.w, 66 + 4 * st);
                const uint32_t g0 = grid4(sel(wbyte(u.w, 2 + 8 * st + 2 * sa), wbyte(u.w, 2 + 8 * st + 2 * sb)));
                const uint32_t g1 = grid4(sel(wbyte(u.w, 3 + 8 * st + 2 * sa), wbyte(u.w, 3 + 8 * st + 2 * sb)));
                const uint32_t sg = iq_ksigns(sel((meta >> (7 * sa)) & 127u, (meta >> (7 * sb)) & 127u));
                lo = iq_biased4(g0, sg), hi = iq_biased4(g1, sg >> 4);
            } else {
                const uint32_t qh = wbyte(u.w, 66 + st);
                const uint32_t a0 = wbyte(u.w, 2 + 8 * st + 2 * sa) | ((qh << (8 - 2 * sa)) & 0x100u);
                const uint32_t a1 = wbyte(u.w, 3 + 8 * st + 2 * sa) | ((qh << (7 - 2 * sa)) & 0x100u);
                const uint32_t b0 = wbyte(u.w, 2 + 8 * st + 2 * sb) | ((qh << (8 - 2 * sb)) & 0x100u);
                const uint32_t b1 = wbyte(u.w, 3 + 8 * st + 2 * sb) | ((qh << (7 - 2 * sb)) & 0x100u);
                const uint32_t sg = sel(wbyte(u.w, 74 + 4 * st + sa), wbyte(u.w, 74 + 4 * st + sb));
                lo = iq_biased4(grid4(sel(a0, b0)), sg), hi = iq_biased4(grid4(sel(a1, b1)), sg >> 4);
            }
            q[2 * k] = lo;
            q[2 * k + 1] = hi;
        }
        sc = (TYPE == Q38_GGML_IQ2_XS || TYPE == Q38_GGML_IQ2_S) ? seli(s.sc[2 * st], s.sc[2 * st + 1]) : s.sc[st];
        off = 64;
    }
}

/* Byte planes of the scaled weights, one MFMA each: the formats whose
 * scaled weights fit a signed byte take one (fold_weights), Q5_K three,
 * the others two. */
template <int TYPE> constexpr int kGemmPlanes =
    (TYPE == Q38_GGML_Q2_K || TYPE == Q38_GGML_Q3_K || TYPE == Q38_GGML_IQ1_S || TYPE == Q38_GGML_IQ1_M) ? 1
    : TYPE == Q38_GGML_Q5_K                                                                           ? 3
                                                                                                      : 2;

/* The one-plane formats' scaled weights as signed bytes, from
 * gemm_step_bytes' unsigned q and scale sc:
 *  - Q2_K w = sc q (sc <= 15, q <= 3: at most 45);
 *  - Q3_K the negated -w = sc (4 - q) (sc in -32..31, q in 0..7: -128..124;
 *    the block sum is negated back), as 16-bit products of the even and
 *    odd bytes whose low bytes are kept;
 *  - IQ1 w = sc (q - 1) (q in 0..2, sc <= 15) as sc q + 128 - sc per byte
 *    (113..158, no carry) with the top bit flipped. */
template <int TYPE>
Q38_DEV uint32_t fold_weights(uint32_t q, int sc) {
    if constexpr (TYPE == Q38_GGML_Q2_K) {
        const u16x2 S = {(unsigned short)sc, (unsigned short)sc};
        return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, q) * S);
    } else if constexpr (TYPE == Q38_GGML_Q3_K) {
        const s16x2 S = {(short)sc, (short)sc}, four = {4, 4};
        const s16x2 e = (four - __builtin_bit_cast(s16x2, q & 0x00FF00FFu)) * S;
        const s16x2 o = (four - __builtin_bit_cast(s16x2, (q >> 8) & 0x00FF00FFu)) * S;
        return (__builtin_bit_cast(uint32_t, e) & 0x00FF00FFu) | ((__builtin_bit_cast(uint32_t, o) & 0x00FF00FFu) << 8);
    } else {
        const u16x2 S = {(unsigned short)sc, (unsigned short)sc};
        const uint32_t p = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, q) * S);
        return (p + (uint32_t)(128 - sc) * 0x01010101u) ^ 0x80808080u;
    }
}

/* One block's f32 terms for a tile of 32 tokens x 32 rows (the lane's 16
 * outputs: row l % 32, tokens 8J + 4(l/32) + i for element 4J + i): the
 * integer sums on the matrix unit, then the reference's f32 block term.
 * A_of(st) gives the lane's 16 activations of k step st (token l % 32,
 * values 32 st + 16 h .. + 15), as_of(e) the activation scale of element e;
 * sink(e, term) takes element e's term. */
template <int TYPE, typename AOf, typename AsOf, typename Sink>
Q38_DEV void gemm_tile_terms(const Unit<TYPE> &u, const UnitScales<TYPE> &s, uint32_t hm, const uint8_t *grid,
                             AOf A_of, AsOf as_of, Sink sink) {
    auto word = [&](int k) { return kGemmHalfUnit<TYPE> ? u.w[k] : (u.w[k] & ~hm) | (u.w[k + 4] & hm); };
    i32x16 wsum = i32x16{}, lsum = i32x16{}, xsum = i32x16{}, msum = i32x16{};
#pragma unroll
    for (int st = 0; st < 8; ++st) {
        i32x4 bh, bl, bx, bm;
        if constexpr (TYPE == Q38_GGML_Q4_K) {
            /* w = sc q with sc = 8 sh + sl: the planes q sh and q sl
             * (at most 15 x 7 = 105 per byte) are packed 16-bit
             * products of the quant bytes, no carry between bytes */
            const unsigned short sh = (unsigned short)(s.sc[st] >> 3), sl = (unsigned short)(s.sc[st] & 7);
            const u16x2 SH = {sh, sh}, SL = {sl, sl};
            const int c = st >> 1, nib = st & 1;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u16x2 q = __builtin_bit_cast(u16x2, (word(4 + 8 * c + j) >> (4 * nib)) & 0x0F0F0F0Fu);
                bh[j] = __builtin_bit_cast(int, q * SH);
                bl[j] = __builtin_bit_cast(int, q * SL);
                bm[j] = s.mn[st] * 0x01010101;
            }
        } else if constexpr (TYPE == Q38_GGML_Q5_K) {
            /* w = sc q, q <= 31: three planes of sc = 16 s2 + 4 s1 +
             * s0 (each at most 3, q s <= 93 per byte) */
            const unsigned short s2 = (unsigned short)(s.sc[st] >> 4), s1 = (unsigned short)((s.sc[st] >> 2) & 3),
                                 s0 = (unsigned short)(s.sc[st] & 3);
            const u16x2 S2 = {s2, s2}, S1 = {s1, s1}, S0 = {s0, s0};
            const int c = st >> 1, nib = st & 1;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t qv = ((word(12 + 8 * c + j) >> (4 * nib)) & 0x0F0F0F0Fu) |
                                    (((word(4 + j) >> st) & 0x01010101u) << 4);
                const u16x2 q = __builtin_bit_cast(u16x2, qv);
                bh[j] = __builtin_bit_cast(int, q * S2);
                bl[j] = __builtin_bit_cast(int, q * S1);
                bx[j] = __builtin_bit_cast(int, q * S0);
                bm[j] = s.mn[st] * 0x01010101;
            }
        } else if constexpr (TYPE == Q38_GGML_Q6_K) {
            const int sc = (int)(((uint32_t)s.sc[2 * st] & ~hm) | ((uint32_t)s.sc[2 * st + 1] & hm));
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int hf = st >> 2, kq = st & 3;
                const uint32_t ql = word(16 * hf + 8 * (kq & 1) + j);
                const uint32_t qh = word(32 + 8 * hf + j);
                const uint32_t q = ((ql >> (4 * (kq >> 1))) & 0x0F0F0F0Fu) | (((qh >> (2 * kq)) & 0x03030303u) << 4);
                uint32_t hi, lo;
                split_weights(q, sc, (short)32, hi, lo);
                bh[j] = (int)hi;
                bl[j] = (int)lo;
            }
        } else {
            uint32_t q[4], second[4];
            int sc;
            short off;
            gemm_step_bytes<TYPE>(u, s, st, hm, grid, q, sc, off, second);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (kGemmPlanes<TYPE> == 1) {
                    bh[j] = (int)fold_weights<TYPE>(q[j], sc);
                } else {
                    uint32_t hi, lo;
                    split_weights(q[j], sc, off, hi, lo);
                    bh[j] = (int)hi;
                    bl[j] = (int)lo;
                }
                bm[j] = (int)second[j];
            }
        }
        const i32x4 A = A_of(st);
        wsum = mfma_i8(A, bh, wsum);
        if constexpr (kGemmPlanes<TYPE> >= 2) lsum = mfma_i8(A, bl, lsum);
        if constexpr (kGemmPlanes<TYPE> >= 3) xsum = mfma_i8(A, bx, xsum);
        if constexpr (kGemmSecond<TYPE>) msum = mfma_i8(A, bm, msum);
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        /* the weighted sum from its planes */
        int ws;
        if constexpr (TYPE == Q38_GGML_Q4_K) ws = wsum[e] * 8 + lsum[e];
        else if constexpr (TYPE == Q38_GGML_Q5_K) ws = wsum[e] * 16 + lsum[e] * 4 + xsum[e];
        else if constexpr (TYPE == Q38_GGML_Q3_K) ws = -wsum[e];
        else if constexpr (kGemmPlanes<TYPE> == 1) ws = wsum[e];
        else ws = wsum[e] * 128 + lsum[e];
        const float as = as_of(e);
        const float d = s.d * as;
        float term;
        if constexpr (TYPE == Q38_GGML_Q2_K || TYPE == Q38_GGML_Q4_K || TYPE == Q38_GGML_Q5_K) {
            const float dmin = s.dmin * as;
            term = d * (float)ws - dmin * (float)msum[e];
        } else if constexpr (TYPE == Q38_GGML_IQ1_S || TYPE == Q38_GGML_IQ1_M) {
            term = d * ((float)ws + 0.125f * (float)msum[e]);
        } else {
            term = d * (float)ws;
        }
        sink(e, term);
    }
}

template <int TYPE>
Q38_DEV void gemm_q8k(const q38_gemv_args &a) {
    __shared__ __align__(16) int8_t act[kGemmTokens][kActRow];
    __shared__ float ascale[kGemmTokens];
    /* an IQ format's lattice grid (the others keep 16 unused bytes) */
    constexpr int kGridBytes = IqGrid<TYPE>::bytes;
    __shared__ __align__(16) uint8_t grid[kGridBytes > 0 ? kGridBytes : 16];
    const int tid = threadIdx.x;
    if constexpr (kGridBytes > 0) {
        const u32x4 *src = static_cast<const u32x4 *>(iq_grid_table<TYPE>());
        for (int i = tid; i < kGridBytes / 16; i += 256) reinterpret_cast<u32x4 *>(grid)[i] = src[i];
    }
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;
    const uint32_t hm = lane_half_mask(h);
    const int width = a.width;
    const int B = width / Q38_Q8K_BLOCK;
    const int rows = a.rows[0];
    const int row = blockIdx.x * kGemmRows + wave * 32 + (lane & 31);
    const int rowc = min(row, rows - 1);
    const int t0 = blockIdx.y * kGemmTokens;
    const int T = a.n_tokens;
    const int8_t *quants = static_cast<const int8_t *>(a.q8k);
    const int16_t *sums = reinterpret_cast<const int16_t *>(quants + (size_t)T * width);
    const float *scales = reinterpret_cast<const float *>(sums + (size_t)T * B * 16);

    float total[kGemmTiles][16];
#pragma unroll
    for (int tt = 0; tt < kGemmTiles; ++tt)
#pragma unroll
        for (int e = 0; e < 16; ++e) total[tt][e] = 0.0f;

    for (int b = 0; b < B; ++b) {
        Unit<TYPE> u;
        if constexpr (kGemmHalfUnit<TYPE>) load_unit_half<TYPE>(a.weights[0], (size_t)rowc * B + b, h, u);
        else load_unit<TYPE>(a.weights[0], (size_t)rowc * B + b, u);
#pragma unroll
        for (int i = 0; i < kStagePieces; ++i) {
            const int p = tid + 256 * i, t = min(t0 + (p >> 4), T - 1), c = p & 15;
            *reinterpret_cast<u32x4 *>(&act[p >> 4][c * 16]) =
                *reinterpret_cast<const u32x4 *>(quants + (size_t)t * width + b * 256 + c * 16);
        }
        if (tid < kGemmTokens) ascale[tid] = scales[(size_t)min(t0 + tid, T - 1) * B + b];
        __syncthreads();
        UnitScales<TYPE> s;
        unit_scales<TYPE>(u, s);
#pragma unroll
        for (int tt = 0; tt < kGemmTiles; ++tt) {
            const int8_t *arow = &act[32 * tt + (lane & 31)][16 * h];
            gemm_tile_terms<TYPE>(
                u, s, hm, grid, [&](int st) { return *reinterpret_cast<const i32x4 *>(arow + 32 * st); },
                [&](int e) { return ascale[32 * tt + 8 * (e >> 2) + 4 * h + (e & 3)]; },
                [&](int e, float term) { total[tt][e] = total[tt][e] + term; });
        }
        __syncthreads();
    }

    if (row < rows) {
#pragma unroll
        for (int tt = 0; tt < kGemmTiles; ++tt)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int tok = t0 + 32 * tt + 8 * (e >> 2) + 4 * h + (e & 3);
                if (tok < T) a.out[0][(size_t)tok * rows + row] = total[tt][e];
            }
    }
}


/* The matrix-unit form with the blocks of a row split over the waves, for
 * grids that the 128-row x 64-token tiles would leave small (few rows or
 * few tokens): a workgroup of W waves (16, 8 or 4 as the grid has at most
 * one workgroup per CU, 1.5, or more) owns 32 rows x 32 tokens, and wave w
 * takes blocks w, w + W, w + 2W, ...  Each block's f32 terms are the ones
 * gemm_q8k forms (gemm_tile_terms); a round of W blocks leaves them in LDS,
 * and the workgroup adds them to the row totals in block order, so every
 * output is the reference's sum bit for bit.  The activations are read
 * straight from the Q8_K rows (tokens past the prompt read the last one;
 * their outputs are not stored).  Up to Q38_GEMV_MAX_MATS matrices of one
 * input share a launch: matrix m takes the 32-row tiles wg_begin[m] ..
 * wg_begin[m+1]-1 along x. */
template <int TYPE, int W>
Q38_DEV void gemm_ks_q8k(const q38_gemv_args &a) {
    constexpr int kThreads = 64 * W;
    /* two rounds' terms: [round & 1][wave][element][lane] */
    __shared__ float terms[2][W][16][64];
    constexpr int kGridBytes = IqGrid<TYPE>::bytes;
    __shared__ __align__(16) uint8_t grid[kGridBytes > 0 ? kGridBytes : 16];
    const int tid = threadIdx.x;
    if constexpr (kGridBytes > 0) {
        const u32x4 *src = static_cast<const u32x4 *>(iq_grid_table<TYPE>());
        for (int i = tid; i < kGridBytes / 16; i += kThreads) reinterpret_cast<u32x4 *>(grid)[i] = src[i];
        __syncthreads();
    }
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;
    const uint32_t hm = lane_half_mask(h);
    const int width = a.width;
    const int B = width / Q38_Q8K_BLOCK;
    /* the matrix of this 32-row tile: matrices take consecutive tile ranges */
    int mat = 0;
#pragma unroll
    for (int i = 1; i < Q38_GEMV_MAX_MATS; ++i) mat += (i < a.n_mats && (int)blockIdx.x >= a.wg_begin[i]) ? 1 : 0;
    const uint8_t *weights = a.weights[mat];
    float *out = a.out[mat];
    const int rows = a.rows[mat];
    const int row0 = ((int)blockIdx.x - a.wg_begin[mat]) * Q38_GEMM_KS_ROWS;
    const int rowc = min(row0 + (lane & 31), rows - 1);
    const int t0 = blockIdx.y * Q38_GEMM_KS_TOKENS;
    const int T = a.n_tokens;
    const int8_t *quants = static_cast<const int8_t *>(a.q8k);
    const int16_t *sums = reinterpret_cast<const int16_t *>(quants + (size_t)T * width);
    const float *scales = reinterpret_cast<const float *>(sums + (size_t)T * B * 16);
    /* the lane's activation row (token t0 + l % 32) and its elements' tokens */
    const int8_t *arow = quants + (size_t)min(t0 + (lane & 31), T - 1) * width + 16 * h;
    int etok[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) etok[e] = min(t0 + 8 * (e >> 2) + 4 * h + (e & 3), T - 1);

    /* the 1024 outputs of the tile: thread i adds up elements i, i + 64 W, ... */
    constexpr int kOwn = 1024 / kThreads;
    float total[kOwn];
#pragma unroll
    for (int k = 0; k < kOwn; ++k) total[k] = 0.0f;
    const int rounds = (B + W - 1) / W;
    for (int r = 0; r < rounds; ++r) {
        const int buf = r & 1;
        const int b = r * W + wave;
        if (b < B) {
            Unit<TYPE> u;
            if constexpr (kGemmHalfUnit<TYPE>) load_unit_half<TYPE>(weights, (size_t)rowc * B + b, h, u);
            else load_unit<TYPE>(weights, (size_t)rowc * B + b, u);
            i32x4 A[8];
#pragma unroll
            for (int st = 0; st < 8; ++st) A[st] = *reinterpret_cast<const i32x4 *>(arow + b * 256 + 32 * st);
            float as[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) as[e] = scales[(size_t)etok[e] * B + b];
            UnitScales<TYPE> s;
            unit_scales<TYPE>(u, s);
            gemm_tile_terms<TYPE>(
                u, s, hm, grid, [&](int st) { return A[st]; }, [&](int e) { return as[e]; },
                [&](int e, float term) { terms[buf][wave][e][lane] = term; });
        }
        __syncthreads();
        /* this round's blocks r W .. r W + W - 1 in order (those that exist) */
        const int nw = min(W, B - r * W);
#pragma unroll
        for (int k = 0; k < kOwn; ++k) {
            const int idx = tid + kThreads * k;
            for (int w = 0; w < nw; ++w) total[k] = total[k] + terms[buf][w][idx >> 6][idx & 63];
        }
    }
#pragma unroll
    for (int k = 0; k < kOwn; ++k) {
        const int idx = tid + kThreads * k, e = idx >> 6, l = idx & 63;
        const int tok = t0 + 8 * (e >> 2) + 4 * (l >> 5) + (e & 3), row = row0 + (l & 31);
        if (tok < T && row < rows) out[(size_t)tok * rows + row] = total[k];
    }
}

}  // namespace

/* IQ4_NL prompts on the int8 matrix unit (tensor_gemm_q8_k's IQ4_NL rows,
 * dot_iq4_nl_q8_k, iq.rs:355-377): 128 rows x 64 tokens per workgroup as in
 * gemm_q8k.  Per block and 32-token tile each 32-value group is one product
 * of the code book's int8 values with the activations, read out at once
 * into its f32 term (the group's f16 scale times the activation scale,
 * times the integer sum), added in group order.  Weights and activations
 * are loaded block by block without prefetch: at 144 registers several
 * workgroups share a CU and cover each other's loads. */
extern "C" __global__ __launch_bounds__(256) void q38_gemm_q8k_iq4nl(q38_gemv_args a) {
    __shared__ __align__(16) int8_t act[kGemmTokens][kActRow];
    __shared__ float ascale[kGemmTokens];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;
    const int width = a.width;
    const int B = width / Q38_Q8K_BLOCK;
    const int rows = a.rows[0];
    const int row = blockIdx.x * kGemmRows + wave * 32 + (lane & 31);
    const int rowc = min(row, rows - 1);
    const int t0 = blockIdx.y * kGemmTokens;
    const int T = a.n_tokens;
    const int8_t *quants = static_cast<const int8_t *>(a.q8k);
    const int16_t *sums = reinterpret_cast<const int16_t *>(quants + (size_t)T * width);
    const float *scales = reinterpret_cast<const float *>(sums + (size_t)T * B * 16);
    float total[kGemmTiles][16];
#pragma unroll
    for (int tt = 0; tt < kGemmTiles; ++tt)
#pragma unroll
        for (int e = 0; e < 16; ++e) total[tt][e] = 0.0f;
    for (int b = 0; b < B; ++b) {
        Unit<Q38_GGML_IQ4_NL> u;
        load_unit<Q38_GGML_IQ4_NL>(a.weights[0], (size_t)rowc * B + b, u);
#pragma unroll
        for (int i = 0; i < kStagePieces; ++i) {
            const int p = tid + 256 * i, t = min(t0 + (p >> 4), T - 1), c = p & 15;
            *reinterpret_cast<u32x4 *>(&act[p >> 4][c * 16]) =
                *reinterpret_cast<const u32x4 *>(quants + (size_t)t * width + b * 256 + c * 16);
        }
        if (tid < kGemmTokens) ascale[tid] = scales[(size_t)min(t0 + tid, T - 1) * B + b];
        __syncthreads();
        float gd[8];
#pragma unroll
        for (int g = 0; g < 8; ++g) gd[g] = q38_f16(whalf(u.w, 18 * g));
#pragma unroll
        for (int tt = 0; tt < kGemmTiles; ++tt) {
            const int8_t *arow = &act[32 * tt + (lane & 31)][16 * h];
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                i32x4 bq;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t w = wword(u.w, 18 * g + 2 + 4 * j);
                    bq[j] = (int)q38_iq4_lookup((h ? w >> 4 : w) & 0x0F0F0F0Fu);
                }
                const i32x16 acc = mfma_i8(*reinterpret_cast<const i32x4 *>(arow + 32 * g), bq, i32x16{});
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const float as = ascale[32 * tt + 8 * (e >> 2) + 4 * h + (e & 3)];
                    total[tt][e] = total[tt][e] + (gd[g] * as) * (float)acc[e];
                }
            }
        }
        __syncthreads();
    }
    if (row < rows) {
#pragma unroll
        for (int tt = 0; tt < kGemmTiles; ++tt)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int tok = t0 + 32 * tt + 8 * (e >> 2) + 4 * h + (e & 3);
                if (tok < T) a.out[0][(size_t)tok * rows + row] = total[tt][e];
            }
    }
}

extern "C" __global__ __launch_bounds__(256) void q38_quantize_q8k(q38_quantize_args a) {
    /* block 16 x + t / 16 of token y by the 16 threads 16 (t / 16) .. + 15,
     * thread g holding values 16 g .. 16 g + 15 (q8k_quantize_group16) */
    const int b = blockIdx.x * 16 + (threadIdx.x >> 4);
    const int g = threadIdx.x & 15;
    const int tok = blockIdx.y;
    const int width = a.width;
    const int blocks = width / Q38_Q8K_BLOCK;
    const int bc = min(b, blocks - 1); /* rows past the last block work on it and store nothing */
    int8_t *quants = static_cast<int8_t *>(a.q8k);
    int16_t *sums = reinterpret_cast<int16_t *>(quants + (size_t)a.n_tokens * width);
    float *scales = reinterpret_cast<float *>(sums + (size_t)a.n_tokens * blocks * 16);
    const size_t k = (size_t)tok * blocks + bc;
    const float *x = a.x + (size_t)tok * width + (size_t)bc * Q38_Q8K_BLOCK + 16 * g;
    f32x4 v[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) v[c] = q38_ld4(x + 4 * c);
    uint32_t qw[4];
    int gsum;
    float scale;
    q8k_quantize_group16(v, g, qw, gsum, scale);
    if (b >= blocks) return;
    *reinterpret_cast<u32x4 *>(quants + k * Q38_Q8K_BLOCK + 16 * g) = u32x4{qw[0], qw[1], qw[2], qw[3]};
    sums[k * 16 + g] = (int16_t)gsum;
    if (g == 0) scales[k] = scale;
}

extern "C" __global__ __launch_bounds__(256) void q38_gemv_q8k_q4k(q38_gemv_args a) { gemv_q8k<Q38_GGML_Q4_K>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemv_q8k_q5k(q38_gemv_args a) { gemv_q8k<Q38_GGML_Q5_K>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemv_q8k_q6k(q38_gemv_args a) { gemv_q8k<Q38_GGML_Q6_K>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemv_q8k_q3k(q38_gemv_args a) { gemv_q8k<Q38_GGML_Q3_K>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemv_q8k_q2k(q38_gemv_args a) { gemv_q8k<Q38_GGML_Q2_K>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemv_q8k_iq4nl(q38_gemv_args a) {
    gemv_q8k<Q38_GGML_IQ4_NL>(a);
}
extern "C" __global__ __launch_bounds__(256) void q38_gemv_q8k_iq2xxs(q38_gemv_args a) {
    gemv_q8k<Q38_GGML_IQ2_XXS>(a);
}
extern "C" __global__ __launch_bounds__(256) void q38_gemv_q8k_iq2xs(q38_gemv_args a) { gemv_q8k<Q38_GGML_IQ2_XS>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemv_q8k_iq2s(q38_gemv_args a) { gemv_q8k<Q38_GGML_IQ2_S>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemv_q8k_iq3xxs(q38_gemv_args a) {
    gemv_q8k<Q38_GGML_IQ3_XXS>(a);
}
extern "C" __global__ __launch_bounds__(256) void q38_gemv_q8k_iq3s(q38_gemv_args a) { gemv_q8k<Q38_GGML_IQ3_S>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemv_q8k_iq1s(q38_gemv_args a) { gemv_q8k<Q38_GGML_IQ1_S>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemv_q8k_iq1m(q38_gemv_args a) { gemv_q8k<Q38_GGML_IQ1_M>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemv_q8k_iq4xs(q38_gemv_args a) {
    gemv_q8k<Q38_GGML_IQ4_XS>(a);
}
/* Q6_K, IQ4_XS, IQ2_XS, IQ2_S and IQ3_XXS are held to 168 registers (three
 * workgroups per CU; a few dwords spill): 4096-token prompts through
 * 17408 x 5120 ran 3-10% faster than at 169-178 registers and two.  Q5_K
 * is held to 256 (two workgroups; 4 dwords spill): left free it takes 259
 * and one, 2.20 against 1.83 ms. */
extern "C" __global__ __launch_bounds__(256) void q38_gemm_q8k_q4k(q38_gemv_args a) { gemm_q8k<Q38_GGML_Q4_K>(a); }
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void q38_gemm_q8k_q5k(q38_gemv_args a) {
    gemm_q8k<Q38_GGML_Q5_K>(a);
}
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void q38_gemm_q8k_q6k(q38_gemv_args a) { gemm_q8k<Q38_GGML_Q6_K>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemm_q8k_q2k(q38_gemv_args a) { gemm_q8k<Q38_GGML_Q2_K>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemm_q8k_q3k(q38_gemv_args a) { gemm_q8k<Q38_GGML_Q3_K>(a); }
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void q38_gemm_q8k_iq4xs(q38_gemv_args a) { gemm_q8k<Q38_GGML_IQ4_XS>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemm_q8k_iq2xxs(q38_gemv_args a) {
    gemm_q8k<Q38_GGML_IQ2_XXS>(a);
}
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void q38_gemm_q8k_iq2xs(q38_gemv_args a) { gemm_q8k<Q38_GGML_IQ2_XS>(a); }
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void q38_gemm_q8k_iq2s(q38_gemv_args a) {
    gemm_q8k<Q38_GGML_IQ2_S>(a);
}
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void q38_gemm_q8k_iq3xxs(q38_gemv_args a) {
    gemm_q8k<Q38_GGML_IQ3_XXS>(a);
}
extern "C" __global__ __launch_bounds__(256) void q38_gemm_q8k_iq3s(q38_gemv_args a) { gemm_q8k<Q38_GGML_IQ3_S>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemm_q8k_iq1s(q38_gemv_args a) { gemm_q8k<Q38_GGML_IQ1_S>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemm_q8k_iq1m(q38_gemv_args a) { gemm_q8k<Q38_GGML_IQ1_M>(a); }
#define Q38_GEMM_KS(name, T)                                                                                      \
    extern "C" __global__ __launch_bounds__(64 * Q38_GEMM_KS_WAVES) void q38_gemm_ks_q8k_##name(q38_gemv_args a) { \
        gemm_ks_q8k<T, Q38_GEMM_KS_WAVES>(a);                                                                     \
    }                                                                                                             \
    extern "C" __global__ __launch_bounds__(64 * Q38_GEMM_KS_WAVES_WIDE) void q38_gemm_ks16_q8k_##name(          \
        q38_gemv_args a) {                                                                                        \
        gemm_ks_q8k<T, Q38_GEMM_KS_WAVES_WIDE>(a);                                                                \
    }                                                                                                             \
    extern "C" __global__ __launch_bounds__(64 * Q38_GEMM_KS_WAVES_NARROW) void q38_gemm_ks4_q8k_##name(         \
        q38_gemv_args a) {                                                                                        \
        gemm_ks_q8k<T, Q38_GEMM_KS_WAVES_NARROW>(a);                                                              \
    }
Q38_GEMM_KS(q4k, Q38_GGML_Q4_K)
Q38_GEMM_KS(q5k, Q38_GGML_Q5_K)
Q38_GEMM_KS(q6k, Q38_GGML_Q6_K)
Q38_GEMM_KS(q2k, Q38_GGML_Q2_K)
Q38_GEMM_KS(q3k, Q38_GGML_Q3_K)
Q38_GEMM_KS(iq4xs, Q38_GGML_IQ4_XS)
Q38_GEMM_KS(iq2xxs, Q38_GGML_IQ2_XXS)
Q38_GEMM_KS(iq2xs, Q38_GGML_IQ2_XS)
Q38_GEMM_KS(iq2s, Q38_GGML_IQ2_S)
Q38_GEMM_KS(iq3xxs, Q38_GGML_IQ3_XXS)
Q38_GEMM_KS(iq3s, Q38_GGML_IQ3_S)
Q38_GEMM_KS(iq1s, Q38_GGML_IQ1_S)
Q38_GEMM_KS(iq1m, Q38_GGML_IQ1_M)
#undef Q38_GEMM_KS

/*
 * Projections of f32 activations by F32, F16 or BF16 weights (the path
 * project() takes for weights it does not quantise for, ops.rs:632-637:
 * tensor_gemv_f32 / tensor_gemm_f32, tensor.rs:1095-1129, :1175-1215; Q8_0
 * weights below) below 16 tokens.  grid (ceil(rows / 4), ceil(T / 8)), 256
 * threads: one wave per weight row, the row read once per pass of up to 8
 * tokens.  A lane takes units of 8 consecutive weights, units lane, lane +
 * 64, ... of the row, decodes them to f32 exactly (f16 and bf16 widen
 * exactly) and adds w * x into its partial sum with fused multiply-adds,
 * unit after unit;
 * the 64 partial sums are then added by a butterfly.  Every product is the
 * reference's; the order of the additions is not (the reference runs one
 * chain over the row on its scalar path and 8-lane partial sums on x86), so
 * results agree within the rounding of a reassociated f32 sum.
 */
template <int TYPE> struct F32Unit;
template <> struct F32Unit<Q38_GGML_F32> { static constexpr int E = 8, bytes = 32; };
template <> struct F32Unit<Q38_GGML_F16> { static constexpr int E = 8, bytes = 16; };
template <> struct F32Unit<Q38_GGML_BF16> { static constexpr int E = 8, bytes = 16; };

/* Unit u of a row starting at `row` (16-byte aligned): its E weights. */
template <int TYPE>
Q38_DEV void f32_unit(const uint8_t *row, int u, float (&w)[F32Unit<TYPE>::E]) {
    if (TYPE == Q38_GGML_F32) {
        u32x4 v0, v1;
        __builtin_memcpy(&v0, row + (size_t)u * 32, 16);
        __builtin_memcpy(&v1, row + (size_t)u * 32 + 16, 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w[i] = __uint_as_float(v0[i]);
            w[4 + i] = __uint_as_float(v1[i]);
        }
    } else {
        u32x4 v;
        __builtin_memcpy(&v, row + (size_t)u * 16, 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (TYPE == Q38_GGML_F16) {
                w[2 * i] = q38_f16(v[i]);
                w[2 * i + 1] = q38_f16(v[i] >> 16);
            } else {
                w[2 * i] = __uint_as_float(v[i] << 16);
                w[2 * i + 1] = __uint_as_float(v[i] & 0xFFFF0000u);
            }
        }
    }
}

template <int TYPE>
Q38_DEV void gemv_f32(const q38_gemv_f32_args &a) {
    constexpr int E = F32Unit<TYPE>::E;
    constexpr int TP = Q38_GEMV_TOKENS;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.rows) return; /* whole waves only: no barrier follows */
    const int tok0 = blockIdx.y * TP;
    const int tp = min(TP, a.n_tokens - tok0);
    const int units = a.width / E;
    const uint8_t *wrow = a.weights + (size_t)row * a.row_bytes;
    float acc[TP];
#pragma unroll
    for (int t = 0; t < TP; ++t) acc[t] = 0.0f;
    for (int u = lane; u < units; u += 64) {
        float w[E];
        f32_unit<TYPE>(wrow, u, w);
#pragma unroll
        for (int t = 0; t < TP; ++t) {
            if (t < tp) {
                const float *x = a.x + (size_t)(tok0 + t) * a.width + (size_t)u * E;
#pragma unroll
                for (int i4 = 0; i4 < E; i4 += 4) {
                    const f32x4 xv = q38_ld4(x + i4);
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc[t] = __builtin_fmaf(w[i4 + c], xv[c], acc[t]);
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < TP; ++t) {
        if (t < tp) {
            float v = acc[t];
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
            if (lane == 0) a.out[(size_t)(tok0 + t) * a.rows + row] = v;
        }
    }
}

extern "C" __global__ __launch_bounds__(256) void q38_gemv_f32_f32(q38_gemv_f32_args a) { gemv_f32<Q38_GGML_F32>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemv_f32_f16(q38_gemv_f32_args a) { gemv_f32<Q38_GGML_F16>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemv_f32_bf16(q38_gemv_f32_args a) { gemv_f32<Q38_GGML_BF16>(a); }

/*
 * The same projections for many tokens on the bf16 matrix unit
 * (v_mfma_f32_32x32x16_bf16, f32 accumulation), exact products:
 *  - every activation x splits by truncation into three bf16 parts,
 *    x = x1 + x2 + x3 exactly (each part takes the next 8 of f32's 24
 *    significant bits; the differences are exact in f32);
 *  - BF16 weights are one part; F16 weights two (w = w1 + w2 exactly, 8 + 3
 *    bits); F32 weights three, like x; Q8_0 weights are their int8 quants,
 *    exact in bf16, the block's f16 scale d applied to the block's sum
 *    (d * q is exact in f32, so d * sum(q x) is the reference's sum of
 *    (d q) x up to the order of the additions);
 *  - a product of two parts is exact in f32 (8 x 8 bits), and the parts'
 *    products below 2^-21 of w x are left out (F16: w2 x3; F32: w2 x3,
 *    w3 x2, w3 x3), so each output is the exact sum up to f32 rounding of
 *    the additions, as for the GEMV above (the reference's own x86 build
 *    reassociates these sums too).
 * Tile: 128 weight rows x 32 TT tokens per workgroup of 4 waves (TT 2 or
 * 4): with TT = 2 wave w computes rows 64 (w & 1) .. +63 of tokens 32 (w >>
 * 1) .. +31, with TT = 4 all 128 rows of tokens 32 w .. +31 (TT 32 x 32
 * accumulators; C column = weight row, so a token's 32 outputs are one
 * 128-byte store; the wider tile reads each activation part from LDS for
 * 4 row tiles instead of 2 and converts each weight for 128 tokens).  The k loop runs in stages of 64: each thread loads 16
 * activations of one token and 32 weights of one row (Q8_0: one block),
 * splits them into bf16 parts in LDS in the operands' lane layout, and the
 * next stage's loads go out before the matrix steps of this one.  Within a
 * 32-k slice, lane half h of substep s takes k 16h + 8s .. +7 for A and B
 * alike.  Tokens past T read the last token and rows past the matrix its
 * last row; neither is stored.  grid (ceil(rows / 128), ceil(T / (32 TT))),
 * 256 threads; width a multiple of 64.
 */
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int TYPE> struct F32wParts { static constexpr int n = 1; };
template <> struct F32wParts<Q38_GGML_F16> { static constexpr int n = 2; };
template <> struct F32wParts<Q38_GGML_F32> { static constexpr int n = 3; };

/* bf16 bits of the upper halves of two f32 bit patterns: a low, b high */
Q38_DEV uint32_t pack_hi16(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

/* eight f32 values into bf16 parts by truncation: v = p0 + p1 (+ p2) */
template <int NP>
Q38_DEV void split_parts(const float (&v)[8], u32x4 (&p)[NP]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float r0 = v[2 * i], r1 = v[2 * i + 1];
#pragma unroll
        for (int k = 0; k < NP; ++k) {
            const uint32_t u0 = __float_as_uint(r0), u1 = __float_as_uint(r1);
            p[k][i] = pack_hi16(u0, u1);
            if (k + 1 < NP) {
                r0 -= __uint_as_float(u0 & 0xFFFF0000u);
                r1 -= __uint_as_float(u1 & 0xFFFF0000u);
            }
        }
    }
}

Q38_DEV f32x16 mfma_bf16(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
}

/* c + the products of x's parts with w's parts above 2^-21 of w x, the
 * smallest first: x1 w1, x2 w1, x3 w1 (+ x1 w2, x2 w2; + x1 w3) */
template <int PW>
Q38_DEV f32x16 f32w_products(const u32x4 (&ax)[3], const u32x4 (&bw)[PW], f32x16 c) {
    if constexpr (PW == 3) c = mfma_bf16(ax[0], bw[2], c);
    if constexpr (PW >= 2) c = mfma_bf16(ax[1], bw[1], c);
    c = mfma_bf16(ax[2], bw[0], c);
    if constexpr (PW >= 2) c = mfma_bf16(ax[0], bw[1], c);
    c = mfma_bf16(ax[1], bw[0], c);
    return mfma_bf16(ax[0], bw[0], c);
}

/* raw weights of one row's 32-k slice (Q8_0: one 34-byte block) */
template <int TYPE> struct F32wRaw { u32x4 v[TYPE == Q38_GGML_F32 ? 8 : 4]; uint32_t tail[2]; };

template <int TYPE>
Q38_DEV void f32w_load(const uint8_t *row, int slice, F32wRaw<TYPE> &r) {
    if constexpr (TYPE == Q38_GGML_Q8_0) {
        /* the block starts 2-byte aligned: 8 dwords from the dword boundary
         * at or below it and the halfwords at 30 and 32 (as f32_unit) */
        const size_t s = (size_t)slice * 34;
        const uint32_t o = (uint32_t)((uintptr_t)(row + s) & 3);
        const u32x4 *base = reinterpret_cast<const u32x4 *>(row + (s - o));
        __builtin_memcpy(&r.v[0], base, 16);
        __builtin_memcpy(&r.v[1], reinterpret_cast<const uint8_t *>(base) + 16, 16);
        r.tail[0] = *reinterpret_cast<const uint16_t *>(row + s + 30);
        r.tail[1] = *reinterpret_cast<const uint16_t *>(row + s + 32);
    } else {
        constexpr int n = TYPE == Q38_GGML_F32 ? 8 : 4;
        const u32x4 *src = reinterpret_cast<const u32x4 *>(row + (size_t)slice * (16 * n));
#pragma unroll
        for (int i = 0; i < n; ++i) r.v[i] = src[i];
    }
}

constexpr int kF32wRows = Q38_GEMM_F32_ROWS, kF32wK = Q38_GEMM_F32_K;
static_assert(kF32wRows == 128 && kF32wK == 64, "the tile the lane mapping below assumes");

template <int TYPE, int TT>
Q38_DEV void gemm_f32w(const q38_gemv_f32_args &a) {
    constexpr int PW = F32wParts<TYPE>::n;
    constexpr int RPW = TT; /* row tiles per wave: 4 row tiles x TT token tiles over 4 waves */
    constexpr int XQ = TT / 2; /* 64-token groups a thread stages */
    /* operand units (16 bytes: 8 bf16 of one lane) in the lane layout */
    __shared__ __align__(16) u32x4 xs[3][TT][2][2][64]; /* [part][token tile][slice][substep][lane] */
    __shared__ __align__(16) u32x4 ws[PW][4][2][2][64]; /* [part][row tile][slice][substep][lane] */
    __shared__ float ds[2][kF32wRows];                   /* Q8_0: [slice][row] block scale */
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int rows = a.rows, W = a.width, T = a.n_tokens;
    const int row0 = blockIdx.x * kF32wRows;
    const int t0 = blockIdx.y * 32 * TT;
    /* this thread's loads: 16 activations of token xt (k 16 c .. +15 of a
     * stage), and slice wj of weight row wr */
    const int xl = tid >> 2, c = tid & 3;
    const float *xp[XQ];
#pragma unroll
    for (int q = 0; q < XQ; ++q) xp[q] = a.x + (size_t)min(t0 + xl + 64 * q, T - 1) * W + 16 * c;
    const int wl = tid >> 1, wj = tid & 1;
    const uint8_t *wrow = a.weights + (size_t)min(row0 + wl, rows - 1) * a.row_bytes;
    const int n_stages = W / kF32wK;

    f32x4 xr[XQ][4];
    F32wRaw<TYPE> wr;
    auto load = [&](int st) {
#pragma unroll
        for (int q = 0; q < XQ; ++q)
#pragma unroll
            for (int i = 0; i < 4; ++i) xr[q][i] = q38_ld4(xp[q] + (size_t)st * kF32wK + 4 * i);
        f32w_load<TYPE>(wrow, 2 * st + wj, wr);
    };

    f32x16 acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[r][e] = 0.0f;
    const int tt = TT == 4 ? wave : wave >> 1;
    const int rt0 = TT == 4 ? 0 : 2 * (wave & 1);

    load(0);
    for (int st = 0; st < n_stages; ++st) {
        /* activations: slice c >> 1, lane half c & 1, substeps 0 and 1 */
#pragma unroll
        for (int q = 0; q < XQ; ++q) {
            const int j = c >> 1, h = c & 1, ln = 32 * h + (xl & 31), xt = (xl >> 5) + 2 * q;
#pragma unroll
            for (int sb = 0; sb < 2; ++sb) {
                float v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = xr[q][2 * sb + (i >> 2)][i & 3];
                u32x4 p[3];
                split_parts<3>(v, p);
#pragma unroll
                for (int k = 0; k < 3; ++k) xs[k][xt][j][sb][ln] = p[k];
            }
        }
        /* weights: row wl, slice wj, lane halves 0 and 1, substeps 0 and 1 */
        {
            const int rt = wl >> 5, rl = wl & 31;
            if constexpr (TYPE == Q38_GGML_Q8_0) {
                uint32_t b[9];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    b[i] = wr.v[0][i];
                    b[4 + i] = wr.v[1][i];
                }
                const uint32_t o = (uint32_t)((uintptr_t)(wrow + (size_t)(2 * st + wj) * 34) & 3);
                uint32_t q[9];
#pragma unroll
                for (int i = 0; i < 7; ++i) q[i] = __builtin_amdgcn_alignbyte(b[i + 1], b[i], o);
                q[7] = __builtin_amdgcn_alignbyte(wr.tail[0], b[7], o);
                q[8] = wr.tail[1];
                /* q[0] bytes 0-1: the f16 scale; quant i is byte 2 + i */
                ds[wj][wl] = q38_f16(q[0]);
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int sb = 0; sb < 2; ++sb) {
                        u32x4 u;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int k0 = 16 * h + 8 * sb + 2 * i + 2; /* byte of the first quant */
                            const int k1 = k0 + 1;
                            const float f0 = (float)(int)(int8_t)(q[k0 >> 2] >> (8 * (k0 & 3)));
                            const float f1 = (float)(int)(int8_t)(q[k1 >> 2] >> (8 * (k1 & 3)));
                            u[i] = pack_hi16(__float_as_uint(f0), __float_as_uint(f1));
                        }
                        ws[0][rt][wj][sb][32 * h + rl] = u;
                    }
            } else {
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int sb = 0; sb < 2; ++sb) {
                        if constexpr (TYPE == Q38_GGML_BF16) {
                            ws[0][rt][wj][sb][32 * h + rl] = wr.v[2 * h + sb];
                        } else {
                            float v[8];
                            if constexpr (TYPE == Q38_GGML_F16) {
                                const u32x4 u = wr.v[2 * h + sb];
#pragma unroll
                                for (int i = 0; i < 4; ++i) {
                                    v[2 * i] = q38_f16(u[i]);
                                    v[2 * i + 1] = q38_f16(u[i] >> 16);
                                }
                            } else {
                                const u32x4 u0 = wr.v[4 * h + 2 * sb], u1 = wr.v[4 * h + 2 * sb + 1];
#pragma unroll
                                for (int i = 0; i < 4; ++i) {
                                    v[i] = __uint_as_float(u0[i]);
                                    v[4 + i] = __uint_as_float(u1[i]);
                                }
                            }
                            u32x4 p[PW];
                            split_parts<PW>(v, p);
#pragma unroll
                            for (int k = 0; k < PW; ++k) ws[k][rt][wj][sb][32 * h + rl] = p[k];
                        }
                    }
            }
        }
        __syncthreads();
        if (st + 1 < n_stages) load(st + 1);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            f32x16 blk[RPW];
            if constexpr (TYPE == Q38_GGML_Q8_0) {
#pragma unroll
                for (int r = 0; r < RPW; ++r)
#pragma unroll
                    for (int e = 0; e < 16; ++e) blk[r][e] = 0.0f;
            }
#pragma unroll
            for (int sb = 0; sb < 2; ++sb) {
                u32x4 ax[3];
#pragma unroll
                for (int k = 0; k < 3; ++k) ax[k] = xs[k][tt][j][sb][lane];
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    u32x4 bw[PW];
#pragma unroll
                    for (int k = 0; k < PW; ++k) bw[k] = ws[k][rt0 + r][j][sb][lane];
                    if constexpr (TYPE == Q38_GGML_Q8_0) blk[r] = f32w_products<PW>(ax, bw, blk[r]);
                    else acc[r] = f32w_products<PW>(ax, bw, acc[r]);
                }
            }
            if constexpr (TYPE == Q38_GGML_Q8_0) {
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    const float d = ds[j][32 * (rt0 + r) + (lane & 31)];
#pragma unroll
                    for (int e = 0; e < 16; ++e) acc[r][e] = __builtin_fmaf(d, blk[r][e], acc[r][e]);
                }
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = row0 + 32 * (rt0 + r) + (lane & 31);
        if (row >= rows) continue;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int tok = t0 + 32 * tt + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
            if (tok < T) a.out[(size_t)tok * rows + row] = acc[r][e];
        }
    }
}

static_assert(Q38_GEMM_F32_TOKENS == 64 && Q38_GEMM_F32_WIDE_TOKENS == 128, "2 and 4 token tiles per workgroup");
/* F32 weights only at 64 tokens: at 128 their three parts per weight take
 * 257 registers (one wave per SIMD) and measured no faster */
extern "C" __global__ __launch_bounds__(256) void q38_gemm_f32_f32(q38_gemv_f32_args a) { gemm_f32w<Q38_GGML_F32, 2>(a); }
#define Q38_GEMM_F32(name, T)                                                                              \
    extern "C" __global__ __launch_bounds__(256) void q38_gemm_f32_##name(q38_gemv_f32_args a) {          \
        gemm_f32w<T, 2>(a);                                                                               \
    }                                                                                                      \
    extern "C" __global__ __launch_bounds__(256) void q38_gemm_f32w_##name(q38_gemv_f32_args a) {         \
        gemm_f32w<T, 4>(a);                                                                               \
    }
Q38_GEMM_F32(f16, Q38_GGML_F16)
Q38_GEMM_F32(bf16, Q38_GGML_BF16)
Q38_GEMM_F32(q8_0, Q38_GGML_Q8_0)
#undef Q38_GEMM_F32

/*
 * The matrix-unit form for few tokens: a workgroup of 4 waves owns 64 rows x
 * 32 tokens (two 32 x 32 accumulators per wave) and the waves split the k
 * range into 4 contiguous parts of 32-value slices, so the grid has a
 * workgroup per 64 rows where the 128 x 64 tiles have one per 128 rows and
 * 64 tokens.  No LDS in the k loop: lane l loads the 16 activations of token
 * l % 32 and the 16 weights of rows l % 32 and 32 + l % 32 that its lane half
 * l / 32 supplies to the slice's two k substeps, splits them into bf16 parts
 * in registers (as the 128 x 64 form: exact parts, the same products), and
 * the next slice's loads go out before this slice's matrix steps.  The four
 * waves' accumulators are added through LDS in wave order, so the sums do
 * not depend on timing.  grid (ceil(rows / 64), ceil(T / 32)), 256 threads;
 * width a multiple of 64.
 */
template <int TYPE> struct F32sRaw { u32x4 v[TYPE == Q38_GGML_F32 ? 4 : 2]; };
template <> struct F32sRaw<Q38_GGML_Q8_0> { u32x4 v[1]; uint32_t tail, d; };

/* lane half h of slice `slice` of a row: its 16 weights (Q8_0: 16 quants of
 * block `slice` and the block's scale) */
template <int TYPE>
Q38_DEV void f32s_load(const uint8_t *row, int slice, int h, F32sRaw<TYPE> &r) {
    if constexpr (TYPE == Q38_GGML_Q8_0) {
        /* quants 16h .. 16h + 15 start 2-byte aligned: 16 bytes from the
         * dword boundary at or below them and the halfword at 14 */
        const uint8_t *p = row + (size_t)slice * 34 + 2 + 16 * h;
        const uint32_t o = (uint32_t)((uintptr_t)p & 3);
        __builtin_memcpy(&r.v[0], p - o, 16);
        r.tail = *reinterpret_cast<const uint16_t *>(p + 14);
        r.d = *reinterpret_cast<const uint16_t *>(row + (size_t)slice * 34);
    } else {
        constexpr int n = TYPE == Q38_GGML_F32 ? 4 : 2;
        const u32x4 *src = reinterpret_cast<const u32x4 *>(row + (size_t)slice * (32 * n) + 16 * n * h);
#pragma unroll
        for (int i = 0; i < n; ++i) r.v[i] = src[i];
    }
}

/* the weights of substep sb as PW bf16 parts */
template <int TYPE>
Q38_DEV void f32s_parts(const F32sRaw<TYPE> &r, int sb, const uint8_t *p, u32x4 (&out)[F32wParts<TYPE>::n]) {
    if constexpr (TYPE == Q38_GGML_BF16) {
        out[0] = r.v[sb];
    } else if constexpr (TYPE == Q38_GGML_Q8_0) {
        const uint32_t o = (uint32_t)((uintptr_t)p & 3);
        uint32_t q[4];
        q[0] = __builtin_amdgcn_alignbyte(r.v[0][1], r.v[0][0], o);
        q[1] = __builtin_amdgcn_alignbyte(r.v[0][2], r.v[0][1], o);
        q[2] = __builtin_amdgcn_alignbyte(r.v[0][3], r.v[0][2], o);
        q[3] = __builtin_amdgcn_alignbyte(r.tail, r.v[0][3], o);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t w = q[2 * sb + (i >> 1)];
            const int b0 = 2 * (i & 1);
            const float f0 = (float)(int)(int8_t)(w >> (8 * b0));
            const float f1 = (float)(int)(int8_t)(w >> (8 * b0 + 8));
            out[0][i] = pack_hi16(__float_as_uint(f0), __float_as_uint(f1));
        }
    } else {
        float v[8];
        if constexpr (TYPE == Q38_GGML_F16) {
            const u32x4 u = r.v[sb];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[2 * i] = q38_f16(u[i]);
                v[2 * i + 1] = q38_f16(u[i] >> 16);
            }
        } else {
            const u32x4 u0 = r.v[2 * sb], u1 = r.v[2 * sb + 1];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[i] = __uint_as_float(u0[i]);
                v[4 + i] = __uint_as_float(u1[i]);
            }
        }
        split_parts<F32wParts<TYPE>::n>(v, out);
    }
}

template <int TYPE>
Q38_DEV void gemm_f32s(const q38_gemv_f32_args &a) {
    constexpr int PW = F32wParts<TYPE>::n;
    __shared__ float red[3][2][16][64]; /* waves 1-3: [wave - 1][tile][element][lane] */
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int h = lane >> 5, l32 = lane & 31;
    const int rows = a.rows, W = a.width, T = a.n_tokens;
    const int row0 = blockIdx.x * 64;
    const int t0 = blockIdx.y * 32;
    const int n_slices = W / 32;
    const int s_begin = n_slices * wave / 4, s_end = n_slices * (wave + 1) / 4;
    const float *xp = a.x + (size_t)min(t0 + l32, T - 1) * W + 16 * h;
    const uint8_t *wp[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) wp[r] = a.weights + (size_t)min(row0 + 32 * r + l32, rows - 1) * a.row_bytes;

    f32x4 xc[4], xn[4];
    F32sRaw<TYPE> wc[2], wn[2];
    auto load = [&](int sl, f32x4(&xr)[4], F32sRaw<TYPE>(&wr)[2]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) xr[i] = q38_ld4(xp + (size_t)sl * 32 + 4 * i);
#pragma unroll
        for (int r = 0; r < 2; ++r) f32s_load<TYPE>(wp[r], sl, h, wr[r]);
    };
    f32x16 acc[2];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[r][e] = 0.0f;
    if (s_begin < s_end) load(s_begin, xc, wc);
    for (int sl = s_begin; sl < s_end; ++sl) {
        if (sl + 1 < s_end) load(sl + 1, xn, wn);
        f32x16 blk[2];
        if constexpr (TYPE == Q38_GGML_Q8_0) {
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int e = 0; e < 16; ++e) blk[r][e] = 0.0f;
        }
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = xc[2 * sb + (i >> 2)][i & 3];
            u32x4 ax[3];
            split_parts<3>(v, ax);
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                u32x4 bw[PW];
                f32s_parts<TYPE>(wc[r], sb, wp[r] + (size_t)sl * 34 + 2 + 16 * h, bw);
                if constexpr (TYPE == Q38_GGML_Q8_0) blk[r] = f32w_products<PW>(ax, bw, blk[r]);
                else acc[r] = f32w_products<PW>(ax, bw, acc[r]);
            }
        }
        if constexpr (TYPE == Q38_GGML_Q8_0) {
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                /* this lane's output column is its own row l % 32 of tile r */
                const float d = q38_f16(wc[r].d);
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[r][e] = __builtin_fmaf(d, blk[r][e], acc[r][e]);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) xc[i] = xn[i];
#pragma unroll
        for (int r = 0; r < 2; ++r) wc[r] = wn[r];
    }
    if (wave > 0) {
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int e = 0; e < 16; ++e) red[wave - 1][r][e][lane] = acc[r][e];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int row = row0 + 32 * r + l32;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float v = ((acc[r][e] + red[0][r][e][lane]) + red[1][r][e][lane]) + red[2][r][e][lane];
            const int tok = t0 + 8 * (e >> 2) + 4 * h + (e & 3);
            if (row < rows && tok < T) a.out[(size_t)tok * rows + row] = v;
        }
    }
}

extern "C" __global__ __launch_bounds__(256) void q38_gemm_f32s_f32(q38_gemv_f32_args a) { gemm_f32s<Q38_GGML_F32>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemm_f32s_f16(q38_gemv_f32_args a) { gemm_f32s<Q38_GGML_F16>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemm_f32s_bf16(q38_gemv_f32_args a) { gemm_f32s<Q38_GGML_BF16>(a); }
extern "C" __global__ __launch_bounds__(256) void q38_gemm_f32s_q8_0(q38_gemv_f32_args a) { gemm_f32s<Q38_GGML_Q8_0>(a); }

/*
 * Q8_0 weights below 16 tokens: a workgroup of 4 waves takes 4 RW rows (RW
 * per wave) and a pass of TP tokens, and walks the row in chunks of 32
 * blocks (1024 values).  Each chunk's activations are staged in LDS once
 * for all the workgroup's rows (a block at a 36-float stride, so 16 lanes
 * reading consecutive blocks with 16-byte reads touch 64 distinct banks);
 * lane l takes block l % 32 of the chunk in rows l / 32, l / 32 + 2, ...
 * of its wave: the 32 quants are converted to f32 and multiplied into the
 * staged activations (fused multiply-adds, the products exact), and the
 * block's f16 scale d is applied to that sum (d * q is exact in f32, so
 * this is the reference's sum of (d q) x up to the order of the additions).
 * The next chunk's weights and activations are loaded while this one is
 * computed; a row's 32 lanes add their sums at the end.  Tokens past T in
 * the last pass repeat token T - 1 and rows past the matrix its last row;
 * neither is stored.  grid (ceil(rows / (4 RW)), ceil(T / TP)), 256 threads.
 */
constexpr int kQ80Stride = 36; /* floats per staged block */

template <int RW, int TP>
Q38_DEV void gemv_q80s(const q38_gemv_f32_args &a) {
    constexpr int U = RW / 2; /* units per lane and chunk */
    __shared__ __align__(16) float xst[TP][32 * kQ80Stride];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int W = a.width, B = W / 32, T = a.n_tokens, rows = a.rows;
    const int tok0 = blockIdx.y * TP;
    const int n_chunks = (B + 31) / 32;
    /* staging: thread -> block sb of the chunk, values sk .. sk + 3 */
    const int sb = tid >> 3, sk = 4 * (tid & 7);
    const float *xsrc[TP];
#pragma unroll
    for (int t = 0; t < TP; ++t) xsrc[t] = a.x + (size_t)min(tok0 + t, T - 1) * W + 32 * sb + sk;
    /* units: block cb of the chunk in rows rw[j] */
    const int cb = lane & 31;
    const int r0 = blockIdx.x * 4 * RW + RW * wave + (lane >> 5);
    const uint8_t *wrow[U];
#pragma unroll
    for (int j = 0; j < U; ++j) wrow[j] = a.weights + (size_t)min(r0 + 2 * j, rows - 1) * a.row_bytes;

    f32x4 xr[TP];
    F32wRaw<Q38_GGML_Q8_0> wc[U], wn[U];
    auto load = [&](int ch, F32wRaw<Q38_GGML_Q8_0>(&w)[U]) {
        const bool xin = 32 * ch + sb < B;
#pragma unroll
        for (int t = 0; t < TP; ++t) xr[t] = xin ? q38_ld4(xsrc[t] + (size_t)ch * 1024) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (32 * ch + cb < B) {
#pragma unroll
            for (int j = 0; j < U; ++j) f32w_load<Q38_GGML_Q8_0>(wrow[j], 32 * ch + cb, w[j]);
        }
    };
    float acc[U][TP];
#pragma unroll
    for (int j = 0; j < U; ++j)
#pragma unroll
        for (int t = 0; t < TP; ++t) acc[j][t] = 0.0f;

    load(0, wc);
    for (int ch = 0; ch < n_chunks; ++ch) {
#pragma unroll
        for (int t = 0; t < TP; ++t) q38_st4(&xst[t][sb * kQ80Stride + sk], xr[t]);
        __syncthreads();
        if (ch + 1 < n_chunks) load(ch + 1, wn);
        const int blk = 32 * ch + cb;
        if (blk < B) {
#pragma unroll
            for (int j = 0; j < U; ++j) {
                uint32_t b[9];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    b[i] = wc[j].v[0][i];
                    b[4 + i] = wc[j].v[1][i];
                }
                const uint32_t o = (uint32_t)((uintptr_t)(wrow[j] + (size_t)blk * 34) & 3);
                uint32_t q[9];
#pragma unroll
                for (int i = 0; i < 7; ++i) q[i] = __builtin_amdgcn_alignbyte(b[i + 1], b[i], o);
                q[7] = __builtin_amdgcn_alignbyte(wc[j].tail[0], b[7], o);
                q[8] = wc[j].tail[1];
                float sum[TP];
#pragma unroll
                for (int t = 0; t < TP; ++t) sum[t] = 0.0f;
#pragma unroll
                for (int i4 = 0; i4 < 8; ++i4) {
                    float wq[4];
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const int byte = 2 + 4 * i4 + c;
                        wq[c] = (float)(int)(int8_t)(q[byte >> 2] >> (8 * (byte & 3)));
                    }
#pragma unroll
                    for (int t = 0; t < TP; ++t) {
                        const f32x4 xv = q38_ld4(&xst[t][cb * kQ80Stride + 4 * i4]);
#pragma unroll
                        for (int c = 0; c < 4; ++c) sum[t] = __builtin_fmaf(wq[c], xv[c], sum[t]);
                    }
                }
                const float d = q38_f16(q[0]);
#pragma unroll
                for (int t = 0; t < TP; ++t) acc[j][t] = __builtin_fmaf(d, sum[t], acc[j][t]);
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < U; ++j) wc[j] = wn[j];
    }
#pragma unroll
    for (int j = 0; j < U; ++j) {
#pragma unroll
        for (int t = 0; t < TP; ++t) {
            float v = acc[j][t];
#pragma unroll
            for (int m = 16; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
            const int row = r0 + 2 * j;
            if (cb == 0 && row < rows && tok0 + t < T) a.out[(size_t)(tok0 + t) * rows + row] = v;
        }
    }
}

#define Q38_GEMV_Q80S(rw, tp)                                                                           \
    extern "C" __global__ __launch_bounds__(256) void q38_gemv_f32_q8_0s_r##rw##_t##tp(q38_gemv_f32_args a) { \
        gemv_q80s<rw, tp>(a);                                                                             \
    }
/* the pairs the host launches: 2 rows a wave for 1-4 tokens a pass, 4 for 8 */
Q38_GEMV_Q80S(2, 1)
Q38_GEMV_Q80S(2, 2)
Q38_GEMV_Q80S(2, 4)
Q38_GEMV_Q80S(4, 8)
#undef Q38_GEMV_Q80S
