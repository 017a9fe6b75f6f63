/*
 * q38_quant_ref.c -- CPU restatement of the reference engine's weight
 * projection path: the Q8_K activation quantiser and the K-quant x Q8_K row
 * dots that tensor_gemv_q8_k / tensor_gemm_q8_k run for every row.
 *
 * TEST INFRASTRUCTURE ONLY (the oracle the HIP projection kernels are
 * compared against); nothing in the product library links or calls it.
 *
 * Follows, operation for operation and in the same order:
 *   f16_to_f32                    src/kernel/quant.rs:22-47
 *   nearest_int                   src/kernel/quant.rs:16-20
 *   quantize_block / quantize_q8_k src/kernel/quant.rs:55-128
 *   scale_min_k4                  src/kernel/tensor.rs:23-32
 *   dot_q4_k_q8_k_scalar          src/kernel/tensor.rs:365-391
 *   dot_q5_k_q8_k_scalar          src/kernel/tensor.rs:393-428
 *   dot_q6_k_q8_k_scalar          src/kernel/tensor.rs:430-457
 *   dot_q2_k_q8_k_scalar          src/kernel/tensor.rs:301-333
 *   unpack_q3_scales              src/kernel/tensor.rs:34-44
 *   dot_q3_k_q8_k_scalar          src/kernel/tensor.rs:335-363
 *   dot_iq4_nl_q8_k               src/kernel/iq.rs:355-377 (iq4_nl_group :96-99)
 *   dot_iq4_xs_q8_k               src/kernel/iq.rs:379-405 (KVALUES_IQ4NL,
 *                                 src/kernel/iq_tables.rs:53-56)
 *   dot_iq3_s_q8_k                src/kernel/iq.rs:407-446
 *   dot_iq3_xxs_q8_k              src/kernel/iq.rs:448-482
 *   dot_iq2_xxs_q8_k              src/kernel/iq.rs:484-512
 *   dot_iq2_xs_q8_k               src/kernel/iq.rs:514-547
 *   dot_iq2_s_q8_k                src/kernel/iq.rs:549-578
 *   dot_iq1_s_q8_k                src/kernel/iq.rs:580-612 (the repacked
 *                                 form, :733-762, does the same integer
 *                                 and f32 operations)
 *   dot_iq1_m_q8_k                src/kernel/iq.rs:614-667
 *                                 (grid32/grid64/sign_of :80-93; the grids
 *                                 are ggml's tables, q38_iq_grids.h;
 *                                 KSIGNS_IQ2XS[i] = i | parity(i) << 7 and
 *                                 KMASK_IQ2XS[j] = 1 << j are formed here)
 *   dot_f32/f16/bf16/q8_0_scalar  src/kernel/tensor.rs:79-117 (the row dots
 *                                 of tensor_gemv_f32 / tensor_gemm_f32,
 *                                 tensor.rs:1095-1129, :1175-1215, for the
 *                                 weights project() does not quantise
 *                                 for, ops.rs:632-637), bf16_to_f32
 *                                 src/kernel/quant.rs:49-51
 *   gemv_rows / gemm_rows         src/kernel/tensor.rs:954-1002 (every
 *                                 output element is one row dot, so the
 *                                 row split across threads does not change it)
 * Integer sums are exact; the f32 operations (the per-block d * weighted -
 * dmin * minimum and the running total over blocks) are kept separate and in
 * block order, as rustc compiles them (no contraction: -ffp-contract=off).
 *
 * Q8_K blocks are held planar here, as the device keeps them: for T tokens
 * of width W (B = W/256 blocks per token) quants int8 [T][W], group sums
 * int16 [T][B][16], scales f32 [T][B].
 */
#include "q38_ref.h"
#include "q38_iq_grids.h"

#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <string.h>

float q38r_f16_to_f32(uint16_t value) {
    const uint32_t sign = (uint32_t)(value & 0x8000) << 16;
    const uint32_t exponent = (value >> 10) & 0x1f;
    const uint32_t mantissa = value & 0x03ff;
    uint32_t bits;
    if (exponent == 0) {
        if (mantissa == 0) {
            bits = sign;
        } else {
            uint32_t normalized = mantissa;
            uint32_t shift = 0;
            while ((normalized & 0x400) == 0) {
                normalized <<= 1;
                shift += 1;
            }
            normalized &= 0x3ff;
            bits = sign | (127u - 14u - shift) << 23 | normalized << 13;
        }
    } else if (exponent == 31) {
        bits = sign | 0x7f800000u | mantissa << 13;
    } else {
        bits = sign | (exponent + 112u) << 23 | mantissa << 13;
    }
    float out;
    memcpy(&out, &bits, sizeof(out));
    return out;
}

static int32_t nearest_int(float value) {
#if Q38R_MUTANT == 13
    return (int32_t)value; /* planted: truncation */
#endif
    const float shifted = value + 12582912.0f;
    uint32_t bits;
    memcpy(&bits, &shifted, sizeof(bits));
    return (int32_t)(bits & 0x007fffff) - 0x00400000;
}

void q38r_quantize_block(const float *values, float *scale, int8_t *quants, int16_t *sums) {
    float maximum = 0.0f;
    float absolute_maximum = 0.0f;
    for (int i = 0; i < Q38R_Q8K_BLOCK; ++i) {
        const float absolute = fabsf(values[i]);
#if Q38R_MUTANT == 14
        if (absolute >= absolute_maximum) { /* planted: the last maximum wins */
#else
        if (absolute > absolute_maximum) {
#endif
            absolute_maximum = absolute;
            maximum = values[i];
        }
    }
    if (absolute_maximum == 0.0f) {
        *scale = 0.0f;
        memset(quants, 0, Q38R_Q8K_BLOCK);
        memset(sums, 0, sizeof(int16_t) * Q38R_Q8K_BLOCK / 16);
        return;
    }
    const float inverse_scale = -127.0f / maximum;
    for (int i = 0; i < Q38R_Q8K_BLOCK; ++i) {
        int32_t quant = nearest_int(inverse_scale * values[i]);
        if (quant > 127) quant = 127;
        quants[i] = (int8_t)quant;
    }
    for (int group = 0; group < Q38R_Q8K_BLOCK / 16; ++group) {
        int32_t sum = 0;
#if Q38R_MUTANT == 18
        for (int i = 0; i < 16; ++i) sum += quants[group * 8 + i]; /* planted: wrong groups */
#else
        for (int i = 0; i < 16; ++i) sum += quants[group * 16 + i];
#endif
        sums[group] = (int16_t)sum;
    }
    *scale = 1.0f / inverse_scale;
}

int q38r_quantize_q8_k(const float *input, int n_tokens, int width, void *planar) {
    if (width % Q38R_Q8K_BLOCK != 0 || n_tokens < 0) return -1;
    const int blocks = width / Q38R_Q8K_BLOCK;
    int8_t *quants = (int8_t *)planar;
    int16_t *sums = (int16_t *)(quants + (size_t)n_tokens * width);
    float *scales = (float *)(sums + (size_t)n_tokens * blocks * 16);
    for (int t = 0; t < n_tokens; ++t)
        for (int b = 0; b < blocks; ++b) {
            const size_t k = (size_t)t * blocks + b;
            q38r_quantize_block(input + (size_t)t * width + (size_t)b * Q38R_Q8K_BLOCK, &scales[k],
                                quants + k * Q38R_Q8K_BLOCK, sums + k * 16);
        }
    return 0;
}

static uint16_t read_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* scale_min_k4, tensor.rs:23-32 */
static void scale_min_k4(int index, const uint8_t *packed, uint8_t *scale, uint8_t *min) {
    if (index < 4) {
        *scale = packed[index] & 63;
        *min = packed[index + 4] & 63;
    } else {
#if Q38R_MUTANT == 15
        *scale = (packed[index + 4] & 15) | ((packed[index] >> 6) << 4); /* planted: wrong high bits */
        *min = (packed[index + 4] >> 4) | ((packed[index - 4] >> 6) << 4);
#else
        *scale = (packed[index + 4] & 15) | ((packed[index - 4] >> 6) << 4);
        *min = (packed[index + 4] >> 4) | ((packed[index] >> 6) << 4);
#endif
    }
}

/* One Q8_K block's view: scale, 256 quants, 16 group sums. */
typedef struct {
    float scale;
    const int8_t *quants;
    const int16_t *sums;
} q8k_view;

static float dot_q4_k(const uint8_t *data, const q8k_view *q, int blocks) {
    float total = 0.0f;
    for (int block = 0; block < blocks; ++block) {
        const q8k_view *b = &q[block];
        const uint8_t *blk = data + (size_t)block * 144;
        const float d = q38r_f16_to_f32(read_u16(blk)) * b->scale;
        const float dmin = q38r_f16_to_f32(read_u16(blk + 2)) * b->scale;
        const uint8_t *scales = blk + 4;
        const uint8_t *quants = blk + 16;
        int32_t weighted = 0, minimum = 0;
        for (int chunk = 0; chunk < 4; ++chunk) {
            uint8_t scale0, min0, scale1, min1;
            scale_min_k4(chunk * 2, scales, &scale0, &min0);
            scale_min_k4(chunk * 2 + 1, scales, &scale1, &min1);
            int32_t dot0 = 0, dot1 = 0;
            for (int i = 0; i < 32; ++i) {
                dot0 += (int32_t)(quants[chunk * 32 + i] & 15) * b->quants[chunk * 64 + i];
                dot1 += (int32_t)(quants[chunk * 32 + i] >> 4) * b->quants[chunk * 64 + 32 + i];
            }
            weighted += (int32_t)scale0 * dot0 + (int32_t)scale1 * dot1;
            minimum += (int32_t)min0 * (int32_t)(b->sums[chunk * 4] + b->sums[chunk * 4 + 1]);
            minimum += (int32_t)min1 * (int32_t)(b->sums[chunk * 4 + 2] + b->sums[chunk * 4 + 3]);
        }
        total += d * (float)weighted - dmin * (float)minimum;
    }
    return total;
}

static float dot_q5_k(const uint8_t *data, const q8k_view *q, int blocks) {
    float total = 0.0f;
    for (int block = 0; block < blocks; ++block) {
        const q8k_view *b = &q[block];
        const uint8_t *blk = data + (size_t)block * 176;
        const float d = q38r_f16_to_f32(read_u16(blk)) * b->scale;
        const float dmin = q38r_f16_to_f32(read_u16(blk + 2)) * b->scale;
        const uint8_t *scales = blk + 4;
        const uint8_t *high = blk + 16;
        const uint8_t *low = blk + 48;
        int32_t minimum = 0, weighted = 0;
        uint8_t high0 = 1, high1 = 2;
        for (int chunk = 0; chunk < 4; ++chunk) {
            uint8_t scale0, min0, scale1, min1;
            scale_min_k4(chunk * 2, scales, &scale0, &min0);
            scale_min_k4(chunk * 2 + 1, scales, &scale1, &min1);
            int32_t dot0 = 0, dot1 = 0;
            for (int i = 0; i < 32; ++i) {
                const int32_t qv0 = (int32_t)(low[chunk * 32 + i] & 15) + ((high[i] & high0) ? 16 : 0);
                const int32_t qv1 = (int32_t)(low[chunk * 32 + i] >> 4) + ((high[i] & high1) ? 16 : 0);
                dot0 += qv0 * b->quants[chunk * 64 + i];
                dot1 += qv1 * b->quants[chunk * 64 + 32 + i];
            }
            weighted += (int32_t)scale0 * dot0 + (int32_t)scale1 * dot1;
            minimum += (int32_t)min0 * (int32_t)(b->sums[chunk * 4] + b->sums[chunk * 4 + 1]);
            minimum += (int32_t)min1 * (int32_t)(b->sums[chunk * 4 + 2] + b->sums[chunk * 4 + 3]);
#if Q38R_MUTANT != 17 /* planted: high bits not advanced per chunk */
            high0 = (uint8_t)(high0 << 2);
            high1 = (uint8_t)(high1 << 2);
#endif
        }
        total += d * (float)weighted - dmin * (float)minimum;
    }
    return total;
}

static float dot_q6_k(const uint8_t *data, const q8k_view *q, int blocks) {
    float total = 0.0f;
    for (int block = 0; block < blocks; ++block) {
        const q8k_view *b = &q[block];
        const uint8_t *blk = data + (size_t)block * 210;
        const float d = q38r_f16_to_f32(read_u16(blk + 208)) * b->scale;
        const uint8_t *scales = blk + 192;
        int32_t weighted = 0;
        for (int half = 0; half < 2; ++half) {
            for (int i = 0; i < 32; ++i) {
                const int si = half * 8 + i / 16;
                const int base = half * 128;
                const uint8_t low_i = blk[half * 64 + i];
                const uint8_t low_i2 = blk[half * 64 + i + 32];
                const uint8_t h = blk[128 + half * 32 + i];
                const int32_t q0 = (int32_t)((low_i & 15) | ((h & 3) << 4)) - 32;
                const int32_t q1 = (int32_t)((low_i2 & 15) | (((h >> 2) & 3) << 4)) - 32;
#if Q38R_MUTANT == 16
                const int32_t q2 = (int32_t)((low_i >> 4) | (((h >> 2) & 3) << 4)) - 32; /* planted */
#else
                const int32_t q2 = (int32_t)((low_i >> 4) | (((h >> 4) & 3) << 4)) - 32;
#endif
                const int32_t q3 = (int32_t)((low_i2 >> 4) | (((h >> 6) & 3) << 4)) - 32;
                weighted += (int32_t)(int8_t)scales[si] * q0 * b->quants[base + i];
                weighted += (int32_t)(int8_t)scales[si + 2] * q1 * b->quants[base + 32 + i];
                weighted += (int32_t)(int8_t)scales[si + 4] * q2 * b->quants[base + 64 + i];
                weighted += (int32_t)(int8_t)scales[si + 6] * q3 * b->quants[base + 96 + i];
            }
        }
        total += d * (float)weighted;
    }
    return total;
}

/* KVALUES_IQ4NL (src/kernel/iq_tables.rs:53-56): ggml's published 16-entry
 * code book of the IQ4_NL / IQ4_XS formats. */
static const int8_t kvalues_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                         1,    13,   25,  38,  53,  69,  89,  113};

/* dot_q2_k_q8_k_scalar, tensor.rs:301-333.  Block: scales[16] (low nibble
 * scale, high nibble minimum) | qs[64] | d | dmin (f16), 84 bytes. */
static float dot_q2_k(const uint8_t *data, const q8k_view *q, int blocks) {
    float total = 0.0f;
    for (int block = 0; block < blocks; ++block) {
        const q8k_view *b = &q[block];
        const uint8_t *blk = data + (size_t)block * 84;
        const uint8_t *scales = blk;
        const uint8_t *quants = blk + 16;
        const float d = q38r_f16_to_f32(read_u16(blk + 80)) * b->scale;
        const float dmin = q38r_f16_to_f32(read_u16(blk + 82)) * b->scale;
        int32_t weighted = 0, minimum = 0;
        for (int half = 0; half < 2; ++half) {
            for (int field = 0; field < 4; ++field) {
                const int scale_index = half * 8 + field * 2;
                const int32_t scale0 = scales[scale_index] & 15;
                const int32_t scale1 = scales[scale_index + 1] & 15;
                const int shift = field * 2;
                int32_t dot0 = 0, dot1 = 0;
                for (int lane = 0; lane < 16; ++lane) {
                    dot0 += (int32_t)((quants[half * 32 + lane] >> shift) & 3) *
                            b->quants[half * 128 + field * 32 + lane];
                    dot1 += (int32_t)((quants[half * 32 + 16 + lane] >> shift) & 3) *
                            b->quants[half * 128 + field * 32 + 16 + lane];
                }
                weighted += scale0 * dot0 + scale1 * dot1;
#if Q38R_MUTANT == 22
                minimum += (int32_t)(scales[scale_index] & 15) * b->sums[scale_index]; /* planted: wrong nibble */
#else
                minimum += (int32_t)(scales[scale_index] >> 4) * b->sums[scale_index];
#endif
                minimum += (int32_t)(scales[scale_index + 1] >> 4) * b->sums[scale_index + 1];
            }
        }
        total += d * (float)weighted - dmin * (float)minimum;
    }
    return total;
}

/* unpack_q3_scales, tensor.rs:34-44: 16 signed 6-bit scales from 12 bytes */
static void unpack_q3_scales(const uint8_t *packed, int8_t *scales) {
    for (int index = 0; index < 16; ++index) {
        const uint8_t low = index < 8 ? (uint8_t)(packed[index] & 15) : (uint8_t)(packed[index - 8] >> 4);
        const uint8_t high = (uint8_t)((packed[8 + index % 4] >> (2 * (index / 4))) & 3);
        scales[index] = (int8_t)((int32_t)(low | (high << 4)) - 32);
    }
}

/* dot_q3_k_q8_k_scalar, tensor.rs:335-363.  Block: hmask[32] | qs[64] |
 * scales[12] | d (f16), 110 bytes. */
static float dot_q3_k(const uint8_t *data, const q8k_view *q, int blocks) {
    float total = 0.0f;
    for (int block = 0; block < blocks; ++block) {
        const q8k_view *b = &q[block];
        const uint8_t *blk = data + (size_t)block * 110;
        const uint8_t *high = blk;
        const uint8_t *low = blk + 32;
        int8_t scales[16];
        unpack_q3_scales(blk + 96, scales);
        const float d = q38r_f16_to_f32(read_u16(blk + 108)) * b->scale;
        int32_t weighted = 0;
        int group = 0;
        for (int half = 0; half < 2; ++half) {
            for (int field = 0; field < 4; ++field) {
                const uint8_t high_bit = (uint8_t)(1u << group);
                const int32_t scale0 = scales[group * 2];
                const int32_t scale1 = scales[group * 2 + 1];
                for (int lane = 0; lane < 32; ++lane) {
#if Q38R_MUTANT == 19
                    const int32_t qv = (int32_t)((low[half * 32 + lane] >> (field * 2)) & 3) -
                                       ((high[lane] & high_bit) ? 4 : 0); /* planted: high-bit sense inverted */
#else
                    const int32_t qv = (int32_t)((low[half * 32 + lane] >> (field * 2)) & 3) -
                                       ((high[lane] & high_bit) ? 0 : 4);
#endif
                    const int32_t scale = lane < 16 ? scale0 : scale1;
                    weighted += scale * qv * b->quants[half * 128 + field * 32 + lane];
                }
                group += 1;
            }
        }
        total += d * (float)weighted;
    }
    return total;
}

/* dot_iq4_nl_q8_k, iq.rs:355-377: eight 18-byte GGUF blocks (f16 d, 16
 * bytes of nibbles) per 256 weights, each group's term added to the total
 * on its own. */
static float dot_iq4_nl(const uint8_t *data, const q8k_view *q, int blocks) {
    float total = 0.0f;
    for (int block = 0; block < blocks; ++block) {
        const q8k_view *b = &q[block];
        const uint8_t *w = data + (size_t)block * 144;
        for (int group = 0; group < 8; ++group) {
            const uint8_t *packed = w + group * 18;
            const float d = q38r_f16_to_f32(read_u16(packed)) * b->scale;
            int32_t weighted = 0;
            for (int lane = 0; lane < 16; ++lane) {
                const uint8_t p = packed[2 + lane];
#if Q38R_MUTANT == 23
                weighted += (int32_t)b->quants[group * 32 + lane] * kvalues_iq4nl[p >> 4]; /* planted: halves swapped */
                weighted += (int32_t)b->quants[group * 32 + lane + 16] * kvalues_iq4nl[p & 15];
#else
                weighted += (int32_t)b->quants[group * 32 + lane] * kvalues_iq4nl[p & 15];
                weighted += (int32_t)b->quants[group * 32 + lane + 16] * kvalues_iq4nl[p >> 4];
#endif
            }
            total += d * (float)weighted;
        }
    }
    return total;
}

/* dot_iq4_xs_q8_k, iq.rs:379-405.  Block: d (f16) | scales_h (u16) |
 * scales_l[4] | qs[128], 136 bytes. */
static float dot_iq4_xs(const uint8_t *data, const q8k_view *q, int blocks) {
    float total = 0.0f;
    for (int block = 0; block < blocks; ++block) {
        const q8k_view *b = &q[block];
        const uint8_t *w = data + (size_t)block * 136;
        const float d = q38r_f16_to_f32(read_u16(w)) * b->scale;
        const uint16_t scale_high = read_u16(w + 2);
        const uint8_t *scale_low = w + 4;
        const uint8_t *quants = w + 8;
        int32_t weighted = 0;
        for (int group = 0; group < 8; ++group) {
            const int32_t scale = (int32_t)((scale_low[group / 2] >> (4 * (group % 2))) & 15) |
                                  (int32_t)((scale_high >> (2 * group)) & 3) << 4;
            int32_t subtotal = 0;
            for (int lane = 0; lane < 16; ++lane) {
                const uint8_t packed = quants[group * 16 + lane];
                subtotal += (int32_t)b->quants[group * 32 + lane] * kvalues_iq4nl[packed & 15];
                subtotal += (int32_t)b->quants[group * 32 + lane + 16] * kvalues_iq4nl[packed >> 4];
            }
#if Q38R_MUTANT == 20
            weighted += scale * subtotal; /* planted: the 32 offset dropped */
#else
            weighted += (scale - 32) * subtotal;
#endif
        }
        total += d * (float)weighted;
    }
    return total;
}

/* ---- IQ formats: lattice-grid codes (iq.rs:407-667) ---- */
static const uint64_t iq2xxs_grid[256] = Q38_IQ2XXS_GRID;
static const uint64_t iq2xs_grid[512] = Q38_IQ2XS_GRID;
static const uint64_t iq2s_grid[1024] = Q38_IQ2S_GRID;
static const uint32_t iq3xxs_grid[256] = Q38_IQ3XXS_GRID;
static const uint32_t iq3s_grid[512] = Q38_IQ3S_GRID;
static const uint64_t iq1s_grid[2048] = Q38_IQ1S_GRID;
static const float iq1_delta = 0.125f; /* IQ1_DELTA, iq.rs:19 */

static uint32_t read_u32(const uint8_t *p) {
    return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}
/* KSIGNS_IQ2XS[i]: the 7 stored sign bits and an eighth that makes the count even */
static uint8_t ksigns(uint32_t i) { return (uint8_t)(i | (uint32_t)(__builtin_popcount(i) & 1) << 7); }
static int32_t sign_of(uint32_t mask, uint32_t bit) { return (mask & bit) ? -1 : 1; }
static int32_t grid64_byte(uint64_t entry, int lane) { return (int32_t)((entry >> (8 * lane)) & 255); }
static int32_t grid32_byte(uint32_t entry, int lane) { return (int32_t)((entry >> (8 * lane)) & 255); }

/* dot_iq3_s_q8_k, iq.rs:407-446.  Block: d (f16) | qs[64] | qh[8] |
 * signs[32] | scales[4], 110 bytes. */
static float dot_iq3_s(const uint8_t *data, const q8k_view *q, int blocks) {
    float total = 0.0f;
    for (int block = 0; block < blocks; ++block) {
        const q8k_view *b = &q[block];
        const uint8_t *w = data + (size_t)block * 110;
        const float d = q38r_f16_to_f32(read_u16(w)) * b->scale;
        const uint8_t *indices = w + 2, *high = w + 66, *signs = w + 74, *scales = w + 106;
        int32_t weighted = 0;
        for (int group = 0; group < 8; ++group) {
            const uint8_t *code = indices + group * 8;
            const uint32_t high_bits = high[group];
            const uint8_t *group_signs = signs + group * 4;
            const int32_t scale = 1 + 2 * (int32_t)((scales[group / 2] >> (4 * (group % 2))) & 15);
            int32_t subtotal = 0;
            for (int section = 0; section < 4; ++section) {
                const uint32_t index0 = code[section * 2] | ((high_bits << (8 - 2 * section)) & 0x100);
#if Q38R_MUTANT == 28
                const uint32_t index1 = code[section * 2 + 1] | ((high_bits << (8 - 2 * section)) & 0x100); /* planted */
#else
                const uint32_t index1 = code[section * 2 + 1] | ((high_bits << (7 - 2 * section)) & 0x100);
#endif
                const uint32_t g0 = iq3s_grid[index0], g1 = iq3s_grid[index1];
                for (int lane = 0; lane < 4; ++lane) {
                    const int32_t sign0 = sign_of(group_signs[section], 1u << lane);
                    const int32_t sign1 = sign_of(group_signs[section], 1u << (lane + 4));
                    subtotal += (int32_t)b->quants[group * 32 + section * 8 + lane] * grid32_byte(g0, lane) * sign0;
                    subtotal += (int32_t)b->quants[group * 32 + section * 8 + lane + 4] * grid32_byte(g1, lane) * sign1;
                }
            }
            weighted += scale * subtotal;
        }
        total += d * (float)weighted;
    }
    return total;
}

/* dot_iq3_xxs_q8_k, iq.rs:448-482.  Block: d (f16) | qs[64] | 8 u32 of
 * 4 x 7 sign bits and a 4-bit scale, 98 bytes. */
static float dot_iq3_xxs(const uint8_t *data, const q8k_view *q, int blocks) {
    float total = 0.0f;
    for (int block = 0; block < blocks; ++block) {
        const q8k_view *b = &q[block];
        const uint8_t *w = data + (size_t)block * 98;
#if Q38R_MUTANT == 27
        const float d = q38r_f16_to_f32(read_u16(w)) * b->scale; /* planted: the 1/4 dropped */
#else
        const float d = 0.25f * q38r_f16_to_f32(read_u16(w)) * b->scale;
#endif
        const uint8_t *indices = w + 2, *metadata = w + 66;
        int32_t weighted = 0;
        for (int group = 0; group < 8; ++group) {
            const uint32_t packed = read_u32(metadata + group * 4);
            const int32_t scale = 1 + 2 * (int32_t)(packed >> 28);
            const uint8_t *code = indices + group * 8;
            int32_t subtotal = 0;
            for (int section = 0; section < 4; ++section) {
                const uint32_t g0 = iq3xxs_grid[code[section * 2]], g1 = iq3xxs_grid[code[section * 2 + 1]];
                const uint8_t signs = ksigns((packed >> (7 * section)) & 127);
                for (int lane = 0; lane < 4; ++lane) {
                    const int32_t sign0 = sign_of(signs, 1u << lane);
                    const int32_t sign1 = sign_of(signs, 1u << (lane + 4));
                    subtotal += (int32_t)b->quants[group * 32 + section * 8 + lane] * grid32_byte(g0, lane) * sign0;
                    subtotal += (int32_t)b->quants[group * 32 + section * 8 + lane + 4] * grid32_byte(g1, lane) * sign1;
                }
            }
            weighted += scale * subtotal;
        }
        total += d * (float)weighted;
    }
    return total;
}

/* dot_iq2_xxs_q8_k, iq.rs:484-512.  Block: d (f16) | 8 groups of 4 grid
 * indices and a u32 of 4 x 7 sign bits and a 4-bit scale, 66 bytes. */
static float dot_iq2_xxs(const uint8_t *data, const q8k_view *q, int blocks) {
    float total = 0.0f;
    for (int block = 0; block < blocks; ++block) {
        const q8k_view *b = &q[block];
        const uint8_t *w = data + (size_t)block * 66;
        const float d = iq1_delta * q38r_f16_to_f32(read_u16(w)) * b->scale;
        const uint8_t *codes = w + 2;
        int32_t weighted = 0;
        for (int group = 0; group < 8; ++group) {
            const uint8_t *code = codes + group * 8;
            const uint32_t metadata = read_u32(code + 4);
#if Q38R_MUTANT == 24
            const int32_t scale = 1 + 2 * (int32_t)((metadata >> 24) & 15); /* planted: wrong nibble */
#else
            const int32_t scale = 1 + 2 * (int32_t)(metadata >> 28);
#endif
            int32_t subtotal = 0;
            for (int section = 0; section < 4; ++section) {
                const uint64_t grid = iq2xxs_grid[code[section]];
                const uint8_t signs = ksigns((metadata >> (7 * section)) & 127);
                for (int lane = 0; lane < 8; ++lane)
                    subtotal += (int32_t)b->quants[group * 32 + section * 8 + lane] * grid64_byte(grid, lane) *
                                sign_of(signs, 1u << lane);
            }
            weighted += scale * subtotal;
        }
        total += d * (float)weighted;
    }
    return total;
}

/* dot_iq2_xs_q8_k, iq.rs:514-547.  Block: d (f16) | 32 u16 codes (9-bit
 * grid index, 7 sign bits) | scales[8], 74 bytes. */
static float dot_iq2_xs(const uint8_t *data, const q8k_view *q, int blocks) {
    float total = 0.0f;
    for (int block = 0; block < blocks; ++block) {
        const q8k_view *b = &q[block];
        const uint8_t *w = data + (size_t)block * 74;
        const float d = iq1_delta * q38r_f16_to_f32(read_u16(w)) * b->scale;
        const uint8_t *codes = w + 2, *scales = w + 66;
        int32_t weighted = 0;
        for (int group = 0; group < 8; ++group) {
            uint16_t code[4];
            for (int section = 0; section < 4; ++section) code[section] = read_u16(codes + group * 8 + section * 2);
#if Q38R_MUTANT == 25
            const int32_t scale0 = 1 + 2 * (int32_t)(scales[group] >> 4); /* planted: nibbles swapped */
            const int32_t scale1 = 1 + 2 * (int32_t)(scales[group] & 15);
#else
            const int32_t scale0 = 1 + 2 * (int32_t)(scales[group] & 15);
            const int32_t scale1 = 1 + 2 * (int32_t)(scales[group] >> 4);
#endif
            int32_t subtotal[2] = {0, 0};
            for (int section = 0; section < 4; ++section) {
                const uint64_t grid = iq2xs_grid[code[section] & 511];
                const uint8_t signs = ksigns(code[section] >> 9);
                for (int lane = 0; lane < 8; ++lane)
                    subtotal[section / 2] += (int32_t)b->quants[group * 32 + section * 8 + lane] *
                                             grid64_byte(grid, lane) * sign_of(signs, 1u << lane);
            }
            weighted += scale0 * subtotal[0] + scale1 * subtotal[1];
        }
        total += d * (float)weighted;
    }
    return total;
}

/* dot_iq2_s_q8_k, iq.rs:549-578.  Block: d (f16) | qs[32] | signs[32] |
 * qh[8] | scales[8], 82 bytes. */
static float dot_iq2_s(const uint8_t *data, const q8k_view *q, int blocks) {
    float total = 0.0f;
    for (int block = 0; block < blocks; ++block) {
        const q8k_view *b = &q[block];
        const uint8_t *w = data + (size_t)block * 82;
        const float d = iq1_delta * q38r_f16_to_f32(read_u16(w)) * b->scale;
        const uint8_t *indices = w + 2, *signs = w + 34, *high = w + 66, *scales = w + 74;
        int32_t weighted = 0;
        for (int group = 0; group < 8; ++group) {
            const int32_t scale0 = 1 + 2 * (int32_t)(scales[group] & 15);
            const int32_t scale1 = 1 + 2 * (int32_t)(scales[group] >> 4);
            int32_t subtotal[2] = {0, 0};
            for (int lane = 0; lane < 32; ++lane) {
                const int section = lane / 8;
#if Q38R_MUTANT == 26
                const uint32_t index = indices[group * 4 + section] |
                                       (((uint32_t)high[group] << (2 + 2 * section)) & 0x300); /* planted */
#else
                const uint32_t index = indices[group * 4 + section] |
                                       (((uint32_t)high[group] << (8 - 2 * section)) & 0x300);
#endif
                const uint64_t grid = iq2s_grid[index];
                const int32_t sign = sign_of(signs[group * 4 + section], 1u << (lane % 8));
                subtotal[section / 2] += (int32_t)b->quants[group * 32 + lane] * grid64_byte(grid, lane % 8) * sign;
            }
            weighted += scale0 * subtotal[0] + scale1 * subtotal[1];
        }
        total += d * (float)weighted;
    }
    return total;
}

/* dot_iq1_s_q8_k, iq.rs:580-612.  Block: d (f16) | qs[32] | qh u16[8]
 * (3 index bits per section, a 3-bit scale, the delta's sign), 50 bytes;
 * grid bytes are signed (-1, 0, 1). */
static float dot_iq1_s(const uint8_t *data, const q8k_view *q, int blocks) {
    float total = 0.0f;
    for (int block = 0; block < blocks; ++block) {
        const q8k_view *b = &q[block];
        const uint8_t *w = data + (size_t)block * 50;
        const float d = q38r_f16_to_f32(read_u16(w)) * b->scale;
        const uint8_t *indices = w + 2, *high = w + 34;
        int32_t weighted = 0, correction = 0;
        for (int group = 0; group < 8; ++group) {
            const uint16_t packed = read_u16(high + group * 2);
            const int32_t scale = 1 + 2 * (int32_t)((packed >> 12) & 7);
#if Q38R_MUTANT == 29
            const int32_t delta = (packed & 0x8000) ? 1 : -1; /* planted: delta sign flipped */
#else
            const int32_t delta = (packed & 0x8000) ? -1 : 1;
#endif
            int32_t subtotal = 0;
            for (int section = 0; section < 4; ++section) {
                const uint32_t index = indices[group * 4 + section] | (uint32_t)((packed >> (3 * section)) & 7) << 8;
                const uint64_t grid = iq1s_grid[index];
                for (int lane = 0; lane < 8; ++lane)
                    subtotal += (int32_t)b->quants[group * 32 + section * 8 + lane] *
                                (int32_t)(int8_t)grid64_byte(grid, lane);
            }
            weighted += scale * subtotal;
            correction += scale * delta * ((int32_t)b->sums[group * 2] + (int32_t)b->sums[group * 2 + 1]);
        }
        total += d * ((float)weighted + iq1_delta * (float)correction);
    }
    return total;
}

/* dot_iq1_m_q8_k, iq.rs:614-667.  Block: qs[32] | qh[16] (3 index bits
 * and a delta sign per section) | scales u16[4] (3-bit scales; the f16 d
 * in their top nibbles), 56 bytes. */
static float dot_iq1_m(const uint8_t *data, const q8k_view *q, int blocks) {
    float total = 0.0f;
    for (int block = 0; block < blocks; ++block) {
        const q8k_view *b = &q[block];
        const uint8_t *w = data + (size_t)block * 56;
        const uint8_t *indices = w, *high = w + 32, *packed_scales = w + 48;
        const uint16_t scale_bits = (uint16_t)((read_u16(packed_scales) >> 12) |
                                               ((read_u16(packed_scales + 2) >> 8) & 0x00f0) |
                                               ((read_u16(packed_scales + 4) >> 4) & 0x0f00) |
                                               (read_u16(packed_scales + 6) & 0xf000));
        const float d = q38r_f16_to_f32(scale_bits) * b->scale;
        int32_t weighted = 0, correction = 0;
        for (int group = 0; group < 8; ++group) {
            int32_t dot[2] = {0, 0}, correction_dot[2] = {0, 0};
            for (int section = 0; section < 4; ++section) {
                const uint32_t group_high = high[group * 2 + section / 2];
                const uint32_t index = indices[group * 4 + section] | ((group_high << (8 - 4 * (section % 2))) & 0x700);
                const uint64_t grid = iq1s_grid[index];
#if Q38R_MUTANT == 30
                const uint32_t delta_bit = 0x08; /* planted: odd sections test the even sections' bit */
#else
                const uint32_t delta_bit = section % 2 == 1 ? 0x80 : 0x08;
#endif
                const int32_t delta = (group_high & delta_bit) ? -1 : 1;
                for (int lane = 0; lane < 8; ++lane) {
                    const int32_t a = b->quants[group * 32 + section * 8 + lane];
                    dot[section / 2] += a * (int32_t)(int8_t)grid64_byte(grid, lane);
                    correction_dot[section / 2] += a * delta;
                }
            }
            const uint16_t scales = read_u16(packed_scales + (group / 2) * 2);
            const int shift = 6 * (group % 2);
            const int32_t scale0 = 1 + 2 * (int32_t)((scales >> shift) & 7);
            const int32_t scale1 = 1 + 2 * (int32_t)((scales >> (shift + 3)) & 7);
            weighted += scale0 * dot[0] + scale1 * dot[1];
            correction += scale0 * correction_dot[0] + scale1 * correction_dot[1];
        }
        total += d * ((float)weighted + iq1_delta * (float)correction);
    }
    return total;
}

int q38r_quant_block_bytes(int ggml_type) {
    switch (ggml_type) {
    case Q38R_GGML_Q2_K: return 84;
    case Q38R_GGML_Q3_K: return 110;
    case Q38R_GGML_IQ4_NL: return 144;
    case Q38R_GGML_Q4_K: return 144;
    case Q38R_GGML_Q5_K: return 176;
    case Q38R_GGML_Q6_K: return 210;
    case Q38R_GGML_IQ4_XS: return 136;
    case Q38R_GGML_IQ2_XXS: return 66;
    case Q38R_GGML_IQ2_XS: return 74;
    case Q38R_GGML_IQ2_S: return 82;
    case Q38R_GGML_IQ3_XXS: return 98;
    case Q38R_GGML_IQ3_S: return 110;
    case Q38R_GGML_IQ1_S: return 50;
    case Q38R_GGML_IQ1_M: return 56;
    default: return 0;
    }
}

float q38r_dot_q8_k(int ggml_type, const uint8_t *row, const void *planar, int n_tokens, int width, int token) {
    const int blocks = width / Q38R_Q8K_BLOCK;
    const int8_t *quants = (const int8_t *)planar;
    const int16_t *sums = (const int16_t *)(quants + (size_t)n_tokens * width);
    const float *scales = (const float *)(sums + (size_t)n_tokens * blocks * 16);
    q8k_view view[256];
    if (blocks > 256) return NAN;
    for (int b = 0; b < blocks; ++b) {
        const size_t k = (size_t)token * blocks + b;
        view[b].scale = scales[k];
        view[b].quants = quants + k * Q38R_Q8K_BLOCK;
        view[b].sums = sums + k * 16;
    }
    switch (ggml_type) {
    case Q38R_GGML_Q4_K: return dot_q4_k(row, view, blocks);
    case Q38R_GGML_Q5_K: return dot_q5_k(row, view, blocks);
    case Q38R_GGML_Q6_K: return dot_q6_k(row, view, blocks);
    case Q38R_GGML_Q2_K: return dot_q2_k(row, view, blocks);
    case Q38R_GGML_Q3_K: return dot_q3_k(row, view, blocks);
    case Q38R_GGML_IQ4_NL: return dot_iq4_nl(row, view, blocks);
    case Q38R_GGML_IQ4_XS: return dot_iq4_xs(row, view, blocks);
    case Q38R_GGML_IQ2_XXS: return dot_iq2_xxs(row, view, blocks);
    case Q38R_GGML_IQ2_XS: return dot_iq2_xs(row, view, blocks);
    case Q38R_GGML_IQ2_S: return dot_iq2_s(row, view, blocks);
    case Q38R_GGML_IQ3_XXS: return dot_iq3_xxs(row, view, blocks);
    case Q38R_GGML_IQ3_S: return dot_iq3_s(row, view, blocks);
    case Q38R_GGML_IQ1_S: return dot_iq1_s(row, view, blocks);
    case Q38R_GGML_IQ1_M: return dot_iq1_m(row, view, blocks);
    default: return NAN;
    }
}

typedef struct {
    int type, rows, width, n_tokens, row0, row1;
    const uint8_t *weights;
    const void *planar;
    float *out;
} gemv_job;

static void *gemv_worker(void *arg) {
    const gemv_job *j = (const gemv_job *)arg;
    const size_t row_bytes = (size_t)(j->width / Q38R_Q8K_BLOCK) * q38r_quant_block_bytes(j->type);
    for (int row = j->row0; row < j->row1; ++row)
        for (int t = 0; t < j->n_tokens; ++t)
            j->out[(size_t)t * j->rows + row] =
                q38r_dot_q8_k(j->type, j->weights + row * row_bytes, j->planar, j->n_tokens, j->width, t);
    return NULL;
}

int q38r_gemv_q8_k(int ggml_type, int rows, int width, const void *weights, const void *planar, int n_tokens,
                   float *out, int n_threads) {
    if (q38r_quant_block_bytes(ggml_type) == 0 || width % Q38R_Q8K_BLOCK != 0 || width / Q38R_Q8K_BLOCK > 256)
        return -1;
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 64) n_threads = 64;
    pthread_t th[64];
    int created[64] = {0};
    gemv_job jobs[64];
    const int per = (rows + n_threads - 1) / n_threads;
    for (int i = 0; i < n_threads; ++i) {
        const int row0 = i * per;
        const int row1 = (i + 1) * per < rows ? (i + 1) * per : rows;
        if (row0 >= row1) break;
        jobs[i] = (gemv_job){ggml_type, rows, width, n_tokens, row0, row1, (const uint8_t *)weights, planar, out};
        if (n_threads > 1 && pthread_create(&th[i], NULL, gemv_worker, &jobs[i]) == 0)
            created[i] = 1;
        else
            gemv_worker(&jobs[i]);
    }
    for (int i = 0; i < n_threads; ++i)
        if (created[i]) pthread_join(th[i], NULL);
    return 0;
}

/* ---------------------------------------------------------------- f32 input */

static float read_f32(const uint8_t *p) {
    float v;
    memcpy(&v, p, sizeof(v));
    return v;
}

/* bf16_to_f32, quant.rs:49-51 */
static float bf16_to_f32(const uint8_t *p) {
    const uint32_t bits = (uint32_t)read_u16(p) << 16;
    float v;
    memcpy(&v, &bits, sizeof(v));
    return v;
}

/* Bytes of one block of `block_elems` weights of an f32-path type. */
int q38r_f32_block(int ggml_type, int *block_elems) {
    switch (ggml_type) {
    case Q38R_GGML_F32: *block_elems = 1; return 4;
    case Q38R_GGML_F16: *block_elems = 1; return 2;
    case Q38R_GGML_BF16: *block_elems = 1; return 2;
    case Q38R_GGML_Q8_0: *block_elems = 32; return 34;
    default: *block_elems = 0; return 0;
    }
}

/* dot_f32_scalar / dot_f16_scalar / dot_bf16_scalar / dot_q8_0_scalar,
 * tensor.rs:79-117: one sequential fused multiply-add chain over the row
 * (mul_add).  Q8_0: d * q rounded first, then the fused add. */
float q38r_dot_f32_row(int ggml_type, const uint8_t *row, const float *input, int n) {
    float total = 0.0f;
    switch (ggml_type) {
    case Q38R_GGML_F32:
        for (int i = 0; i < n; ++i) total = fmaf(read_f32(row + (size_t)i * 4), input[i], total);
        return total;
    case Q38R_GGML_F16:
        for (int i = 0; i < n; ++i) total = fmaf(q38r_f16_to_f32(read_u16(row + (size_t)i * 2)), input[i], total);
        return total;
    case Q38R_GGML_BF16:
#if Q38R_MUTANT == 21
        for (int i = 0; i < n; ++i) total = fmaf(bf16_to_f32(row + (size_t)(i ^ 1) * 2), input[i], total); /* planted */
#else
        for (int i = 0; i < n; ++i) total = fmaf(bf16_to_f32(row + (size_t)i * 2), input[i], total);
#endif
        return total;
    case Q38R_GGML_Q8_0: {
        int base = 0, block = 0;
        while (base < n) {
            const float d = q38r_f16_to_f32(read_u16(row + (size_t)block * 34));
            for (int i = 0; i < 32; ++i) {
                const int8_t q = (int8_t)row[(size_t)block * 34 + 2 + i];
                total = fmaf(d * (float)q, input[base + i], total);
            }
            base += 32;
            block += 1;
        }
        return total;
    }
    default:
        return NAN;
    }
}

typedef struct {
    int type, rows, width, n_tokens, row0, row1;
    size_t row_bytes;
    const uint8_t *weights;
    const float *input;
    float *out;
} gemv_f32_job;

static void *gemv_f32_worker(void *arg) {
    const gemv_f32_job *j = (const gemv_f32_job *)arg;
    for (int row = j->row0; row < j->row1; ++row)
        for (int t = 0; t < j->n_tokens; ++t)
            j->out[(size_t)t * j->rows + row] = q38r_dot_f32_row(j->type, j->weights + (size_t)row * j->row_bytes,
                                                                 j->input + (size_t)t * j->width, j->width);
    return NULL;
}

/* tensor_gemv_f32 / tensor_gemm_f32 (tensor.rs:1095-1129, :1175-1215):
 * out[t*rows + row] = dot_row(row, input token t); rows over threads. */
int q38r_gemv_f32(int ggml_type, int rows, int width, const void *weights, const float *input, int n_tokens,
                  float *out, int n_threads) {
    int be = 0;
    const int bb = q38r_f32_block(ggml_type, &be);
    if (bb == 0 || width % be != 0 || rows < 0 || n_tokens < 0) return -1;
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 64) n_threads = 64;
    pthread_t th[64];
    int created[64] = {0};
    gemv_f32_job jobs[64];
    const int per = (rows + n_threads - 1) / n_threads;
    for (int i = 0; i < n_threads; ++i) {
        const int row0 = i * per;
        const int row1 = (i + 1) * per < rows ? (i + 1) * per : rows;
        if (row0 >= row1) break;
        jobs[i] = (gemv_f32_job){ggml_type, rows, width, n_tokens, row0, row1, (size_t)(width / be) * bb,
                                 (const uint8_t *)weights, input, out};
        if (n_threads > 1 && pthread_create(&th[i], NULL, gemv_f32_worker, &jobs[i]) == 0)
            created[i] = 1;
        else
            gemv_f32_worker(&jobs[i]);
    }
    for (int i = 0; i < n_threads; ++i)
        if (created[i]) pthread_join(th[i], NULL);
    return 0;
}
