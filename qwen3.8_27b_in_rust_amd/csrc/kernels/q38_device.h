/*
 * Device helpers for the gfx950 (CDNA4, wave64) kernels: DPP and permlane
 * cross-lane reductions, 128-bit vector access, and the exp/sigmoid forms the
 * attention path uses.
 */
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../q38_kargs.h"

typedef float f32x4 __attribute__((ext_vector_type(4)));

#define Q38_DEV __device__ __forceinline__

template <int CTRL>
Q38_DEV float q38_dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

/* All-reduce (sum) over each row of 16 lanes: quad_perm [1,0,3,2], quad_perm
 * [2,3,0,1], row_half_mirror, row_mirror.  Every lane of the row ends with the
 * row's total; no LDS traffic. */
Q38_DEV float q38_sum16(float x) {
    x += q38_dpp<0xB1>(x);
    x += q38_dpp<0x4E>(x);
    x += q38_dpp<0x141>(x);
    x += q38_dpp<0x140>(x);
    return x;
}

Q38_DEV float q38_max16(float x) {
    x = fmaxf(x, q38_dpp<0xB1>(x));
    x = fmaxf(x, q38_dpp<0x4E>(x));
    x = fmaxf(x, q38_dpp<0x141>(x));
    x = fmaxf(x, q38_dpp<0x140>(x));
    return x;
}

/* Exchange rows 0<->1 and 2<->3 (lane i gets lane i^16): v_permlane16_swap
 * applied to two copies of x returns {x with odd rows replaced by the even
 * rows, x with even rows replaced by the odd rows}; summing the two gives the
 * pairwise row total in every lane. */
Q38_DEV float q38_pair_rows_sum(float x) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

/* All-reduce (sum) over each half-wave of 32 lanes. */
Q38_DEV float q38_sum32(float x) { return q38_pair_rows_sum(q38_sum16(x)); }

/* The two half-waves' copies of x: after v_permlane32_swap on two copies of
 * x, one result holds the low half's value in every lane and the other the
 * high half's.  Callers combine them symmetrically, so which is which does
 * not matter. */
struct q38_halves {
    float a, b;
};
Q38_DEV q38_halves q38_both_halves(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}

Q38_DEV f32x4 q38_ld4(const float *p) { return *reinterpret_cast<const f32x4 *>(p); }
Q38_DEV void q38_st4(float *p, f32x4 v) { *reinterpret_cast<f32x4 *>(p) = v; }

/* Streaming loads that are read once: keep them out of the way of reused
 * data with the non-temporal hint. */
Q38_DEV f32x4 q38_ld4_stream(const float *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
}

/* Streaming store of data no kernel of this launch reads again. */
Q38_DEV void q38_st4_stream(float *p, f32x4 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<f32x4 *>(p));
}

Q38_DEV float q38_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

/* 1/(1+exp(-x)), ops.rs:501-503, with the accurate expf. */
Q38_DEV float q38_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
/* x/(1+exp(-x)), ops.rs:506-508 */
Q38_DEV float q38_silu(float x) { return x / (1.0f + expf(-x)); }
/* ops.rs:511-516 */
Q38_DEV float q38_softplus(float x) { return x > 20.0f ? x : logf(1.0f + expf(x)); }

Q38_DEV float q38_dot4(f32x4 a, f32x4 b, float acc) {
    acc = __builtin_fmaf(a.x, b.x, acc);
    acc = __builtin_fmaf(a.y, b.y, acc);
    acc = __builtin_fmaf(a.z, b.z, acc);
    acc = __builtin_fmaf(a.w, b.w, acc);
    return acc;
}

Q38_DEV f32x4 q38_fma4(float s, f32x4 v, f32x4 acc) {
    acc.x = __builtin_fmaf(s, v.x, acc.x);
    acc.y = __builtin_fmaf(s, v.y, acc.y);
    acc.z = __builtin_fmaf(s, v.z, acc.z);
    acc.w = __builtin_fmaf(s, v.w, acc.w);
    return acc;
}

/* f64 all-reduce over the wave (64 lanes) through ds_swizzle-free shuffles. */
Q38_DEV double q38_wave_sum_f64(double x) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
    return x;
}

/* s_waitcnt immediate (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4,
 * lgkmcnt 11:8) that waits until at most `vm` vector memory operations and
 * `lgkm` LDS/scalar operations of this wave are outstanding. */
constexpr int q38_waitcnt(int vm, int lgkm) { return (vm & 0xF) | ((vm >> 4) << 14) | (0x7 << 4) | (lgkm << 8); }

/* Workgroup barrier once this wave's LDS operations and all but its VM
 * youngest vector memory operations have completed.  Vector memory
 * operations complete in issue order, so loads issued ahead as prefetch (the
 * VM youngest) stay in flight across it; __syncthreads() would wait for
 * them, as its fences count direct-to-LDS loads as outstanding LDS writes. */
template <int VM>
Q38_DEV void q38_barrier_vm() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(q38_waitcnt(VM, 0));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

/* ------------------------------------------------ bf16x3 matrix-core tiles */

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

/* x = hi + lo with hi = bf16(x), lo = bf16(x - hi): hi + lo is within
 * ~2^-16 of x, so hi*hi + hi*lo + lo*hi carries f32-class products. */
Q38_DEV void q38_split8(const float (&x)[8], bf16x8 &hi, bf16x8 &lo) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const __bf16 h = (__bf16)x[j];
        hi[j] = h;
        lo[j] = (__bf16)(x[j] - (float)h);
    }
}

/*
 * One 16x16 output tile on v_mfma_f32_16x16x32_bf16 with bf16x3 products,
 * c += A B (A 16 x KD, B KD x 16, KD a multiple of 32), both operands already
 * split into bf16 hi/lo arrays (LDS): A row m at a_hi/a_lo + m*lda, and B
 * given by its columns, B(k, n) = b[n*ldb + k], each contiguous in k.  Lane l
 * supplies A row l%16 and B column l%16 at k = k0 + 8(l/16) .. +7 (one 16-byte
 * read per fragment half); the tile it returns holds rows 4(l/16) + i
 * (i = 0..3) of column l%16.  Row strides and the arrays must keep 16-byte
 * alignment.
 */
template <int KD>
Q38_DEV f32x4 q38_mma16_split(f32x4 c, const __bf16 *a_hi, const __bf16 *a_lo, int lda, const __bf16 *b_hi,
                              const __bf16 *b_lo, int ldb) {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4;
    const int r = lane & 15;
#pragma unroll
    for (int k0 = 0; k0 < KD; k0 += 32) {
        const int ao = r * lda + k0 + 8 * g;
        const int bo = r * ldb + k0 + 8 * g;
        const bf16x8 ah = *reinterpret_cast<const bf16x8 *>(a_hi + ao);
        const bf16x8 al = *reinterpret_cast<const bf16x8 *>(a_lo + ao);
        const bf16x8 bh = *reinterpret_cast<const bf16x8 *>(b_hi + bo);
        const bf16x8 bl = *reinterpret_cast<const bf16x8 *>(b_lo + bo);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, c, 0, 0, 0);
    }
    return c;
}
