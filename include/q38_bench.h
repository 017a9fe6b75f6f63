/*
 * q38_bench.h -- instrumentation exported by libq38attn.so beside the C ABI
 * of q38_attn.h: stream events, per-kernel dispatch timing, the seeded
 * device generator and a calibration copy.  None of these has a counterpart
 * in the reference (a CPU engine with no device); the benchmark and the
 * tests use them to produce inputs and to time kernels.  A caller that only
 * replaces the reference's attention path needs q38_attn.h alone.
 */
#ifndef Q38_BENCH_H
#define Q38_BENCH_H

#include "q38_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Events on the context's stream, for timing. */
int q38_event_create(q38_ctx *ctx, void **event);
int q38_event_record(q38_ctx *ctx, void *event);
int q38_event_elapsed_ms(void *start, void *stop, float *ms);
int q38_event_destroy(void *event);

/* Time every launch of one kernel of this library (by its symbol name, e.g.
 * "q38_attn_decode_split") with a pair of events on the context's stream,
 * for up to max_launches launches; stop returns the summed kernel time. */
int q38_kernel_timer_start(q38_ctx *ctx, const char *kernel_name, int max_launches);
int q38_kernel_timer_stop(q38_ctx *ctx, float *total_ms, int *launches);

/* Seeded N(mean, sigma^2) f32 fill on the device: element i equals what the
 * host generator (SplitMix64 + Box-Muller, qwen3.8_27b_in_rust_amd/synth.py)
 * gives for the same seed.  For benchmark inputs of many gigabytes. */
int q38_fill_normal(q38_ctx *ctx, float *d_out, size_t n, uint64_t seed, float sigma, float mean);

/* Plain device-to-device copy by a kernel of this library (bytes a multiple
 * of 16, pointers 16-byte aligned): reads and writes exactly `bytes` each,
 * the calibration figure for hardware memory counters.  No counterpart in
 * the reference (which has no device). */
int q38_device_copy(q38_ctx *ctx, void *d_dst, const void *d_src, size_t bytes);

/* Launch an empty kernel (one 64-thread workgroup) on the context's
 * stream: the launch floor that one dependent launch costs. */
int q38_device_noop(q38_ctx *ctx);

#ifdef __cplusplus
}
#endif
#endif
