/*
 * q38_gguf.h -- the model file on the device: a GGUF reader with the
 * reference's validation and a streamed upload of the tensor data into one
 * device allocation, plus the device-side checkpoint of the recurrent state.
 *
 * Same conventions as q38_attn.h: 0 on success, -1 on failure with the
 * message in q38_last_error(); a failed call changes nothing.
 */
#ifndef Q38_GGUF_H
#define Q38_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "q38_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

#define Q38_GGUF_MAX_DIMS 8

typedef struct q38_gguf q38_gguf;

/*
 * Gguf::open (src/gguf/mod.rs:459-532): map the file and parse the header
 * (magic "GGUF", version 2 or 3, at least one tensor), the metadata
 * (parse_metadata, :347-409: scalars, strings, arrays of non-array types)
 * and the tensor table (parse_tensors, :411-457: 1..8 dimensions, non-zero
 * extents without overflow, a known ggml type whose block divides the first
 * extent), then general.alignment (a power of two, default 32), the data
 * offset (the table's end rounded up to it) and every tensor's bounds.  Each
 * rejection carries the reference's message ("invalid GGUF: ...").
 * Reads only the host file; no device is touched.
 */
int q38_gguf_open(const char *path, q38_gguf **out);
int q38_gguf_close(q38_gguf *g);

int q38_gguf_info(const q38_gguf *g, uint32_t *version, uint32_t *alignment, uint64_t *data_offset,
                  int *n_tensors, int *n_metadata);

/* find_tensor (:313-315): the first tensor of that name; -1 if absent. */
int q38_gguf_find_tensor(const q38_gguf *g, const char *name, int *index);

/* One tensor entry (TensorEntry, :207-216): name (NUL-terminated, owned by
 * the handle), ggml type id, dimensions, extents (shape[0] is the row
 * length), offset within the data section and byte size. */
int q38_gguf_tensor(const q38_gguf *g, int index, const char **name, int *ggml_type, int *n_dims,
                    uint64_t shape[Q38_GGUF_MAX_DIMS], uint64_t *offset, uint64_t *nbytes);

/* meta_u32 (:331-337): a Uint32 metadata value; -1 if absent or not Uint32. */
int q38_gguf_meta_u32(const q38_gguf *g, const char *key, uint32_t *value);

/*
 * The tensor data of the file in one device allocation of *bytes bytes (the
 * data section up to the end of its last tensor), tensor i at d_base +
 * offset_i: the reference maps the file (:467-468) and reads each tensor in
 * place; here the bytes are streamed from the file through two pinned
 * staging buffers into HBM on the context's stream, once.  Offsets keep the
 * file's alignment (32 bytes or more), so Q4_K/Q5_K/Q6_K matrices can go to
 * q38_gemv_q8_k and F32 vectors to the cores as they are.  The caller frees
 * d_base with q38_free.  Returns after the copy is complete.
 */
int q38_gguf_upload(q38_ctx *ctx, const q38_gguf *g, void **d_base, size_t *bytes);

/*
 * checkpoint_state / restore_target_state (src/model/ops.rs:1627-1647) on
 * the device: copy a sequence's recurrent state -- conv_state
 * [48][10240][3] (per layer, channel-major with the 3 taps of a channel
 * adjacent) and delta_state [48][48][128][128] f32, n_conv and
 * n_delta floats (multiples of 4, 16-byte aligned) -- to the checkpoint and
 * back, ordered on the context's stream (no host round trip).  The position
 * the reference saves with it is the caller's scalar; the KV cache rolls
 * back by position with q38_seq_truncate.
 */
int q38_recurrent_checkpoint(q38_ctx *ctx, const float *d_conv_state, const float *d_delta_state,
                             size_t n_conv, size_t n_delta, float *d_conv_ckpt, float *d_delta_ckpt);
int q38_recurrent_restore(q38_ctx *ctx, const float *d_conv_ckpt, const float *d_delta_ckpt, size_t n_conv,
                          size_t n_delta, float *d_conv_state, float *d_delta_state);

#ifdef __cplusplus
}
#endif
#endif
