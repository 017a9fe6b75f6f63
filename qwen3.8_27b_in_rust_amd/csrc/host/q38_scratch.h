/*
 * Internal to libq38attn.so: the device address of the fixed scratch array
 * of q38_scratch.hip on one device.
 */
#ifndef Q38_SCRATCH_H
#define Q38_SCRATCH_H

#define Q38_SCRATCH_MAX_DEVICES 64

#ifdef __cplusplus
extern "C" {
#endif

/* With `device` current: the device address of its copy of the scratch
 * array (looked up once per device, then cached).  Returns 0, or a
 * hipError_t code. */
int q38_scratch_address(int device, void **ptr);

#ifdef __cplusplus
}
#endif
#endif
