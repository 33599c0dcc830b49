/*
 * gliner_decide_diag.h -- diagnostic entry points of libgliner_decide_hip.so.
 *
 * No counterpart in the reference: these measure the device, not the model.
 * Same conventions as gliner_decide.h (device pointers, void* HIP stream,
 * gd_status return).
 */
#ifndef GLINER_DECIDE_DIAG_H_
#define GLINER_DECIDE_DIAG_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#pragma GCC visibility push(default)
#endif

/* c[i] = a[i] + b[i] over n fp16 values (n % 32 == 0, 16-byte aligned
 * pointers): two reads and one write of the same size with 16-byte
 * non-temporal accesses, four per lane, and no other work -- the streaming
 * ceiling of the residual LayerNorm's access pattern (x and residual read,
 * the output written once) on this device. */
int gd_stream_probe_add(const void* a, const void* b, void* c, int64_t n, void* stream);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif

#ifdef __cplusplus
}
#endif

#endif /* GLINER_DECIDE_DIAG_H_ */
