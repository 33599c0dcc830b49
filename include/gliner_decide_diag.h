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

/* The two MFMA forms of one 16-product K slice, per 32 x 32 tile t
 * (0 <= tiles <= 2^20): d32[t] = A[t] W[t]^T + C0[t] through one
 * v_mfma_f32_32x32x16_f16 and d16[t] through four v_mfma_f32_16x16x16_f16.
 * a, w: fp16 [tiles][32][16]; c0, d32, d16: fp32 [tiles][32][32], row-major.
 * The GEMM for at most 32 rows uses the second form and the tile kernels the
 * first; their rows agree bit for bit only if d32 and d16 do. */
int gd_diag_mfma_forms(const void* a, const void* w, const float* c0, float* d32, float* d16, int64_t tiles,
                       void* stream);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif

#ifdef __cplusplus
}
#endif

#endif /* GLINER_DECIDE_DIAG_H_ */
