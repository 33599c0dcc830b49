// Shared helpers for the gfx950 kernels and the C-ABI: status codes, error
// reporting, fp16 vector types, wave64 reductions and MFMA wrappers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "gliner_decide.h"

namespace gd {

// ---------------------------------------------------------------------------
// Error reporting: every C-ABI call returns a gd_status; the message of the
// last failure on the calling thread is kept for gd_last_error().
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
const char* last_error();
void clear_error();

inline int fail(int code, const char* msg) {
  set_error("%s", msg);
  return code;
}

#define GD_CHECK_ARG(cond, ...)                  \
  do {                                           \
    if (!(cond)) {                               \
      ::gd::set_error(__VA_ARGS__);              \
      return GD_ERR_INVALID_ARGUMENT;            \
    }                                            \
  } while (0)

#define GD_CHECK_SHAPE(cond, ...)                \
  do {                                           \
    if (!(cond)) {                               \
      ::gd::set_error(__VA_ARGS__);              \
      return GD_ERR_SHAPE;                       \
    }                                            \
  } while (0)

// On failure the thread's HIP error state is cleared (hipGetLastError), so a
// failed call is reported once, by its own entry point, and not again by the
// next launch check.
#define GD_HIP_CHECK(expr)                                                        \
  do {                                                                            \
    hipError_t gd_hip_err_ = (expr);                                              \
    if (gd_hip_err_ != hipSuccess) {                                              \
      (void)hipGetLastError();                                                    \
      ::gd::set_error("HIP error %s (%d) at %s:%d: %s", hipGetErrorName(gd_hip_err_), \
                      (int)gd_hip_err_, __FILE__, __LINE__, #expr);               \
      return GD_ERR_HIP;                                                          \
    }                                                                             \
  } while (0)

// After a kernel launch: report launch failures as GD_ERR_HIP.
#define GD_LAUNCH_CHECK() GD_HIP_CHECK(hipGetLastError())

#define GD_RETURN_IF_ERROR(expr)      \
  do {                                \
    int gd_status_ = (expr);          \
    if (gd_status_ != GD_OK) return gd_status_; \
  } while (0)

// ---------------------------------------------------------------------------
// Device-side types
// ---------------------------------------------------------------------------
typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t uint4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Round-trip through fp16 (round to nearest even), staying in fp32.
__device__ __forceinline__ float round_f16(float x) { return (float)(half_t)x; }

// Butterfly reductions across the 64 lanes of a wave.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Sum across the 64 lanes in VALU data-parallel-primitive moves (no LDS
// round trips): quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror and
// row_mirror leave every lane holding the sum of its 16-lane row; the four
// row sums are read out and added (every lane gets the same value).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);  // row_half_mirror
  v += dpp_mov<0x140>(v);  // row_mirror
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Max and sum over the four 16-lane rows of a wave (lanes l, l ^ 16, l ^ 32,
// l ^ 48), every lane receiving the result: gfx950's row-swapping permlanes
// (v_permlane16_swap: odd rows of the first operand <-> even rows of the
// second; v_permlane32_swap: upper half of the first <-> lower half of the
// second) give each lane its partner's value in VALU, without an LDS round
// trip.  The pairs are combined as x_l op x_(l^16), then op x_(l^32): the
// same operands, in the same order up to commutation, as the two xor
// shuffles they replace, so the results are bitwise the same.
__device__ __forceinline__ float rows_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                  false, false);
  const uint32_t a0 = a[0], a1 = a[1];  // (elements extracted before the casts)
  v = fmaxf(__builtin_bit_cast(float, a0), __builtin_bit_cast(float, a1));
  const auto b = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                  false, false);
  const uint32_t b0 = b[0], b1 = b[1];
  return fmaxf(__builtin_bit_cast(float, b0), __builtin_bit_cast(float, b1));
}
__device__ __forceinline__ float rows_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                  false, false);
  const uint32_t a0 = a[0], a1 = a[1];
  v = __builtin_bit_cast(float, a0) + __builtin_bit_cast(float, a1);
  const auto b = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                  false, false);
  const uint32_t b0 = b[0], b1 = b[1];
  return __builtin_bit_cast(float, b0) + __builtin_bit_cast(float, b1);
}

// Orders this wave's LDS writes before its later LDS reads by other lanes of
// the same wave.  LDS operations of one wavefront execute in issue order, so
// wavefront-scope fences emit no wait; they only stop the compiler from
// moving the accesses across this point.  Outstanding global loads are left
// in flight (a workgroup-scope fence would drain them).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// vmcnt(N) with lgkmcnt / expcnt left unconstrained (gfx9 s_waitcnt encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (((N >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier for pipelines that load LDS by DMA: this wave's LDS
// accesses are complete (lgkmcnt(0)); global loads, including DMA into LDS
// still in flight, are waited for explicitly by the caller (__syncthreads
// would drain them).  The empty asm statements keep the compiler from moving
// memory accesses across.
__device__ __forceinline__ void stage_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// MFMA wrappers (gfx950 double-rate fp16 forms).
//  16x16x32: A lane l -> row l%16, k = 8*(l/16)+[0,8); B lane l -> col l%16,
//            same k; C lane l -> col l%16, rows 4*(l/16)+[0,4).
//  32x32x16: A lane l -> row l%32, k = 8*(l/32)+[0,8); B likewise; C lane l
//            -> col l%32, rows 8*(i/4) + 4*(l/32) + i%4 for acc index i.
__device__ __forceinline__ float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float16_t mfma32x32x16(half8_t a, half8_t b, float16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// DeBERTa log-bucket relative position -> index into the 2*span relative
// tables: clip(bucket(r) + span, 0, 2*span - 1).  Evaluated in fp32.  For
// bucket_size 256 / max_position 512 and |r| <= 511 the exact value
// x = ln(|r|/128) / ln(511/128) * 127 is either an integer (only at
// |r| = 511, x = 127) or at least 0.003 away from one, so ceil(x - 1e-3)
// reproduces the float64 reference exactly even when the two logs are
// rounded differently (e.g. one constant-folded at compile time).
__device__ __forceinline__ int relative_index(int r, int bucket_size, int max_position) {
  const int mid = bucket_size >> 1;
  int bucket;
  const int a = r < 0 ? -r : r;
  if (a <= mid) {
    bucket = r;
  } else {
    const float x = logf((float)a / (float)mid) / logf((float)(max_position - 1) / (float)mid) * (float)(mid - 1);
    const int lp = (int)ceilf(x - 1e-3f) + mid;
    bucket = r < 0 ? -lp : lp;
  }
  int idx = bucket + bucket_size;
  idx = idx < 0 ? 0 : idx;
  idx = idx > 2 * bucket_size - 1 ? 2 * bucket_size - 1 : idx;
  return idx;
}

}  // namespace gd
