// Residual-add LayerNorm and the embedding gather + LayerNorm + mask stage.
//
// Reference: FusedKernels.swift:125-155 (residual LN Metal kernel, one
// 32-lane simdgroup per row, three passes over x and residual) and the
// default graph ops DeBERTa.swift:94-106, 285-292, 449-464.
//
// gfx950 design: one wave64 per row.  For the model width (1024) each lane
// owns 16 elements loaded as two 16-byte vectors per tensor, so a row is read
// exactly once, held in registers, reduced across the wave with DPP moves
// (mean, then the centred second moment; no LDS round trips) and written
// once: 3 x 2 KiB of HBM traffic per row for residual LN, the algorithmic
// minimum.  gamma and beta are loaded before the row so their latency does
// not sit between the reductions and the stores.

#include "gd_common.hpp"
#include "gd_kernels.hpp"

namespace gd {
namespace {

constexpr int kRowsPerBlock = 4;  // 4 waves, one row each

template <int VPL>
struct RowVec {
  float v[VPL][8];
};

// Loads one row (VPL 8-wide vectors per lane) of x (+ residual), optionally
// rounding the sum to fp16.  Returns the lane's partial sum.
template <int VPL>
__device__ __forceinline__ float load_row_sum(const half_t* x, const half_t* res,
                                              int64_t row, int lane, bool round_sum, RowVec<VPL>& r) {
  constexpr int C = 64 * 8 * VPL;
  const half8_t* xr = reinterpret_cast<const half8_t*>(x + row * C);
  const half8_t* rr = res ? reinterpret_cast<const half8_t*>(res + row * C) : nullptr;
  half8_t a[VPL], b[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) a[j] = __builtin_nontemporal_load(xr + j * 64 + lane);
  if (rr) {
#pragma unroll
    for (int j = 0; j < VPL; ++j) b[j] = __builtin_nontemporal_load(rr + j * 64 + lane);
  }
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float s = (float)a[j][e];
      if (rr) {
        s += (float)b[j][e];
        if (round_sum) s = round_f16(s);
      }
      r.v[j][e] = s;
      sum += s;
    }
  }
  return sum;
}

// gamma / beta of this lane's elements, loaded once before the row data so
// their latency is off the path between the reductions and the stores.
template <int VPL>
struct Affine {
  half8_t g[VPL], b[VPL];
  __device__ __forceinline__ void load(const half_t* __restrict__ gamma, const half_t* __restrict__ beta, int lane) {
    const half8_t* g8 = reinterpret_cast<const half8_t*>(gamma);
    const half8_t* b8 = reinterpret_cast<const half8_t*>(beta);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      g[j] = g8[j * 64 + lane];
      b[j] = b8[j * 64 + lane];
    }
  }
};

template <int VPL>
__device__ __forceinline__ void normalize_store(RowVec<VPL>& r, float sum, const Affine<VPL>& aff, half_t* out,
                                                int64_t row, int lane, float eps, float scale_mask) {
  constexpr int C = 64 * 8 * VPL;
  const float mean = wave_sum_dpp(sum) * (1.0f / C);
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < VPL; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = r.v[j][e] - mean;
      sq += d * d;
    }
  const float var = wave_sum_dpp(sq) * (1.0f / C);
  const float inv = 1.0f / sqrtf(var + eps);
  half8_t* o8 = reinterpret_cast<half8_t*>(out + row * C);
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const half8_t g = aff.g[j];
    const half8_t bb = aff.b[j];
    half8_t o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float y = (r.v[j][e] - mean) * inv * (float)g[e] + (float)bb[e];
      if (scale_mask != 1.0f) y = (float)(half_t)y * scale_mask;  // fp16 LN output times fp16 mask
      o[e] = (half_t)y;
    }
    o8[j * 64 + lane] = o;
  }
}

// Each wave normalises RPW consecutive rows; their loads are all issued
// before the first reduction so more bytes are in flight per wave.
// x, res and out carry no __restrict__: out may alias x or res (each lane
// reads its elements before it writes the same elements).
template <int VPL, int RPW>
__global__ __launch_bounds__(256) void residual_ln_kernel(const half_t* x, const half_t* res,
                                                          const half_t* __restrict__ gamma,
                                                          const half_t* __restrict__ beta, half_t* out,
                                                          int64_t rows, float eps, int round_sum) {
  const int lane = threadIdx.x & 63;
  const int64_t row0 = ((int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6)) * RPW;
  Affine<VPL> aff;
  aff.load(gamma, beta, lane);
  RowVec<VPL> r[RPW];
  float sum[RPW];
#pragma unroll
  for (int i = 0; i < RPW; ++i)
    if (row0 + i < rows) sum[i] = load_row_sum<VPL>(x, res, row0 + i, lane, round_sum != 0, r[i]);
#pragma unroll
  for (int i = 0; i < RPW; ++i)
    if (row0 + i < rows) normalize_store<VPL>(r[i], sum[i], aff, out, row0 + i, lane, eps, 1.0f);
}

// Any width that is a multiple of 8: three passes like the reference kernel
// (mean, variance, output), re-reading the row from memory.
__global__ __launch_bounds__(256) void residual_ln_generic_kernel(const half_t* x, const half_t* res,
                                                                  const half_t* __restrict__ gamma,
                                                                  const half_t* __restrict__ beta, half_t* out, int64_t rows, int64_t cols,
                                                                  float eps, int round_sum) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const half_t* xr = x + row * cols;
  const half_t* rr = res ? res + row * cols : nullptr;
  auto value = [&](int64_t j) {
    float s = (float)xr[j];
    if (rr) {
      s += (float)rr[j];
      if (round_sum) s = round_f16(s);
    }
    return s;
  };
  float sum = 0.f;
  for (int64_t j = lane; j < cols; j += 64) sum += value(j);
  const float mean = wave_sum(sum) / (float)cols;
  float sq = 0.f;
  for (int64_t j = lane; j < cols; j += 64) {
    const float d = value(j) - mean;
    sq += d * d;
  }
  const float inv = 1.0f / sqrtf(wave_sum(sq) / (float)cols + eps);
  // Read every input before the first write: `out` may alias x or res, and
  // all lanes must finish reading the row before any lane overwrites it.
  __builtin_amdgcn_wave_barrier();
  half_t* orow = out + row * cols;
  for (int64_t j0 = 0; j0 < cols; j0 += 64) {
    const int64_t j = j0 + lane;
    float y = 0.f;
    if (j < cols) y = (value(j) - mean) * inv * (float)gamma[j] + (float)beta[j];
    __builtin_amdgcn_wave_barrier();
    if (j < cols) orow[j] = (half_t)y;
  }
}

// Output row t of the embedding reads token row_map[t] of ids / mask (packed
// rows), or token t without a map; a map entry outside [0, sources) reads
// token 0 and raises the error flag.
__device__ __forceinline__ int64_t source_row(const int32_t* __restrict__ row_map, int64_t t, int64_t sources,
                                              int32_t* __restrict__ error_flag, int lane) {
  if (row_map == nullptr) return t;
  int64_t s = row_map[t];
  if (s < 0 || s >= sources) {
    if (error_flag && lane == 0) atomicOr(error_flag, 1);
    s = 0;
  }
  return s;
}

template <int VPL>
__global__ __launch_bounds__(256) void embedding_ln_kernel(const int32_t* __restrict__ ids,
                                                           const half_t* __restrict__ mask,
                                                           const half_t* __restrict__ table,
                                                           const half_t* __restrict__ gamma,
                                                           const half_t* __restrict__ beta, half_t* __restrict__ out,
                                                           int64_t tokens, int64_t vocab, float eps,
                                                           int32_t* __restrict__ error_flag,
                                                           const int32_t* __restrict__ row_map, int64_t sources) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (t >= tokens) return;
  const int64_t src = source_row(row_map, t, sources, error_flag, lane);
  int64_t id = ids[src];
  if (id < 0 || id >= vocab) {
    if (error_flag && lane == 0) atomicOr(error_flag, 1);
    id = 0;
  }
  Affine<VPL> aff;
  aff.load(gamma, beta, lane);
  RowVec<VPL> r;
  const float sum = load_row_sum<VPL>(table, nullptr, id, lane, false, r);
  const float m = (float)mask[src];
  // out = fp16(fp16(LN) * fp16(mask)); for the usual 0/1 mask this is LN or 0.
  normalize_store<VPL>(r, sum, aff, out, t, lane, eps, m);
}

__global__ __launch_bounds__(256) void embedding_ln_generic_kernel(const int32_t* __restrict__ ids,
                                                                   const half_t* __restrict__ mask,
                                                                   const half_t* __restrict__ table,
                                                                   const half_t* __restrict__ gamma,
                                                                   const half_t* __restrict__ beta,
                                                                   half_t* __restrict__ out, int64_t tokens,
                                                                   int64_t cols, int64_t vocab, float eps,
                                                                   int32_t* __restrict__ error_flag,
                                                                   const int32_t* __restrict__ row_map,
                                                                   int64_t sources) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (t >= tokens) return;
  const int64_t src = source_row(row_map, t, sources, error_flag, lane);
  int64_t id = ids[src];
  if (id < 0 || id >= vocab) {
    if (error_flag && lane == 0) atomicOr(error_flag, 1);
    id = 0;
  }
  const half_t* xr = table + id * cols;
  float sum = 0.f;
  for (int64_t j = lane; j < cols; j += 64) sum += (float)xr[j];
  const float mean = wave_sum(sum) / (float)cols;
  float sq = 0.f;
  for (int64_t j = lane; j < cols; j += 64) {
    const float d = (float)xr[j] - mean;
    sq += d * d;
  }
  const float inv = 1.0f / sqrtf(wave_sum(sq) / (float)cols + eps);
  const float m = (float)mask[src];
  half_t* orow = out + t * cols;
  for (int64_t j = lane; j < cols; j += 64) {
    const float y = ((float)xr[j] - mean) * inv * (float)gamma[j] + (float)beta[j];
    orow[j] = (half_t)((float)(half_t)y * m);
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Streaming reference of the LayerNorm's traffic (gd_stream_probe_add): each
// lane reads four 16-byte pieces of a and of b and writes four of c, all
// non-temporal; a block of 256 lanes covers 1024 consecutive pieces.
__global__ __launch_bounds__(256) void stream_probe_kernel(const half8_t* __restrict__ a,
                                                           const half8_t* __restrict__ b, half8_t* __restrict__ c,
                                                           int64_t n8) {
  const int64_t base = (int64_t)blockIdx.x * 1024 + threadIdx.x;
  half8_t x[4], y[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int64_t i = base + v * 256;
    if (i < n8) {
      x[v] = __builtin_nontemporal_load(a + i);
      y[v] = __builtin_nontemporal_load(b + i);
    }
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int64_t i = base + v * 256;
    if (i < n8) __builtin_nontemporal_store(x[v] + y[v], c + i);
  }
}

}  // namespace

int launch_stream_probe_add(const void* a, const void* b, void* c, int64_t n, hipStream_t stream) {
  if (n == 0) return GD_OK;
  const int64_t n8 = n / 8;
  hipLaunchKernelGGL(stream_probe_kernel, dim3((unsigned)((n8 + 1023) / 1024)), dim3(256), 0, stream,
                     static_cast<const half8_t*>(a), static_cast<const half8_t*>(b), static_cast<half8_t*>(c), n8);
  GD_LAUNCH_CHECK();
  return GD_OK;
}

int launch_residual_layer_norm(const void* x, const void* residual, const void* gamma, const void* beta, void* out,
                               int64_t rows, int64_t cols, float eps, uint32_t flags, hipStream_t stream) {
  if (rows == 0) return GD_OK;
  const dim3 block(256);
  const dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock));
  const int round_sum = (flags & GD_LN_SUM_F16) ? 1 : 0;
  auto X = static_cast<const half_t*>(x);
  auto R = static_cast<const half_t*>(residual);
  auto G = static_cast<const half_t*>(gamma);
  auto Bt = static_cast<const half_t*>(beta);
  auto O = static_cast<half_t*>(out);
  const bool vec_ok = aligned16(x) && (!residual || aligned16(residual)) && aligned16(gamma) && aligned16(beta) &&
                      aligned16(out);
  if (vec_ok && cols == 1024) {
    hipLaunchKernelGGL((residual_ln_kernel<2, 1>), grid, block, 0, stream, X, R, G, Bt, O, rows, eps, round_sum);
  } else if (vec_ok && cols == 512) {
    hipLaunchKernelGGL((residual_ln_kernel<1, 1>), grid, block, 0, stream, X, R, G, Bt, O, rows, eps, round_sum);
  } else if (vec_ok && cols == 2048) {
    hipLaunchKernelGGL((residual_ln_kernel<4, 1>), grid, block, 0, stream, X, R, G, Bt, O, rows, eps, round_sum);
  } else {
    hipLaunchKernelGGL(residual_ln_generic_kernel, grid, block, 0, stream, X, R, G, Bt, O, rows, cols, eps, round_sum);
  }
  GD_LAUNCH_CHECK();
  return GD_OK;
}

int launch_embedding_layer_norm(const int32_t* ids, const void* mask, const void* table, const void* gamma,
                                const void* beta, void* out, int64_t tokens, int64_t cols, int64_t vocab, float eps,
                                int32_t* error_flag, hipStream_t stream, const int32_t* row_map, int64_t sources) {
  if (tokens == 0) return GD_OK;
  const dim3 block(256);
  const dim3 grid((unsigned)((tokens + kRowsPerBlock - 1) / kRowsPerBlock));
  auto M = static_cast<const half_t*>(mask);
  auto T = static_cast<const half_t*>(table);
  auto G = static_cast<const half_t*>(gamma);
  auto Bt = static_cast<const half_t*>(beta);
  auto O = static_cast<half_t*>(out);
  const bool vec_ok = aligned16(table) && aligned16(gamma) && aligned16(beta) && aligned16(out);
  if (vec_ok && cols == 1024) {
    hipLaunchKernelGGL(embedding_ln_kernel<2>, grid, block, 0, stream, ids, M, T, G, Bt, O, tokens, vocab, eps,
                       error_flag, row_map, sources);
  } else {
    hipLaunchKernelGGL(embedding_ln_generic_kernel, grid, block, 0, stream, ids, M, T, G, Bt, O, tokens, cols, vocab,
                       eps, error_flag, row_map, sources);
  }
  GD_LAUNCH_CHECK();
  return GD_OK;
}

}  // namespace gd
