// General-index attention kernels with the Metal kernels' semantics, and the
// relative index table.
//
// Reference: FusedKernels.swift:13-81 (fused attention) and :83-123 (relative
// bias), launched at :160-258; the index math DeBERTa.swift:498-551.  These
// take the c2p / p2c index tables as inputs (any indices, bounds-checked) and
// back the FusedKernels-shaped entry points.  The encoder itself runs the
// staged kernel of deberta_attention.hip, which derives the indices from the
// bucket function directly.
#include <cmath>

#include "gd_common.hpp"
#include "gd_kernels.hpp"

namespace gd {
namespace {

// ---------------------------------------------------------------------------
// General-index kernels with the Metal kernels' semantics (API parity).
// One wave64 per (b, h, query); lanes stride over keys (scores) and then over
// the head dimension (context).  fp32 arithmetic throughout, as the reference.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void relative_bias_general_kernel(
    const half_t* __restrict__ q, const half_t* __restrict__ k, const half_t* __restrict__ pos_key,
    const half_t* __restrict__ pos_query, const int32_t* __restrict__ c2p_idx, const int32_t* __restrict__ p2c_idx,
    const half_t* __restrict__ key_mask, float scale, int H, int L, int D, int P, half_t* __restrict__ out,
    int32_t* __restrict__ error_flag) {
  extern __shared__ float qcache[];
  const int row = blockIdx.x;  // (b*H + h)*L + query
  const int query = row % L;
  const int h = (row / L) % H;
  const int b = row / (H * L);
  const int lane = threadIdx.x;
  const half_t* qrow = q + (int64_t)row * D;
  for (int d = lane; d < D; d += 64) qcache[d] = (float)qrow[d];
  __syncthreads();
  for (int key = lane; key < L; key += 64) {
    const half_t* krow = k + (((int64_t)b * H + h) * L + key) * D;
    int ci = c2p_idx[((int64_t)h * L + query) * L + key];
    int pi = p2c_idx[((int64_t)h * L + key) * L + query];
    if (ci < 0 || ci >= P || pi < 0 || pi >= P) {
      if (error_flag) atomicOr(error_flag, 1);
      ci = ci < 0 ? 0 : (ci >= P ? P - 1 : ci);
      pi = pi < 0 ? 0 : (pi >= P ? P - 1 : pi);
    }
    const half_t* pk = pos_key + ((int64_t)h * P + ci) * D;
    const half_t* pq = pos_query + ((int64_t)h * P + pi) * D;
    float c2p = 0.f, p2c = 0.f;
    for (int d = 0; d < D; ++d) {
      const float kd = (float)krow[d];
      c2p += qcache[d] * (float)pk[d];
      p2c += kd * (float)pq[d];
    }
    float score = (c2p + p2c) * scale;
    if ((float)key_mask[(int64_t)b * L + key] < -60000.f) score = -65504.f;
    out[(int64_t)row * L + key] = (half_t)score;
  }
}

__global__ __launch_bounds__(64) void fused_attention_general_kernel(
    const half_t* __restrict__ q, const half_t* __restrict__ k, const half_t* __restrict__ v,
    const half_t* __restrict__ pos_key, const half_t* __restrict__ pos_query, const int32_t* __restrict__ c2p_idx,
    const int32_t* __restrict__ p2c_idx, const half_t* __restrict__ key_mask, float scale, int H, int L, int D, int P,
    half_t* __restrict__ out, int32_t* __restrict__ error_flag) {
  extern __shared__ float shm[];  // D floats of q, then L weights
  float* qcache = shm;
  float* weights = shm + D;
  const int row = blockIdx.x;
  const int query = row % L;
  const int h = (row / L) % H;
  const int b = row / (H * L);
  const int lane = threadIdx.x;
  const half_t* qrow = q + (int64_t)row * D;
  for (int d = lane; d < D; d += 64) qcache[d] = (float)qrow[d];
  __syncthreads();
  float local_max = -65504.f;
  for (int key = lane; key < L; key += 64) {
    const half_t* krow = k + (((int64_t)b * H + h) * L + key) * D;
    int ci = c2p_idx[((int64_t)h * L + query) * L + key];
    int pi = p2c_idx[((int64_t)h * L + key) * L + query];
    if (ci < 0 || ci >= P || pi < 0 || pi >= P) {
      if (error_flag) atomicOr(error_flag, 1);
      ci = ci < 0 ? 0 : (ci >= P ? P - 1 : ci);
      pi = pi < 0 ? 0 : (pi >= P ? P - 1 : pi);
    }
    const half_t* pk = pos_key + ((int64_t)h * P + ci) * D;
    const half_t* pq = pos_query + ((int64_t)h * P + pi) * D;
    float qk = 0.f, c2p = 0.f, p2c = 0.f;
    for (int d = 0; d < D; ++d) {
      const float kd = (float)krow[d];
      qk += qcache[d] * kd;
      c2p += qcache[d] * (float)pk[d];
      p2c += kd * (float)pq[d];
    }
    float score = (qk + c2p + p2c) * scale;
    if ((float)key_mask[(int64_t)b * L + key] < -60000.f) score = -65504.f;
    weights[key] = score;
    local_max = fmaxf(local_max, score);
  }
  const float gmax = wave_max(local_max);
  float local_sum = 0.f;
  for (int key = lane; key < L; key += 64) local_sum += expf(weights[key] - gmax);
  const float gsum = wave_sum(local_sum);
  for (int key = lane; key < L; key += 64) weights[key] = expf(weights[key] - gmax) / gsum;
  __syncthreads();
  for (int d = lane; d < D; d += 64) {
    float acc = 0.f;
    for (int key = 0; key < L; ++key) acc += weights[key] * (float)v[(((int64_t)b * H + h) * L + key) * D + d];
    out[(((int64_t)b * L + query) * H + h) * D + d] = (half_t)acc;
  }
}

__global__ void relative_index_table_kernel(int32_t* __restrict__ out, int n, int bucket_size, int max_position) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < 2 * n - 1) out[i] = relative_index(i - (n - 1), bucket_size, max_position);
}

}  // namespace

int launch_relative_bias_general(const void* q, const void* k, const void* pos_key, const void* pos_query,
                                 const int32_t* c2p, const int32_t* p2c, const void* key_mask, float scale, int64_t B,
                                 int64_t H, int64_t L, int64_t D, int64_t P, void* out, int32_t* error_flag,
                                 hipStream_t stream) {
  if (B * H * L == 0) return GD_OK;
  hipLaunchKernelGGL(relative_bias_general_kernel, dim3((unsigned)(B * H * L)), dim3(64), (size_t)D * sizeof(float),
                     stream, static_cast<const half_t*>(q), static_cast<const half_t*>(k),
                     static_cast<const half_t*>(pos_key), static_cast<const half_t*>(pos_query), c2p, p2c,
                     static_cast<const half_t*>(key_mask), scale, (int)H, (int)L, (int)D, (int)P,
                     static_cast<half_t*>(out), error_flag);
  GD_LAUNCH_CHECK();
  return GD_OK;
}

int launch_fused_attention_general(const void* q, const void* k, const void* v, const void* pos_key,
                                   const void* pos_query, const int32_t* c2p, const int32_t* p2c, const void* key_mask,
                                   float scale, int64_t B, int64_t H, int64_t L, int64_t D, int64_t P, void* out,
                                   int32_t* error_flag, hipStream_t stream) {
  if (B * H * L == 0) return GD_OK;
  hipLaunchKernelGGL(fused_attention_general_kernel, dim3((unsigned)(B * H * L)), dim3(64),
                     (size_t)(D + L) * sizeof(float), stream, static_cast<const half_t*>(q),
                     static_cast<const half_t*>(k), static_cast<const half_t*>(v), static_cast<const half_t*>(pos_key),
                     static_cast<const half_t*>(pos_query), c2p, p2c, static_cast<const half_t*>(key_mask), scale,
                     (int)H, (int)L, (int)D, (int)P, static_cast<half_t*>(out), error_flag);
  GD_LAUNCH_CHECK();
  return GD_OK;
}

int launch_relative_index_table(int32_t* out, int n, int bucket_size, int max_position, hipStream_t stream) {
  const int count = 2 * n - 1;
  hipLaunchKernelGGL(relative_index_table_kernel, dim3((count + 255) / 256), dim3(256), 0, stream, out, n, bucket_size,
                     max_position);
  GD_LAUNCH_CHECK();
  return GD_OK;
}

}  // namespace gd
