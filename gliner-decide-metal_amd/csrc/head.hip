// GLiNER classification head around the marker tokens.
//
// Reference: DeBERTa.swift:430-444.  flat = marker_indices + b*L selects the
// marker rows of the final hidden states; classifier.0 (C -> 2048) + ReLU runs
// on MFMA through the row-gathering linear kernel; this file holds the
// index set-up and the last projection classifier.2 (2048 -> 1), whose single
// output column is a dot product per marker row fused with the
// where(marker_mask > 0, v, -10000) select.
#include "gd_common.hpp"
#include "gd_kernels.hpp"

namespace gd {
namespace {

__global__ void marker_rows_kernel(const int32_t* __restrict__ marker_indices, int32_t* __restrict__ rows_out,
                                   int64_t total, int64_t seq_len, int64_t markers_per_row,
                                   int32_t* __restrict__ error_flag, const int32_t* __restrict__ row_off) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t b = i / markers_per_row;
  int64_t m = marker_indices[i];
  if (m < 0 || m >= seq_len) {
    if (error_flag) atomicOr(error_flag, 1);
    m = 0;
  }
  rows_out[i] = (int32_t)((row_off ? (int64_t)row_off[b] : b * seq_len) + m);
}

// One wave per marker row: v = fp16(inner[row] . w2 + b2);
// logits[row] = marker_mask[row] > 0 ? v : -10000.
__global__ __launch_bounds__(256) void head_output_kernel(const half_t* __restrict__ inner, const half_t* __restrict__ w2,
                                                          const half_t* __restrict__ b2,
                                                          const float* __restrict__ marker_mask,
                                                          half_t* __restrict__ logits, int64_t rows, int64_t width) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const half_t* x = inner + row * width;
  float acc = 0.f;
  for (int64_t j = 8 * lane; j < width; j += 512) {
    const half8_t a = *reinterpret_cast<const half8_t*>(x + j);
    const half8_t w = *reinterpret_cast<const half8_t*>(w2 + j);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += (float)a[e] * (float)w[e];
  }
  acc = wave_sum(acc);
  if (lane == 0) {
    const half_t v = (half_t)(acc + (float)b2[0]);
    logits[row] = marker_mask[row] > 0.f ? v : (half_t)-10000.0f;
  }
}

}  // namespace

int launch_marker_rows(const int32_t* marker_indices, int32_t* rows_out, int64_t batch, int64_t seq_len,
                       int64_t markers_per_row, int32_t* error_flag, hipStream_t stream, const int32_t* row_off) {
  const int64_t total = batch * markers_per_row;
  if (total == 0) return GD_OK;
  hipLaunchKernelGGL(marker_rows_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, marker_indices,
                     rows_out, total, seq_len, markers_per_row, error_flag, row_off);
  GD_LAUNCH_CHECK();
  return GD_OK;
}

namespace {
// One thread per 16-byte piece: dst[i, 8c .. 8c + 7] = src[rows[i], ...].
__global__ __launch_bounds__(256) void gather_rows_kernel(const half_t* __restrict__ src,
                                                          const int32_t* __restrict__ rows, int64_t n,
                                                          int64_t src_rows, int64_t pieces,
                                                          half_t* __restrict__ dst) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n * pieces) return;
  const int64_t i = t / pieces, c = t - i * pieces;
  int64_t r = rows[i];
  r = r < 0 ? 0 : (r >= src_rows ? src_rows - 1 : r);
  *reinterpret_cast<half8_t*>(dst + (i * pieces + c) * 8) =
      *reinterpret_cast<const half8_t*>(src + (r * pieces + c) * 8);
}
}  // namespace

int launch_gather_rows(const void* src, const int32_t* rows, int64_t n, int64_t src_rows, int64_t cols, void* dst,
                       hipStream_t stream) {
  if (n <= 0) return GD_OK;
  if (cols % 8 != 0 || src_rows <= 0) return fail(GD_ERR_SHAPE, "gather_rows: cols must be a multiple of 8");
  const int64_t threads = n * (cols / 8);
  hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream,
                     static_cast<const half_t*>(src), rows, n, src_rows, cols / 8, static_cast<half_t*>(dst));
  GD_LAUNCH_CHECK();
  return GD_OK;
}

int launch_head_output(const void* inner, const void* w2, const void* b2, const float* marker_mask, void* logits,
                       int64_t rows, int64_t width, hipStream_t stream) {
  if (rows == 0) return GD_OK;
  hipLaunchKernelGGL(head_output_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream,
                     static_cast<const half_t*>(inner), static_cast<const half_t*>(w2), static_cast<const half_t*>(b2),
                     marker_mask, static_cast<half_t*>(logits), rows, width);
  GD_LAUNCH_CHECK();
  return GD_OK;
}

}  // namespace gd
