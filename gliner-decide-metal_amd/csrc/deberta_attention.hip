// Per-forward helper kernels of the attention (row extents, the item
// schedule, packed-row offsets), the relative index table the attention
// kernel reads, and the dispatch of launch_deberta_attention over the score
// modes (each instantiated in its own attention_sm_*.hip).
#include <algorithm>
#include <atomic>
#include <climits>
#include <cmath>
#include <mutex>
#include <type_traits>
#include "gd_common.hpp"
#include "gd_kernels.hpp"

namespace gd {

// Compute units of the current device (cached per device).
int device_cu_count() {
  static std::atomic<int> cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

namespace {

constexpr int kWaves = 8;
constexpr int kQT = 128;
// idx(r) for every r in [-511, 511] at bucket size 256 and 512 positions,
// filled once per device (ensure_relative_index_table) by relative_index().
constexpr int kRelSpan = 511;
__device__ __attribute__((aligned(16))) int16_t g_rel_idx[2 * kRelSpan + 1];

__global__ void fill_relative_index_kernel() {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < 2 * kRelSpan + 1) g_rel_idx[i] = (int16_t)relative_index(i - kRelSpan, 256, 512);
}

// One workgroup (4 waves) per batch row.  Without a mask: the marker part
// only (the query extent).
__global__ __launch_bounds__(256) void row_extent_kernel(const half_t* __restrict__ mask,
                                                         const int32_t* __restrict__ markers,
                                                         const float* __restrict__ marker_mask, int L, int slots,
                                                         int32_t* __restrict__ out) {
  const int b = blockIdx.x;
  int ext = 0;
  if (mask != nullptr)
    for (int l = threadIdx.x; l < L; l += 256)
      if ((float)mask[(int64_t)b * L + l] > 0.f) ext = l + 1;  // l grows: the last hit is the largest
  for (int s = threadIdx.x; s < slots; s += 256)
    if (marker_mask[(int64_t)b * slots + s] > 0.f) {
      const int p = markers[(int64_t)b * slots + s];
      const int e = (p >= 0 && p < L) ? p + 1 : 1;
      ext = e > ext ? e : ext;
    }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const int o = __shfl_xor(ext, off, 64);
    ext = o > ext ? o : ext;
  }
  __shared__ int wave_max[4];
  if ((threadIdx.x & 63) == 0) wave_max[threadIdx.x >> 6] = ext;
  __syncthreads();
  if (threadIdx.x == 0) {
    int m = wave_max[0];
    for (int w = 1; w < 4; ++w) m = wave_max[w] > m ? wave_max[w] : m;
    out[b] = m;
  }
}

// Item schedule of the persistent attention under row extents (L <= 256,
// one workgroup per CU, G workgroups).  Items differ in cost (chunks up to
// the extent, active waves), so the (b, h) pairs are ranked by their cost
// (largest first; equal costs by index) and dealt in rounds of G / 2 over CU
// pairs (w, w + 8: one XCD), snaking (odd rounds run the pairs backwards),
// each pair's two query tiles side by side (swapped on odd rounds); with one
// query tile, items are dealt over all G workgroups the same way.  sched[w +
// r G] = bh * ntq + qt is workgroup w's item of round r, -1 where a round has
// no item.  Costs, in thousandths of a full chunk: 1000 per chunk with two
// waves per SIMD active, 775 with one, plus 600 for the tail.
__device__ __forceinline__ int attention_item_cost(int len, int qt) {
  const int q0 = qt * kQT;
  if (q0 >= len) return 50;
  const int nch = (((len + 15) >> 4) + 3) >> 2;
  const int active = min(kWaves, (len - q0 + 15) >> 4);
  return nch * (active > 4 ? 1000 : 775) + 600;
}

constexpr int kSchedMaxPairs = 2048;

__global__ __launch_bounds__(1024) void attention_schedule_kernel(const int32_t* __restrict__ row_len, int B, int H,
                                                                  int L, int G, int32_t* __restrict__ sched,
                                                                  int n_slots) {
  // An item's cost depends on its batch row only, so the rank of pair
  // i = b H + h in the order (cost descending, index ascending) over all
  // B H pairs is H (rows of higher cost + earlier rows of equal cost) + h.
  __shared__ int cost[kSchedMaxPairs];
  const int t = threadIdx.x;
  const int ntq = (L + kQT - 1) / kQT;
  const int n = B * H;
  for (int b = t; b < B; b += 1024) {
    const int len = row_len[b];
    int c = 0;
    for (int qt = 0; qt < ntq; ++qt) c += attention_item_cost(len, qt);
    cost[b] = c;
  }
  for (int s = t; s < n_slots; s += 1024) sched[s] = -1;
  __syncthreads();  // costs complete; the -1 stores land before any item store below
  for (int i = t; i < n; i += 1024) {
    const int b = i / H;
    const int cb = cost[b];
    int before = 0;
    for (int j = 0; j < B; ++j) {
      const int cj = cost[j];
      before += (cj > cb) || (cj == cb && j < b);
    }
    const int rank = before * H + (i - b * H);
    if (ntq == 2) {
      const int P = G >> 1;  // CU pairs
      const int r = rank / P, pp = rank - r * P;
      const int p = (r & 1) ? P - 1 - pp : pp;
      const int w0 = (p & 7) | ((p >> 3) << 4), w1 = w0 | 8;
      const int qa = r & 1;
      sched[w0 + r * G] = i * 2 + qa;
      sched[w1 + r * G] = i * 2 + (1 - qa);
    } else {
      const int r = rank / G, pp = rank - r * G;
      sched[((r & 1) ? G - 1 - pp : pp) + r * G] = i;
    }
  }
}

// One workgroup per batch row b: its offset is the sum of the extents before
// it (B is a batch size, so the O(B^2) reads are few).
__global__ __launch_bounds__(256) void pack_rows_kernel(const int32_t* __restrict__ row_len, int B, int L,
                                                        int64_t total, int exact, int32_t* __restrict__ row_off,
                                                        int32_t* __restrict__ row_map,
                                                        int32_t* __restrict__ error_flag) {
  const int b = blockIdx.x;
  int part = 0;
  for (int i = threadIdx.x; i < b; i += 256) part += row_len[i];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off, 64);
  __shared__ int wave_sum[4];
  if ((threadIdx.x & 63) == 0) wave_sum[threadIdx.x >> 6] = part;
  __syncthreads();
  const int64_t off = (int64_t)wave_sum[0] + wave_sum[1] + wave_sum[2] + wave_sum[3];
  const int len = row_len[b];
  if (threadIdx.x == 0) {
    row_off[b] = (int32_t)off;
    if (b == B - 1) {
      row_off[B] = (int32_t)(off + len);
      if ((exact ? off + len != total : off + len > total) && error_flag) atomicOr(error_flag, 1);
    }
  }
  for (int l = threadIdx.x; l < len; l += 256)
    if (off + l < total) row_map[off + l] = b * L + l;
  if (b == B - 1)  // rows past the extents (a capacity above their sum) embed token 0
    for (int64_t t = off + len + threadIdx.x; t < total; t += 256) row_map[t] = 0;
}

}  // namespace

int launch_row_extent(const void* mask, const int32_t* markers, const float* marker_mask, int64_t B, int64_t L,
                      int64_t slots, int32_t* out, hipStream_t stream) {
  if (B <= 0) return GD_OK;
  hipLaunchKernelGGL(row_extent_kernel, dim3((unsigned)B), dim3(256), 0, stream, static_cast<const half_t*>(mask),
                     markers, marker_mask, (int)L, (int)slots, out);
  GD_LAUNCH_CHECK();
  return GD_OK;
}

int launch_query_extent(const int32_t* markers, const float* marker_mask, int64_t B, int64_t L, int64_t slots,
                        int32_t* out, hipStream_t stream) {
  if (B <= 0) return GD_OK;
  hipLaunchKernelGGL(row_extent_kernel, dim3((unsigned)B), dim3(256), 0, stream, nullptr, markers, marker_mask,
                     (int)L, (int)slots, out);
  GD_LAUNCH_CHECK();
  return GD_OK;
}

int launch_pack_rows(const int32_t* row_len, int64_t B, int64_t L, int64_t total, bool exact, int32_t* row_off,
                     int32_t* row_map, int32_t* error_flag, hipStream_t stream) {
  if (B <= 0) return GD_OK;
  hipLaunchKernelGGL(pack_rows_kernel, dim3((unsigned)B), dim3(256), 0, stream, row_len, (int)B, (int)L, total,
                     exact ? 1 : 0, row_off, row_map, error_flag);
  GD_LAUNCH_CHECK();
  return GD_OK;
}

namespace {
std::mutex g_rel_mu;
const int16_t* g_rel_ptr[64] = {};  // device address of g_rel_idx, per device, once filled
}  // namespace

int ensure_relative_index_table(hipStream_t stream) {
  auto& mu = g_rel_mu;
  static bool ready[64] = {};
  int dev = 0;
  GD_HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) {
    set_error("device index %d out of range", dev);
    return GD_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (ready[dev]) return GD_OK;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (stream && hipStreamIsCapturing(stream, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone) {
    set_error("the relative index table of device %d is filled on first use, which cannot happen during graph "
              "capture: run one attention call (or create the classifier) first", dev);
    return GD_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL(fill_relative_index_kernel, dim3((2 * kRelSpan + 1 + 255) / 256), dim3(256), 0, stream);
  GD_LAUNCH_CHECK();
  GD_HIP_CHECK(hipStreamSynchronize(stream));  // visible to every stream from here on
  // The kernels that read the table live in other translation units: they
  // take its device address (this device's copy) as an argument.
  void* addr = nullptr;
  GD_HIP_CHECK(hipGetSymbolAddress(&addr, HIP_SYMBOL(g_rel_idx)));
  g_rel_ptr[dev] = static_cast<const int16_t*>(addr);
  ready[dev] = true;
  return GD_OK;
}

int relative_index_table_device(const int16_t** out, hipStream_t stream) {
  GD_RETURN_IF_ERROR(ensure_relative_index_table(stream));
  int dev = 0;
  GD_HIP_CHECK(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_rel_mu);
  *out = g_rel_ptr[dev];
  return *out ? GD_OK : fail(GD_ERR_HIP, "relative index table has no device address");
}

int attention_schedule_slots(int64_t B, int64_t H, int64_t L) {
  const int64_t ntq = (L + kQT - 1) / kQT;
  const int64_t items = B * H * ntq;
  const int64_t G = items < device_cu_count() ? items : device_cu_count();
  if (L > 256 || ntq > 2 || B * H > kSchedMaxPairs || G % 16 != 0) return 0;
  return (int)((items + G - 1) / G * G);
}

int launch_attention_schedule(const int32_t* row_len, int64_t B, int64_t H, int64_t L, int32_t* sched,
                              hipStream_t stream) {
  const int n_slots = attention_schedule_slots(B, H, L);
  if (n_slots == 0) return GD_OK;
  const int64_t items = B * H * ((L + kQT - 1) / kQT);
  const int G = (int)(items < device_cu_count() ? items : device_cu_count());
  hipLaunchKernelGGL(attention_schedule_kernel, dim3(1), dim3(1024), 0, stream, row_len, (int)B, (int)H, (int)L, G,
                     sched, n_slots);
  GD_LAUNCH_CHECK();
  return GD_OK;
}

int launch_deberta_attention(const AttentionArgs& a, hipStream_t stream) {
  if (a.bucket_size != 256 || a.P != 512) return fail(GD_ERR_SHAPE, "attention: bucket size 256 and 512 positions");
  if (a.row_len != nullptr && a.output != GD_ATTN_OUT_CONTEXT)
    return fail(GD_ERR_INVALID_ARGUMENT, "attention: row extents apply to the context output only");
  if (a.row_off != nullptr && a.row_len == nullptr)
    return fail(GD_ERR_INVALID_ARGUMENT, "attention: packed rows need row extents");
  if (a.q_len != nullptr && a.row_len == nullptr)
    return fail(GD_ERR_INVALID_ARGUMENT, "attention: query extents need row extents");
  if (a.sched != nullptr && (a.row_len == nullptr || a.n_sched != attention_schedule_slots(a.B, a.H, a.L)))
    return fail(GD_ERR_INVALID_ARGUMENT, "attention: schedule does not match the launch");
  for (int64_t st : {a.qsb, a.qsh, a.qsl, a.ksb, a.ksh, a.ksl, a.vsb, a.vsh, a.vsl, a.pksh, a.pksp, a.pqsh, a.pqsp, a.ldo})
    if (st < 0 || st > INT32_MAX) return fail(GD_ERR_SHAPE, "attention: strides must lie in [0, 2^31)");
  // the stage loads address a table row by its 32-bit byte offset from the head's first row
  if (((a.P - 1) * std::max(a.pksp, a.pqsp) + 64) * 2 > INT32_MAX)
    return fail(GD_ERR_SHAPE, "attention: position-table rows must lie within 2 GiB of a head's first row");
  if (a.output != GD_ATTN_OUT_PROBS && a.output != GD_ATTN_OUT_CONTEXT && a.output != GD_ATTN_OUT_BIAS)
    return fail(GD_ERR_INVALID_ARGUMENT, "attention: unknown output kind");
  if (a.output == GD_ATTN_OUT_BIAS && a.score != kScoreDefault && a.score != kScoreKernelBias)
    return fail(GD_ERR_INVALID_ARGUMENT, "attention: the bias output exists for the default and the kernel-bias "
                                         "score chains only (the others add no bias of their own)");
  AttentionArgs b = a;
  GD_RETURN_IF_ERROR(relative_index_table_device(&b.rel_idx, stream));
  switch (a.score) {
    case kScoreDefault:
      return launch_attention_default(b, stream);
    case kScoreExplicit:
      return launch_attention_explicit(b, stream);
    case kScoreKernelBias:
    case kScoreKernelBiasExplicit:
      return launch_attention_kernel_bias(b, stream);
    case kScoreFused:
      return launch_attention_fused(b, stream);
    default:
      return fail(GD_ERR_INVALID_ARGUMENT, "attention: unknown score chain");
  }
}

}  // namespace gd
