// Dense projections of the encoder: C = epilogue(A W^T + b).
//
// Reference: LinearWeight / FusedProjectionWeight (DeBERTa.swift:60-92) --
// MLX addMM(bias, x, W^T) with W stored [out, in] -- and the GELU / ReLU that
// follow the intermediate and classifier projections (DeBERTa.swift:421,437).
//
// gfx950 design.  Both operands are K-contiguous (A is [M, K] row-major, W is
// [N, K] row-major), so every MFMA fragment is one 16-byte row segment.  A
// block of 256 threads (4 waves, 2 x 2) owns a BM x BN tile and walks K in
// steps of 64:
//   * global -> registers -> LDS, double-buffered: the loads of step k+1 are
//     in flight while the MFMAs of step k run;
//   * LDS rows are 128 B (64 halfs) with the 16-byte chunk index XOR-swizzled
//     by (row & 7), so the fragment reads of 8 consecutive rows hit 8
//     different chunk positions (no bank conflicts on ds_read_b128);
//   * each wave runs v_mfma_f32_32x32x16_f16 over a (BM/2) x (BN/2) sub-tile
//     with fp32 accumulators;
//   * the epilogue adds the bias, rounds to fp16 (the addMM output), applies
//     GELU (exact erf) or ReLU in fp32 and rounds again -- the two fp16
//     rounding points of `gelu(linear(x))` in the reference graph.
//   * workgroups are dispatched round-robin over the 8 XCDs; the tile order is
//     remapped so each XCD works on a compact 4-tile-row band and its private
//     L2 serves the A rows and W columns it shares.
#include "gd_common.hpp"
#include "gd_kernels.hpp"

namespace gd {
namespace {

constexpr int kBK = 64;
constexpr int kThreads = 256;
constexpr int kGroupM = 4;  // tile rows per band of the tile order

__device__ __forceinline__ int lds_swz(int row, int chunk) { return row * kBK + ((chunk ^ (row & 7)) << 3); }

__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f)); }

template <int EPI>
__device__ __forceinline__ half_t epilogue(float acc, float b) {
  if (EPI == GD_EPI_NONE) return (half_t)acc;
  const half_t y = (half_t)(acc + b);  // addMM output rounding
  if (EPI == GD_EPI_BIAS) return y;
  if (EPI == GD_EPI_BIAS_GELU) return (half_t)gelu_erf((float)y);
  // GD_EPI_BIAS_RELU
  return y > (half_t)0 ? y : (half_t)0;
}

template <int BM, int BN, int EPI, bool GATHER>
__global__ __launch_bounds__(kThreads) void gemm_nt_kernel(const half_t* __restrict__ A, const half_t* __restrict__ W,
                                                           const half_t* __restrict__ bias, half_t* __restrict__ C,
                                                           int M, int N, int K, int64_t lda, int64_t ldc,
                                                           const int32_t* __restrict__ a_rows, int a_row_count,
                                                           int tiles_m, int tiles_n) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_IT = BM / 32, B_IT = BN / 32;
  static_assert(TM >= 1 && TN >= 1, "tile too small");
  __shared__ __attribute__((aligned(16))) half_t smem[2 * (BM + BN) * kBK];

  // ---- tile order: XCD-aware band-major mapping ----
  const int nwg = tiles_m * tiles_n;
  int bid = blockIdx.x;
  if ((nwg & 7) == 0) bid = (bid & 7) * (nwg >> 3) + (bid >> 3);
  const int band = bid / (kGroupM * tiles_n);
  const int first_m = band * kGroupM;
  const int gm = min(kGroupM, tiles_m - first_m);
  const int in_band = bid - band * kGroupM * tiles_n;
  const int tile_m = first_m + in_band % gm;
  const int tile_n = in_band / gm;

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lk = lane >> 5;
  const int ld_c = t & 7, ld_r = t >> 3;  // load mapping: chunk, row (0..31)

  // Per-thread source row pointers (fixed across K).
  const half_t* a_src[A_IT];
#pragma unroll
  for (int i = 0; i < A_IT; ++i) {
    int m = tile_m * BM + ld_r + 32 * i;
    m = m < M ? m : M - 1;
    int64_t src = m;
    if (GATHER) {
      src = a_rows[m];
      src = src < 0 ? 0 : (src >= a_row_count ? a_row_count - 1 : src);
    }
    a_src[i] = A + src * lda + ld_c * 8;
  }
  const half_t* b_src[B_IT];
#pragma unroll
  for (int i = 0; i < B_IT; ++i) b_src[i] = W + (int64_t)(tile_n * BN + ld_r + 32 * i) * K + ld_c * 8;

  half8_t ra[A_IT], rb[B_IT];
  auto load_regs = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_IT; ++i) ra[i] = *reinterpret_cast<const half8_t*>(a_src[i] + k0);
#pragma unroll
    for (int i = 0; i < B_IT; ++i) rb[i] = *reinterpret_cast<const half8_t*>(b_src[i] + k0);
  };
  auto store_lds = [&](int buf) {
    half_t* As = smem + buf * (BM + BN) * kBK;
    half_t* Bs = As + BM * kBK;
#pragma unroll
    for (int i = 0; i < A_IT; ++i) *reinterpret_cast<half8_t*>(As + lds_swz(ld_r + 32 * i, ld_c)) = ra[i];
#pragma unroll
    for (int i = 0; i < B_IT; ++i) *reinterpret_cast<half8_t*>(Bs + lds_swz(ld_r + 32 * i, ld_c)) = rb[i];
  };

  float16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int nk = K / kBK;
  load_regs(0);
  store_lds(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) load_regs((kt + 1) * kBK);
    const half_t* As = smem + (kt & 1) * (BM + BN) * kBK;
    const half_t* Bs = As + BM * kBK;
#pragma unroll
    for (int s = 0; s < kBK / 16; ++s) {
      half8_t fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        fa[i] = *reinterpret_cast<const half8_t*>(As + lds_swz(wm * WM + i * 32 + lr, 2 * s + lk));
#pragma unroll
      for (int j = 0; j < TN; ++j)
        fb[j] = *reinterpret_cast<const half8_t*>(Bs + lds_swz(wn * WN + j * 32 + lr, 2 * s + lk));
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma32x32x16(fa[i], fb[j], acc[i][j]);
    }
    if (kt + 1 < nk) store_lds((kt + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue ----
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int col = tile_n * BN + wn * WN + j * 32 + lr;
    const float b = (EPI != GD_EPI_NONE) ? (float)bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row0 = tile_m * BM + wm * WM + i * 32 + 4 * lk;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = row0 + 8 * (e >> 2) + (e & 3);
        if (row < M) C[(int64_t)row * ldc + col] = epilogue<EPI>(acc[i][j][e], b);
      }
    }
  }
}

template <int BM, int BN, bool GATHER>
int launch_tile(const half_t* A, const half_t* W, const half_t* bias, half_t* C, int M, int N, int K, int64_t lda,
                int64_t ldc, const int32_t* a_rows, int a_row_count, int epi, hipStream_t stream) {
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = N / BN;
  const dim3 grid(tiles_m * tiles_n), block(kThreads);
  switch (epi) {
    case GD_EPI_NONE:
      hipLaunchKernelGGL((gemm_nt_kernel<BM, BN, GD_EPI_NONE, GATHER>), grid, block, 0, stream, A, W, bias, C, M, N, K,
                         lda, ldc, a_rows, a_row_count, tiles_m, tiles_n);
      break;
    case GD_EPI_BIAS:
      hipLaunchKernelGGL((gemm_nt_kernel<BM, BN, GD_EPI_BIAS, GATHER>), grid, block, 0, stream, A, W, bias, C, M, N, K,
                         lda, ldc, a_rows, a_row_count, tiles_m, tiles_n);
      break;
    case GD_EPI_BIAS_GELU:
      hipLaunchKernelGGL((gemm_nt_kernel<BM, BN, GD_EPI_BIAS_GELU, GATHER>), grid, block, 0, stream, A, W, bias, C, M,
                         N, K, lda, ldc, a_rows, a_row_count, tiles_m, tiles_n);
      break;
    default:
      hipLaunchKernelGGL((gemm_nt_kernel<BM, BN, GD_EPI_BIAS_RELU, GATHER>), grid, block, 0, stream, A, W, bias, C, M,
                         N, K, lda, ldc, a_rows, a_row_count, tiles_m, tiles_n);
      break;
  }
  GD_LAUNCH_CHECK();
  return GD_OK;
}

}  // namespace

int launch_linear(const void* a, const void* w, const void* bias, void* c, int64_t m, int64_t n, int64_t k, int64_t lda,
                  int64_t ldc, const int32_t* a_rows, int64_t a_row_count, int epilogue_kind, hipStream_t stream) {
  if (m == 0) return GD_OK;
  auto A = static_cast<const half_t*>(a);
  auto Wt = static_cast<const half_t*>(w);
  auto Bv = static_cast<const half_t*>(bias);
  auto Cm = static_cast<half_t*>(c);
  const int M = (int)m, N = (int)n, K = (int)k;
  // Tile choice: 256-row tiles once there are enough rows to fill the chip,
  // smaller tiles for short inputs (classifier head, short buckets).
  if (a_rows) {
    if (M >= 1024) return launch_tile<128, 128, true>(A, Wt, Bv, Cm, M, N, K, lda, ldc, a_rows, (int)a_row_count, epilogue_kind, stream);
    return launch_tile<64, 128, true>(A, Wt, Bv, Cm, M, N, K, lda, ldc, a_rows, (int)a_row_count, epilogue_kind, stream);
  }
  if (M >= 4096) return launch_tile<256, 128, false>(A, Wt, Bv, Cm, M, N, K, lda, ldc, a_rows, (int)a_row_count, epilogue_kind, stream);
  if (M >= 1024) return launch_tile<128, 128, false>(A, Wt, Bv, Cm, M, N, K, lda, ldc, a_rows, (int)a_row_count, epilogue_kind, stream);
  return launch_tile<64, 128, false>(A, Wt, Bv, Cm, M, N, K, lda, ldc, a_rows, (int)a_row_count, epilogue_kind, stream);
}

}  // namespace gd
