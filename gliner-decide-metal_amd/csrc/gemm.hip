// Dense projections of the encoder: C = epilogue(A W^T + b).
//
// Reference: LinearWeight / FusedProjectionWeight (DeBERTa.swift:60-92) --
// MLX addMM(bias, x, W^T) with W stored [out, in] -- and the GELU / ReLU that
// follow the intermediate and classifier projections (DeBERTa.swift:421,437).
//
// gfx950 design.  Both operands are K-contiguous (A is [M, K] row-major, W is
// [N, K] row-major), so every MFMA fragment is one 16-byte row segment, and
// the epilogue adds the bias, rounds to fp16 (the addMM output) and applies
// GELU (the correctly rounded fp16 GELU of that fp16 value, from a table) or
// ReLU -- the two fp16 rounding points of `gelu(linear(x))` in the reference
// graph.  Three kernel families:
//   * gemm_nt_lds_kernel, the main path: tiles from 64 x 64 to 320 x 256 of
//     4 or 8 waves, operands brought into LDS by direct-to-LDS DMA
//     (global_load_lds_dwordx4) two to five 64-deep stages ahead, 128-byte
//     LDS rows with an XOR swizzle (conflict-free ds_read_b128 fragments),
//     v_mfma_f32_32x32x16_f16 with fp32 accumulators, the output staged
//     through LDS into coalesced row segments; gemm_lds_split160_kernel is
//     its 160 x 128 tile on eight waves of unequal row counts (bias
//     epilogues);
//   * gemm_skinny_kernel for at most 32 rows (one short sequence): 32 x 16
//     tiles of two waves on v_mfma_f32_16x16x16_f16, eight 128-deep stages;
//   * gemm_nt_kernel, register-staged (global -> registers -> LDS, one K step
//     ahead): operands whose rows are gathered through an index list (the
//     classifier's marker rows) or that exceed 32-bit element offsets.
// Every kernel accumulates an element over the same 16-wide K slices in the
// same order, so a row's bits do not depend on M or on the kernel chosen.
// launch_linear chooses the kernel and tile: up to 4,096 rows by a cost model
// fitted to a sweep of every tile kernel, above that by rounds of tiles per
// CU weighted by each tile's measured cost.  Workgroups are dispatched
// round-robin over the 8 XCDs; the tile order is remapped so each XCD works
// on a compact 4-tile-row band and its private L2 serves the A rows and W
// columns it shares.
#include <atomic>
#include <cmath>
#include <cstring>
#include <mutex>
#include <type_traits>
#include <vector>

#include "gd_common.hpp"
#include "gd_kernels.hpp"

namespace gd {
namespace {

constexpr int kBK = 64;
constexpr int kThreads = 256;
constexpr int kGroupM = 4;  // tile rows per band of the tile order

// 128-byte LDS rows; the 16-byte chunk index is XORed with bits 1..3 of the
// row.  gfx950's LDS serves ds_read_b128 16 lanes at a time over 64 banks
// (256 B), and a fragment read has 16 consecutive rows at one logical chunk:
// their (row parity, physical chunk) pairs are all distinct -- no conflicts.
__device__ __forceinline__ int lds_swz(int row, int chunk) {
  return row * kBK + ((chunk ^ ((row >> 1) & 7)) << 3);
}

// Logical chunk fetched by lane `lane` of the 1 KiB direct-to-LDS block `blk`
// (8 rows): it lands at physical chunk lane%8 of row 8*blk + lane/8.
__device__ __forceinline__ int dma_chunk(int lane, int blk) {
  return (lane & 7) ^ (((blk & 1) << 2) | (lane >> 4));
}

// ---------------------------------------------------------------------------
// GELU by table.  The GELU epilogue's input is the fp16 addMM output, so its
// correctly rounded fp16 GELU can be looked up: one entry per fp16 value with
// |y| < 8 (exponent field 0..17, both signs: 2 x 18432 entries, 72 KiB),
// computed once per device on the host in double precision through erfc (no
// cancellation in either tail).  |y| >= 8 needs no table: GELU(y) rounds to y
// for y >= 8 and to -0 for y <= -8; y * 0 gives -0, and NaN for -inf / NaN.
// ---------------------------------------------------------------------------
constexpr int kGeluHalf = 18 * 1024;      // entries per sign
constexpr int kGeluEntries = 2 * kGeluHalf;
__device__ __attribute__((aligned(16))) half_t g_gelu_table[kGeluEntries];

// The table may be split over two LDS buffers: entries [0, split) in tab,
// the rest in tab2.
__device__ __forceinline__ half_t gelu_from_table(half_t y, const half_t* tab, const half_t* tab2 = nullptr,
                                                  uint32_t split = kGeluEntries) {
  const uint32_t u = __builtin_bit_cast(uint16_t, y);
  const uint32_t mag = u & 0x7FFFu;
  const uint32_t idx = (u >> 15) * kGeluHalf + (mag < (uint32_t)kGeluHalf ? mag : kGeluHalf - 1);
  const half_t big = (u >> 15) ? (half_t)(y * (half_t)0) : y;
  const half_t* p = idx < split ? tab + idx : tab2 + (idx - split);
  const half_t small = *p;
  return mag < (uint32_t)kGeluHalf ? small : big;
}

// The correctly rounded GELU of every fp16 bit pattern (65,536 entries,
// 128 KiB), filled on the device from the lookup below, so each entry is
// exactly what that lookup returns (NaN payloads included): tiles whose
// stage buffers hold it replace the lookup's arithmetic by one read.
__device__ __attribute__((aligned(16))) half_t g_gelu_full[65536];

// The same lookup in the global copy of the table.
__device__ __forceinline__ half_t gelu_from_global_table(half_t y) {
  const uint32_t u = __builtin_bit_cast(uint16_t, y);
  const uint32_t mag = u & 0x7FFFu;
  const uint32_t idx = (u >> 15) * kGeluHalf + (mag < (uint32_t)kGeluHalf ? mag : kGeluHalf - 1);
  const half_t big = (u >> 15) ? (half_t)(y * (half_t)0) : y;
  const half_t small = g_gelu_table[idx];
  return mag < (uint32_t)kGeluHalf ? small : big;
}

__global__ __launch_bounds__(256) void gelu_full_table_kernel() {
  const int u = blockIdx.x * 256 + threadIdx.x;
  g_gelu_full[u] = gelu_from_global_table(__builtin_bit_cast(half_t, (uint16_t)u));
}

// Epilogue of one output element: the fp16 addMM output (acc + bias rounded
// once), then GELU (the correctly rounded table, here read from global
// memory) or ReLU.  Every kernel gives the same bits for the same element.
template <int EPI>
__device__ __forceinline__ half_t epilogue(float acc, float b) {
  if (EPI == GD_EPI_NONE) return (half_t)acc;
  const half_t y = (half_t)(acc + b);  // addMM output rounding
  if (EPI == GD_EPI_BIAS) return y;
  if (EPI == GD_EPI_BIAS_GELU) return gelu_from_global_table(y);
  // GD_EPI_BIAS_RELU
  return y > (half_t)0 ? y : (half_t)0;
}

// Register-staged tiles: a block of 256 threads (4 waves, 2 x 2) owns a
// BM x BN tile and walks K in steps of 64, global -> registers -> LDS double
// buffered (the loads of step k + 1 in flight while the MFMAs of step k
// run), each wave on a (BM/2) x (BN/2) sub-tile.  With GATHER, A row i is
// row a_rows[i] of the operand (the classifier's marker rows).
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

// ---------------------------------------------------------------------------
// Large-M kernel: 8 waves (two per SIMD), direct global -> LDS loads through an
// NSTAGE-deep pipeline of BK-wide K steps.
//
// Each 1 KiB piece of a stage is fetched with global_load_lds_dwordx4 (64
// lanes x 16 B straight into LDS at M0 + 16*lane), so no VGPRs stage the
// tiles.  The XOR swizzle is applied on the global side: lane l of a block
// fetches the logical chunk that lands, at its physical position, where
// StageLayout::offset() reads it.
//
// Every stage is its own __shared__ array and the K loop is unrolled by
// NSTAGE, so each LDS access names its buffer at compile time.  That is what
// lets the compiler wait only for the DMA into the buffer being read instead
// of for every load in flight (vmcnt(0)); likewise the stage barrier is a bare
// s_barrier behind explicit waits -- __syncthreads() would also drain all
// loads in flight and collapse the pipeline to one stage.
//
// Per K step: the fragments of K slice s+1 are read while the MFMAs of slice
// s run (register double buffering); before the last slice's MFMAs each wave
// waits for its own loads of the next stage, the barrier makes every wave's
// loads visible and frees this stage's buffer, the buffer is refilled with
// the step NSTAGE ahead, and slice 0 of the next stage is read under the
// remaining MFMAs.  The MFMAs take W as the A operand, so a lane's
// accumulators hold four consecutive output columns per group; the epilogue
// stages the fp16 tile through the stage buffers with one conflict-free
// 8-byte store per group and writes coalesced 8-byte row pieces.
// ---------------------------------------------------------------------------

typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ void load_lds16(const half_t* g, half_t* lds_block) {
  __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(g), (lds_void_t*)(lds_block), 16, 0, 0);
}


// LDS layout of one operand tile: rows of BK halfs; the 16-byte chunk index
// is XORed with the row's position inside its 256-byte bank line group, so a
// fragment read (16 consecutive rows, one logical chunk, per ds_read_b128
// pass over gfx950's 64 banks) touches every bank once.
template <int BK>
struct StageLayout {
  static constexpr int kChunks = BK / 8;             // 16-byte chunks per row
  static constexpr int kRowsPer256 = 256 / (BK * 2);  // rows sharing one pass of the banks
  static constexpr int kRowsPerBlock = 1024 / (BK * 2);
  __device__ static __forceinline__ int offset(int row, int chunk) {
    return row * BK + ((chunk ^ ((row / kRowsPer256) & (kChunks - 1))) << 3);
  }
  // Logical chunk that lane `lane` of 1 KiB block `blk` must fetch: the lane
  // writes physical chunk lane % kChunks of row blk * kRowsPerBlock + lane / kChunks.
  __device__ static __forceinline__ int dma_chunk(int lane, int blk) {
    const int row = blk * kRowsPerBlock + lane / kChunks;
    return (lane % kChunks) ^ ((row / kRowsPer256) & (kChunks - 1));
  }
};

template <int V>
using ic = std::integral_constant<int, V>;

template <int BM, int BN, int WAVES_M, int BK, int NSTAGE, int EPI, int NW>
__global__ __launch_bounds__(64 * NW) void gemm_nt_lds_kernel(const half_t* __restrict__ A,
                                                                const half_t* __restrict__ W,
                                                                const half_t* __restrict__ bias,
                                                                half_t* __restrict__ C, int M, int N, int K,
                                                                int64_t lda, int64_t ldc, int tiles_m, int tiles_n) {
  using Lay = StageLayout<BK>;
  constexpr int NT = 64 * NW;  // threads
  constexpr int WAVES_N = NW / WAVES_M;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_BLK = BM / Lay::kRowsPerBlock / NW;  // 1 KiB blocks per wave per stage
  constexpr int B_BLK = BN / Lay::kRowsPerBlock / NW;
  constexpr int LPS = A_BLK + B_BLK;                    // loads per wave per stage
  constexpr int STAGE = (BM + BN) * BK;                 // halfs per stage buffer
  constexpr int S = BK / 16;                            // MFMA K slices per stage
  constexpr int RPA = STAGE / BN / 32 * 32;             // epilogue rows per stage buffer (32-row groups)
  static_assert(TM >= 1 && TN >= 1 && A_BLK >= 1 && B_BLK >= 1, "tile shape");
  static_assert(S % 2 == 0, "fragment sets alternate per slice");
  static_assert(NSTAGE >= 2 && NSTAGE <= 5, "pipeline depth");
  static_assert(NSTAGE * STAGE * 2 <= 160 * 1024, "LDS budget");
  static_assert(RPA % 32 == 0 && (EPI == GD_EPI_BIAS_GELU || NSTAGE * RPA >= BM),
                "epilogue staging must fit in the stage buffers");
  static_assert((NSTAGE - 1) * LPS < 64, "vmcnt range");

  // The GELU epilogue reads the correctly rounded table from LDS: the full
  // 65,536-entry table where the joined stage buffers hold it (below), else
  // the compact one, copied after the K loop into st1 (two stages: st1 sized
  // for all of it; more stages: its first STAGE entries to st1, the rest to
  // st2), with C through st0.  C passes take RPA rows, each wave's WM rows
  // inside one pass (or, where they do not fit one, one 32-row group of every
  // wave row per pass).
  constexpr bool GELU_TABLE = EPI == GD_EPI_BIAS_GELU && (RPA % WM == 0 || WAVES_M * 32 <= RPA) &&
                              (NSTAGE == 2 || 2 * STAGE >= kGeluEntries);
  static_assert(EPI != GD_EPI_BIAS_GELU || GELU_TABLE || NSTAGE * RPA >= BM, "GELU epilogue staging");
  // Tiles whose stage buffers hold 128 KiB (and whose GELU values all fit
  // the registers before C is staged) read the full 65,536-entry table:
  // the stages are then one array, the table lands in it after the K loop.
  // The 320-row tiles stage C one wave row (160 rows) per pass in that array
  // (FFN-up at 4,896 rows 52.4-53.3 -> 51.4-52.7 us against the compact table
  // DMA'd under the last K step; the packed step +1.3%, its FFN-down reading
  // the plainly stored output).
  constexpr int RPF = NSTAGE * STAGE / BN / WM * WM;  // whole wave rows that the joined stages hold
  constexpr bool FULLTAB = GELU_TABLE && NSTAGE * STAGE >= 65536 && (BM == 320 ? RPF >= WM : RPA % WM == 0);
  constexpr int RPP = FULLTAB && BM == 320 ? RPF : RPA;  // C rows per pass of the GELU epilogue
  constexpr int TAB1 = NSTAGE == 2 || kGeluEntries <= STAGE ? kGeluEntries : STAGE;  // entries in st1
  constexpr int kA = FULLTAB ? 16 : 1024;  // alignment of the separate buffers (unused with FULLTAB)
  __shared__ __attribute__((aligned(1024))) half_t stall[FULLTAB ? NSTAGE * STAGE : 8];
  __shared__ __attribute__((aligned(kA))) half_t st0[FULLTAB ? 8 : STAGE];
  __shared__ __attribute__((aligned(kA)))
  half_t st1[FULLTAB ? 8 : (GELU_TABLE && NSTAGE == 2 && kGeluEntries > STAGE ? kGeluEntries : STAGE)];
  __shared__ __attribute__((aligned(kA))) half_t st2[NSTAGE > 2 && !FULLTAB ? STAGE : 8];
  __shared__ __attribute__((aligned(kA))) half_t st3[NSTAGE > 3 && !FULLTAB ? STAGE : 8];
  __shared__ __attribute__((aligned(kA))) half_t st4[NSTAGE > 4 && !FULLTAB ? STAGE : 8];
  auto stage = [&](auto b) -> half_t* {
    constexpr int B = decltype(b)::value;
    if constexpr (FULLTAB) return stall + B * STAGE;
    else if constexpr (B == 0) return st0;
    else if constexpr (B == 1) return st1;
    else if constexpr (B == 2) return st2;
    else if constexpr (B == 3) return st3;
    else return st4;
  };

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
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int lr = lane & 31, lk = lane >> 5;

  // Element offsets of this lane's 16-byte pieces from A and W (fixed across
  // K), 32-bit: the launchers keep both operands within 2^31 elements, so a
  // piece is addressed as the uniform base plus one VGPR.
  uint32_t a_off[A_BLK], b_off[B_BLK];
#pragma unroll
  for (int j = 0; j < A_BLK; ++j) {
    const int blk = wave * A_BLK + j;
    int m = tile_m * BM + blk * Lay::kRowsPerBlock + lane / Lay::kChunks;
    m = m < M ? m : M - 1;
    a_off[j] = (uint32_t)((int64_t)m * lda + Lay::dma_chunk(lane, blk) * 8);
  }
#pragma unroll
  for (int j = 0; j < B_BLK; ++j) {
    const int blk = wave * B_BLK + j;
    const int n = tile_n * BN + blk * Lay::kRowsPerBlock + lane / Lay::kChunks;
    b_off[j] = (uint32_t)((int64_t)n * K + Lay::dma_chunk(lane, blk) * 8);
  }
  auto issue = [&](half_t* st, int k0) {
#pragma unroll
    for (int j = 0; j < A_BLK; ++j) load_lds16(A + (a_off[j] + (uint32_t)k0), st + (wave * A_BLK + j) * 512);
#pragma unroll
    for (int j = 0; j < B_BLK; ++j)
      load_lds16(W + (b_off[j] + (uint32_t)k0), st + BM * BK + (wave * B_BLK + j) * 512);
  };

  float16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Fragment sets: fa[set][i] = A rows of MFMA tile i, fb[set][j] = W rows of tile j.
  half8_t fa[2][TM], fb[2][TN];
  // Every fragment row is wm * WM + i * 32 + lr (or wn * WN + j * 32 + lr),
  // congruent to lr modulo 16, so its swizzle term is the lane's own and
  // Lay::offset(row, 2 s + lk) = row_base * BK + (lane_off ^ 16 s): one lane
  // offset per operand, fragments apart by constants, slices by an XOR.
  static_assert(WM % 16 == 0 && WN % 16 == 0 && 16 % Lay::kRowsPer256 == 0, "fragment address form");
  const int swz = (lr / Lay::kRowsPer256) & (Lay::kChunks - 1);  // the rows' swizzle term
  const int lane_off = lr * BK + 8 * (lk ^ (swz & 1)) + 16 * (swz >> 1);
  const int a_frag0 = wm * WM * BK, b_frag0 = BM * BK + wn * WN * BK;
  auto read_frags = [&](const half_t* st, int slice, int set) {
    const int lo = lane_off ^ (16 * slice);
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[set][i] = *reinterpret_cast<const half8_t*>(st + a_frag0 + i * 32 * BK + lo);
#pragma unroll
    for (int j = 0; j < TN; ++j) fb[set][j] = *reinterpret_cast<const half8_t*>(st + b_frag0 + j * 32 * BK + lo);
  };
  // W rows as the MFMA A operand and A rows as B: lane (lr, lk) of tile (i, j)
  // accumulates C row i * 32 + lr at columns j * 32 + 8 q + 4 lk + e % 4
  // (q = e / 4), four consecutive columns per q.
  auto mma = [&](int set) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = mfma32x32x16(fb[set][j], fa[set][i], acc[i][j]);
  };
  // Issue order of a [read slice s+1][MFMAs of slice s] block: MFMAs and
  // fragment reads alternate from the block's start (an MFMA first, so the
  // wait for slice s's operands covers only reads issued a block earlier),
  // then the remaining MFMAs follow; a sched_barrier closes the block.
  // Without it the scheduler folds the two fragment sets into one and puts
  // an lgkmcnt(0) wait in front of every MFMA group.
  auto interleave = [&]() {
#pragma unroll
    for (int r = 0; r < TM + TN; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one DS read
    }
    if constexpr (TM * TN > TM + TN) __builtin_amdgcn_sched_group_barrier(0x008, TM * TN - (TM + TN), 0);
    __builtin_amdgcn_sched_barrier(0);
  };

  // Every step issues exactly one stage (past the end of K the last K step is
  // fetched again into a buffer nobody reads), so the number of loads in
  // flight behind any stage is a constant and each wait is a plain vmcnt(N).
  const int nk = K / BK;
  const int last_k0 = (nk - 1) * BK;
  auto prologue_issue = [&](auto b) {
    constexpr int B = decltype(b)::value;
    issue(stage(b), min(B * BK, last_k0));
  };
  prologue_issue(ic<0>{});
  prologue_issue(ic<1>{});
  if constexpr (NSTAGE > 2) prologue_issue(ic<2>{});
  if constexpr (NSTAGE > 3) prologue_issue(ic<3>{});
  if constexpr (NSTAGE > 4) prologue_issue(ic<4>{});
  wait_vmcnt<(NSTAGE - 1) * LPS>();  // stage 0 landed
  stage_barrier();
  read_frags(stage(ic<0>{}), 0, 0);

  // One K step on stage buffer B.
  auto step = [&](auto b, int kt) {
    constexpr int B = decltype(b)::value;
#pragma unroll
    for (int s = 0; s + 1 < S; ++s) {
      read_frags(stage(b), s + 1, (s + 1) & 1);
      mma(s & 1);
      interleave();
    }
    // Stage kt + 1 must have landed everywhere; the NSTAGE - 2 stages issued
    // after it may stay in flight.
    wait_vmcnt<(NSTAGE - 2) * LPS>();
    stage_barrier();
    issue(stage(b), min((kt + NSTAGE) * BK, last_k0));
    read_frags(stage(ic<(B + 1) % NSTAGE>{}), 0, 0);  // unused after the last step
    mma((S - 1) & 1);
    interleave();
  };
  // Whole groups of NSTAGE steps run branch-free (a branch between steps
  // would merge waitcnt states and cost a full vmcnt(0) drain); the
  // remaining nk % NSTAGE steps follow the loop.
  int kt = 0;
  for (; kt + NSTAGE <= nk; kt += NSTAGE) {
    step(ic<0>{}, kt);
    step(ic<1>{}, kt + 1);
    if constexpr (NSTAGE > 2) step(ic<2>{}, kt + 2);
    if constexpr (NSTAGE > 3) step(ic<3>{}, kt + 3);
    if constexpr (NSTAGE > 4) step(ic<4>{}, kt + 4);
  }
  if (kt < nk) step(ic<0>{}, kt);
  if constexpr (NSTAGE > 2) if (kt + 1 < nk) step(ic<1>{}, kt + 1);
  if constexpr (NSTAGE > 3) if (kt + 2 < nk) step(ic<2>{}, kt + 2);
  if constexpr (NSTAGE > 4) if (kt + 3 < nk) step(ic<3>{}, kt + 3);
  wait_vmcnt<0>();  // every DMA (the GELU table's too) landed
  __syncthreads();  // all waves done reading the stage buffers

  // ---- epilogue: C tile staged in LDS in rows of BN halfs, 8-byte unit u of
  // row r at unit u ^ (r & 15): a lane's four consecutive columns are one
  // 8-byte store and the 16 rows of a wave's store pass land on 16 distinct
  // units (conflict-free); rows leave as 8-byte pieces, 16 lanes per 128 B.
  constexpr int UPR = BN / 4;  // 8-byte units per row
  static_assert(UPR % 16 == 0, "row swizzle stays inside the row");
  // this lane's unit of tile (j, q) before the swizzle
  auto unit_of = [&](int j, int q) { return (wn * WN + j * 32) / 4 + 2 * q + lk; };
  // bias of this lane's columns
  float bq[TN][4][4];
  if constexpr (EPI != GD_EPI_NONE) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) bq[j][q][e] = (float)bias[tile_n * BN + 4 * unit_of(j, q) + e];
  }
  // rows [row0, row0 + nrows) of the tile, staged at `buf(r)`, to global.
  // Non-temporal stores: the output is read by the next kernel only, and
  // streaming it past the L2 keeps the L2 for the operand tiles that other
  // workgroups still re-read (1-2 us less per launch on the 8,192-row
  // projections, +1% on the whole classify step; the LayerNorm and
  // attention outputs measured slower the same way and keep plain stores).
  // The full-GELU-table tiles are the exception: plain stores take 2.5-3 us
  // off FFN-up at 8,192 rows.
  auto store_rows = [&](int row0, int nrows, auto&& buf) {
#pragma unroll 4
    for (int idx = t; idx < nrows * UPR; idx += NT) {
      const int r = idx / UPR, u = idx - r * UPR;
      const int row = tile_m * BM + row0 + r;
      if (row < M) {
        const half4_t v = *reinterpret_cast<const half4_t*>(buf(r) + 4 * (u ^ (r & 15)));
        half4_t* dst = reinterpret_cast<half4_t*>(C + (int64_t)row * ldc + tile_n * BN + 4 * u);
        if constexpr (FULLTAB) *dst = v;
        else __builtin_nontemporal_store(v, dst);
      }
    }
  };
  if constexpr (GELU_TABLE) {
    // ---- GELU epilogue: the full table in the joined stages, or the
    // compact one in st1 (+ st2), C through st0 in passes ----
    const half_t* tab = FULLTAB ? stall : st1;
    const half_t* tab2 = stage(ic<2 % NSTAGE>{});
    constexpr uint32_t kSplit = TAB1;
    half_t* const cst = FULLTAB ? stall : st0;
    if constexpr (FULLTAB) {
      // the full table by DMA into the stage buffers (all read: the K loop's
      // last barrier), wave w taking 1 KiB blocks w, w + NW, ...
      for (int j = wave; j < 65536 / 512; j += NW) load_lds16(g_gelu_full + j * 512 + lane * 8, stall + j * 512);
      wait_vmcnt<0>();
      __syncthreads();
    } else {
      // All of this thread's table pieces are loaded before any is stored,
      // so the L2 latency is paid once.
      constexpr int kPieces = kGeluEntries / 8;
      constexpr int kPerThread = (kPieces + NT - 1) / NT;
      half8_t piece[kPerThread];
#pragma unroll
      for (int r = 0; r < kPerThread; ++r) {
        const int i = t + r * NT;
        if (i < kPieces) piece[r] = *reinterpret_cast<const half8_t*>(g_gelu_table + 8 * i);
      }
#pragma unroll
      for (int r = 0; r < kPerThread; ++r) {
        const int i = t + r * NT;
        if (i < kPieces)
          *reinterpret_cast<half8_t*>(8 * i < TAB1 ? st1 + 8 * i : stage(ic<2 % NSTAGE>{}) + (8 * i - TAB1)) = piece[r];
      }
      __syncthreads();
    }
    auto gelu_of = [&](int i, int j, int q) {
      half4_t r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const half_t y = (half_t)(acc[i][j][4 * q + e] + bq[j][q][e]);
        if constexpr (FULLTAB)
          r[e] = tab[__builtin_bit_cast(uint16_t, y)];
        else
          r[e] = gelu_from_table(y, tab, tab2, kSplit);
      }
      return r;
    };
    if constexpr (RPP % WM == 0) {
      half4_t res[TM][TN][4];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) res[i][j][q] = gelu_of(i, j, q);
      if constexpr (FULLTAB) __syncthreads();  // every wave's table reads precede the staging writes
      constexpr int NPASS = (BM + RPP - 1) / RPP;
#pragma unroll
      for (int pass = 0; pass < NPASS; ++pass) {
        const int row_lo = wm * WM - pass * RPP;  // this wave's first row within the pass
        if (row_lo >= 0 && row_lo < RPP) {
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
              for (int q = 0; q < 4; ++q)
                *reinterpret_cast<half4_t*>(cst + (row_lo + i * 32 + lr) * BN + 4 * (unit_of(j, q) ^ (lr & 15))) =
                    res[i][j][q];
        }
        __syncthreads();
        const int pass_rows = BM - pass * RPP < RPP ? BM - pass * RPP : RPP;
        store_rows(pass * RPP, pass_rows, [&](int r) { return cst + r * BN; });
        __syncthreads();
      }
    } else {
      // A wave's rows do not fit one pass (the 160- and 192-row tiles with the
      // compact table): pass i takes the
      // i-th 32-row group of every wave row, WAVES_M x 32 rows through st0,
      // its GELU evaluated in the pass.
#pragma unroll
      for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<half4_t*>(cst + (wm * 32 + lr) * BN + 4 * (unit_of(j, q) ^ (lr & 15))) = gelu_of(i, j, q);
        __syncthreads();
#pragma unroll
        for (int g = 0; g < WAVES_M; ++g)
          store_rows(g * WM + i * 32, 32, [&](int r) { return cst + (g * 32 + r) * BN; });
        __syncthreads();
      }
    }
    return;
  }

  // ---- epilogue: bias/activation in registers, fp16 tile staged in LDS ----
  // Rows [p * RPA, (p + 1) * RPA) of the tile go to stage buffer p.
  auto rows_of = [&](int p) -> half_t* {
    half_t* r = st0;
    r = p == 1 ? st1 : r;
    if constexpr (NSTAGE > 2) r = p == 2 ? st2 : r;
    if constexpr (NSTAGE > 3) r = p == 3 ? st3 : r;
    if constexpr (NSTAGE > 4) r = p == 4 ? st4 : r;
    return r;
  };
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int rb = wm * WM + i * 32;  // a 32-row group lies inside one buffer
    half_t* Cs = rows_of(rb / RPA) + (rb % RPA + lr) * BN;
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        half4_t v;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = epilogue<EPI>(acc[i][j][4 * q + e], EPI != GD_EPI_NONE ? bq[j][q][e] : 0.f);
        *reinterpret_cast<half4_t*>(Cs + 4 * (unit_of(j, q) ^ (lr & 15))) = v;
      }
  }
  __syncthreads();
  store_rows(0, BM, [&](int r) { return rows_of(r / RPA) + (r % RPA) * BN; });
}

template <int BM, int BN, int WAVES_M, int BK, int NSTAGE, int NW = 8>
int launch_lds_tile(const half_t* A, const half_t* W, const half_t* bias, half_t* C, int M, int N, int K, int64_t lda,
                    int64_t ldc, int epi, hipStream_t stream) {
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = N / BN;
  const dim3 grid(tiles_m * tiles_n), block(64 * NW);
#define GD_LDS_GEMM(E)                                                                                               \
  hipLaunchKernelGGL((gemm_nt_lds_kernel<BM, BN, WAVES_M, BK, NSTAGE, E, NW>), grid, block, 0, stream, A, W, bias, C, M, N, \
                     K, lda, ldc, tiles_m, tiles_n)
  switch (epi) {
    case GD_EPI_NONE: GD_LDS_GEMM(GD_EPI_NONE); break;
    case GD_EPI_BIAS: GD_LDS_GEMM(GD_EPI_BIAS); break;
    case GD_EPI_BIAS_GELU: GD_LDS_GEMM(GD_EPI_BIAS_GELU); break;
    default: GD_LDS_GEMM(GD_EPI_BIAS_RELU); break;
  }
#undef GD_LDS_GEMM
  GD_LAUNCH_CHECK();
  return GD_OK;
}

// 160 x 128 tiles of eight waves (three 64-deep stages, 108 KiB) for the bias
// epilogues: the rows split unevenly, a wave taking three or two 32-row groups
// of one 32-column strip (rows 0-95 or 96-159), so that every SIMD holds one
// wave of each kind and two waves cover each other's LDS and barrier waits,
// where the four-wave form of the tile has one wave per SIMD.  Stage layout,
// DMA order, fragment reads, K order and epilogue are gemm_nt_lds_kernel's.
template <int EPI>
__global__ __launch_bounds__(512) void gemm_lds_split160_kernel(const half_t* __restrict__ A,
                                                               const half_t* __restrict__ W,
                                                               const half_t* __restrict__ bias,
                                                               half_t* __restrict__ C, int M, int N, int K,
                                                               int64_t lda, int64_t ldc, int tiles_m, int tiles_n) {
  constexpr int BM = 160, BN = 128, BK = 64, NSTAGE = 3, NT = 512;
  using Lay = StageLayout<BK>;
  constexpr int WN = 32, TN = 1;
  constexpr int B_BLK = BN / Lay::kRowsPerBlock / 8;  // 1 KiB W blocks per wave per stage
  constexpr int STAGE = (BM + BN) * BK;
  constexpr int S = BK / 16;
  constexpr int RPA = STAGE / BN / 32 * 32;  // epilogue rows per stage buffer
  static_assert(EPI != GD_EPI_BIAS_GELU, "bias epilogues only");
  static_assert(BM / Lay::kRowsPerBlock == 4 * 3 + 4 * 2 && B_BLK == 2, "A blocks: four waves take 3, four take 2");
  static_assert(NSTAGE * RPA >= BM && RPA % 32 == 0, "epilogue staging must fit in the stage buffers");
  __shared__ __attribute__((aligned(1024))) half_t st0[STAGE];
  __shared__ __attribute__((aligned(1024))) half_t st1[STAGE];
  __shared__ __attribute__((aligned(1024))) half_t st2[STAGE];
  auto stage = [&](auto b) -> half_t* {
    constexpr int B = decltype(b)::value;
    if constexpr (B == 0) return st0;
    else if constexpr (B == 1) return st1;
    else return st2;
  };

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
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wn = wave >> 1;  // column strip
  const int lr = lane & 31, lk = lane >> 5;

  // A wave of TM row groups from row wrow0, its A blocks a_blk0 .. a_blk0 + TM - 1.
  auto run = [&](auto tm_c, const int wrow0, const int a_blk0) {
    constexpr int TM = decltype(tm_c)::value;
    constexpr int A_BLK = TM;
    constexpr int LPS = A_BLK + B_BLK;
    uint32_t a_off[A_BLK], b_off[B_BLK];
#pragma unroll
    for (int j = 0; j < A_BLK; ++j) {
      const int blk = a_blk0 + j;
      int m = tile_m * BM + blk * Lay::kRowsPerBlock + lane / Lay::kChunks;
      m = m < M ? m : M - 1;
      a_off[j] = (uint32_t)((int64_t)m * lda + Lay::dma_chunk(lane, blk) * 8);
    }
#pragma unroll
    for (int j = 0; j < B_BLK; ++j) {
      const int blk = wave * B_BLK + j;
      const int n = tile_n * BN + blk * Lay::kRowsPerBlock + lane / Lay::kChunks;
      b_off[j] = (uint32_t)((int64_t)n * K + Lay::dma_chunk(lane, blk) * 8);
    }
    auto issue = [&](half_t* st, int k0) {
#pragma unroll
      for (int j = 0; j < A_BLK; ++j) load_lds16(A + (a_off[j] + (uint32_t)k0), st + (a_blk0 + j) * 512);
#pragma unroll
      for (int j = 0; j < B_BLK; ++j)
        load_lds16(W + (b_off[j] + (uint32_t)k0), st + BM * BK + (wave * B_BLK + j) * 512);
    };

    float16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][0][e] = 0.f;
    half8_t fa[2][TM], fb[2][TN];
    const int swz = (lr / Lay::kRowsPer256) & (Lay::kChunks - 1);
    const int lane_off = lr * BK + 8 * (lk ^ (swz & 1)) + 16 * (swz >> 1);
    const int a_frag0 = wrow0 * BK, b_frag0 = BM * BK + wn * WN * BK;
    auto read_frags = [&](const half_t* st, int slice, int set) {
      const int lo = lane_off ^ (16 * slice);
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[set][i] = *reinterpret_cast<const half8_t*>(st + a_frag0 + i * 32 * BK + lo);
      fb[set][0] = *reinterpret_cast<const half8_t*>(st + b_frag0 + lo);
    };
    auto mma = [&](int set) {
#pragma unroll
      for (int i = 0; i < TM; ++i) acc[i][0] = mfma32x32x16(fb[set][0], fa[set][i], acc[i][0]);
    };
    auto interleave = [&]() {
#pragma unroll
      for (int r = 0; r < TM + TN; ++r) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one DS read
      }
      __builtin_amdgcn_sched_barrier(0);
    };

    const int nk = K / BK;
    const int last_k0 = (nk - 1) * BK;
    issue(st0, 0);
    issue(st1, min(BK, last_k0));
    issue(st2, min(2 * BK, last_k0));
    wait_vmcnt<(NSTAGE - 1) * LPS>();  // stage 0 landed
    stage_barrier();
    read_frags(st0, 0, 0);
    auto step = [&](auto b, int kt) {
      constexpr int B = decltype(b)::value;
#pragma unroll
      for (int s = 0; s + 1 < S; ++s) {
        read_frags(stage(b), s + 1, (s + 1) & 1);
        mma(s & 1);
        interleave();
      }
      wait_vmcnt<(NSTAGE - 2) * LPS>();
      stage_barrier();
      issue(stage(b), min((kt + NSTAGE) * BK, last_k0));
      read_frags(stage(ic<(B + 1) % NSTAGE>{}), 0, 0);
      mma((S - 1) & 1);
      interleave();
    };
    int kt = 0;
    for (; kt + NSTAGE <= nk; kt += NSTAGE) {
      step(ic<0>{}, kt);
      step(ic<1>{}, kt + 1);
      step(ic<2>{}, kt + 2);
    }
    if (kt < nk) step(ic<0>{}, kt);
    if (kt + 1 < nk) step(ic<1>{}, kt + 1);
    wait_vmcnt<0>();
    __syncthreads();

    // Epilogue as in gemm_nt_lds_kernel: rows [p RPA, (p + 1) RPA) of the
    // tile staged in stage buffer p, 8-byte unit u of row r at u ^ (r & 15).
    constexpr int UPR = BN / 4;
    auto unit_of = [&](int q) { return (wn * WN) / 4 + 2 * q + lk; };
    float bq[4][4];
    if constexpr (EPI != GD_EPI_NONE) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) bq[q][e] = (float)bias[tile_n * BN + 4 * unit_of(q) + e];
    }
    auto rows_of = [&](int p) -> half_t* { return p == 0 ? st0 : (p == 1 ? st1 : st2); };
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int rb = wrow0 + i * 32;
      half_t* Cs = rows_of(rb / RPA) + (rb % RPA + lr) * BN;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        half4_t v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = epilogue<EPI>(acc[i][0][4 * q + e], EPI != GD_EPI_NONE ? bq[q][e] : 0.f);
        *reinterpret_cast<half4_t*>(Cs + 4 * (unit_of(q) ^ (lr & 15))) = v;
      }
    }
    __syncthreads();
#pragma unroll 4
    for (int idx = t; idx < BM * UPR; idx += NT) {
      const int r = idx / UPR, u = idx - r * UPR;
      const int row = tile_m * BM + r;
      if (row < M) {
        const half4_t v = *reinterpret_cast<const half4_t*>(rows_of(r / RPA) + (r % RPA) * BN + 4 * (u ^ (r & 15)));
        __builtin_nontemporal_store(v, reinterpret_cast<half4_t*>(C + (int64_t)row * ldc + tile_n * BN + 4 * u));
      }
    }
  };
  // Waves 0, 2, 5 and 7 take three row groups, 1, 3, 4 and 6 two: waves w
  // and w + 4 share a SIMD (the HW_ID register read on the device), so each
  // SIMD holds one of each (as it would with waves dealt to the SIMDs in
  // pairs).
  if (((wave ^ (wave >> 2)) & 1) == 0) run(ic<3>{}, 0, 5 * wn);
  else run(ic<2>{}, 96, 5 * wn + 3);
}

int launch_lds_split160(const half_t* A, const half_t* W, const half_t* bias, half_t* C, int M, int N, int K,
                        int64_t lda, int64_t ldc, int epi, hipStream_t stream) {
  const int tiles_m = (M + 159) / 160;
  const int tiles_n = N / 128;
  const dim3 grid(tiles_m * tiles_n), block(512);
#define GD_SPLIT_GEMM(E)                                                                                 \
  hipLaunchKernelGGL((gemm_lds_split160_kernel<E>), grid, block, 0, stream, A, W, bias, C, M, N, K, lda, ldc, \
                     tiles_m, tiles_n)
  switch (epi) {
    case GD_EPI_NONE: GD_SPLIT_GEMM(GD_EPI_NONE); break;
    case GD_EPI_BIAS: GD_SPLIT_GEMM(GD_EPI_BIAS); break;
    default: GD_SPLIT_GEMM(GD_EPI_BIAS_RELU); break;
  }
#undef GD_SPLIT_GEMM
  GD_LAUNCH_CHECK();
  return GD_OK;
}

// 320 x 256 tiles (two 64-deep stages, 144 KiB, the full GELU table in them
// after the K loop), GELU epilogue only: one round over up to 320 rows per
// tile row where 256-row tiles need a second.
int launch_lds_tile_gelu320(const half_t* A, const half_t* W, const half_t* bias, half_t* C, int M, int N, int K,
                            int64_t lda, int64_t ldc, hipStream_t stream) {
  const int tiles_m = (M + 319) / 320;
  const int tiles_n = N / 256;
  hipLaunchKernelGGL((gemm_nt_lds_kernel<320, 256, 2, 64, 2, GD_EPI_BIAS_GELU, 8>), dim3(tiles_m * tiles_n), dim3(512),
                     0, stream, A, W, bias, C, M, N, K, lda, ldc, tiles_m, tiles_n);
  GD_LAUNCH_CHECK();
  return GD_OK;
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

// ---------------------------------------------------------------------------
// Skinny products: at most 32 rows (one short sequence, a few marker rows).
// The time of such a product is the chain of dependent MFMAs per accumulator
// (K / 16 of them) plus how fast the workgroups stream W; the tile kernels
// above give N / 64 workgroups with one 32 x 32 accumulator per wave.  Here
// a workgroup of two waves owns a 32 x 16 tile (N / 16 workgroups), wave w
// rows 16 w .. 16 w + 15 in one v_mfma_f32_16x16x16_f16 chain, and keeps
// eight 128-deep stages of A and W in flight (96 KiB).  The 16 x 16 x 16 MFMA
// sums the same 16 products per K slice as the 32 x 32 x 16 form, bit for bit
// (gd_diag_mfma_forms runs both on the device; a GPU test compares them over
// wide-range, cancelling and large-accumulator operands), and the
// slices run in the same order, so each element has the bits the tile
// kernels give it.
//
// Stage layout: rows of 128 halfs (256 B), A rows 0..31 then W rows 32..47;
// the 16-byte chunk index is XORed with the row's low four bits, so the 16
// rows of a fragment read at one logical chunk cover the 64 banks once.
// ---------------------------------------------------------------------------
constexpr int kSkBK = 128;                        // K per stage
constexpr int kSkStages = 8;
constexpr int kSkRows = 48;                       // 32 A rows + 16 W rows
constexpr int kSkStage = kSkRows * kSkBK;         // halfs per stage
constexpr int kSkLoads = kSkStage * 2 / 1024 / 2;  // 1 KiB DMA blocks per wave per stage (6)
static_assert((kSkStages - 1) * kSkLoads < 64, "vmcnt range");

__device__ __forceinline__ int sk_offset(int row, int chunk) { return row * kSkBK + ((chunk ^ (row & 15)) << 3); }

template <int EPI>
__global__ __launch_bounds__(128) void gemm_skinny_kernel(const half_t* __restrict__ A, const half_t* __restrict__ W,
                                                         const half_t* __restrict__ bias, half_t* __restrict__ C,
                                                         int M, int N, int K, int64_t lda, int64_t ldc) {
  // One named array per stage: every LDS read names its buffer at compile
  // time, so the compiler's waits cover only the DMA into that buffer.
  __shared__ __attribute__((aligned(1024))) half_t sk0[kSkStage];
  __shared__ __attribute__((aligned(1024))) half_t sk1[kSkStage];
  __shared__ __attribute__((aligned(1024))) half_t sk2[kSkStage];
  __shared__ __attribute__((aligned(1024))) half_t sk3[kSkStage];
  __shared__ __attribute__((aligned(1024))) half_t sk4[kSkStage];
  __shared__ __attribute__((aligned(1024))) half_t sk5[kSkStage];
  __shared__ __attribute__((aligned(1024))) half_t sk6[kSkStage];
  __shared__ __attribute__((aligned(1024))) half_t sk7[kSkStage];
  static_assert(kSkStages == 8, "one named buffer per stage");
  auto stage = [&](auto b) -> half_t* {
    constexpr int B = decltype(b)::value;
    if constexpr (B == 0) return sk0;
    else if constexpr (B == 1) return sk1;
    else if constexpr (B == 2) return sk2;
    else if constexpr (B == 3) return sk3;
    else if constexpr (B == 4) return sk4;
    else if constexpr (B == 5) return sk5;
    else if constexpr (B == 6) return sk6;
    else return sk7;
  };

  const int tile_n = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int g = lane >> 4, r = lane & 15;

  // This lane's 16-byte pieces: block j of the wave (stage block 6 w + j)
  // holds rows 4 blk .. 4 blk + 3, lane l row 4 blk + l / 16 at physical
  // chunk l % 16, which is logical chunk (l % 16) ^ (row & 15).  Rows past M
  // repeat row M - 1 (never stored).  Offsets in elements, 32-bit.
  uint32_t off[kSkLoads];
  bool is_w[kSkLoads];
#pragma unroll
  for (int j = 0; j < kSkLoads; ++j) {
    const int blk = wave * kSkLoads + j;
    const int row = 4 * blk + (lane >> 4);
    const int chunk = (lane & 15) ^ (row & 15);
    is_w[j] = row >= 32;
    if (row < 32) {
      const int m = row < M ? row : M - 1;
      off[j] = (uint32_t)((int64_t)m * lda + chunk * 8);
    } else {
      off[j] = (uint32_t)((int64_t)(tile_n * 16 + row - 32) * K + chunk * 8);
    }
  }
  auto issue = [&](half_t* st, int k0) {
#pragma unroll
    for (int j = 0; j < kSkLoads; ++j)
      load_lds16((is_w[j] ? W : A) + (off[j] + (uint32_t)k0), st + (wave * kSkLoads + j) * 512);
  };

  // Fragments of K slice s of a stage: lane (g, r) holds k = 16 s + 4 g ..
  // + 3 of A row 16 w + r and of W row r; W is the MFMA A operand, so the
  // lane accumulates C row 16 w + r at columns 4 g .. 4 g + 3 of the tile.
  half4_t fa[2][kSkBK / 16], fw[2][kSkBK / 16];
  auto read_frags = [&](const half_t* st, int set) {
#pragma unroll
    for (int s = 0; s < kSkBK / 16; ++s) {
      const int chunk = 2 * s + (g >> 1), sub = 4 * (g & 1);
      fa[set][s] = *reinterpret_cast<const half4_t*>(st + sk_offset(16 * wave + r, chunk) + sub);
      fw[set][s] = *reinterpret_cast<const half4_t*>(st + sk_offset(32 + r, chunk) + sub);
    }
  };
  float4_t acc = {0.f, 0.f, 0.f, 0.f};

  // Every step issues exactly one stage (past the end of K the last stage is
  // fetched again into a buffer nobody reads), so each wait is a plain
  // vmcnt(N).
  const int nk = K / kSkBK;
  const int last_k0 = (nk - 1) * kSkBK;
  // (the eight buffers as compile-time constants, in order)
  auto each_buffer = [&](auto&& f) {
    f(ic<0>{}), f(ic<1>{}), f(ic<2>{}), f(ic<3>{}), f(ic<4>{}), f(ic<5>{}), f(ic<6>{}), f(ic<7>{});
  };
  each_buffer([&](auto b) { issue(stage(b), min(decltype(b)::value * kSkBK, last_k0)); });
  wait_vmcnt<(kSkStages - 1) * kSkLoads>();  // stage 0 landed
  stage_barrier();
  read_frags(stage(ic<0>{}), 0);

  // Step kt on buffer B: stage kt + 1 landed everywhere and every wave is
  // done with buffer B (its fragments were read a step earlier); B is
  // refilled with stage kt + 8; the fragments of stage kt + 1 are read, and
  // their LDS latency passes under the MFMA chain of stage kt, whose
  // fragments are already in registers.
  auto step = [&](auto b, int kt) {
    constexpr int B = decltype(b)::value;
    wait_vmcnt<(kSkStages - 2) * kSkLoads>();
    stage_barrier();
    issue(stage(b), min((kt + kSkStages) * kSkBK, last_k0));
    read_frags(stage(ic<(B + 1) % kSkStages>{}), (B + 1) & 1);  // unused after the last step
    // (the scheduler would otherwise pull each MFMA up to the fragment read
    // it needs next and wait for that read inside the chain)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < kSkBK / 16; ++s)
      acc = __builtin_amdgcn_mfma_f32_16x16x16f16(fw[B & 1][s], fa[B & 1][s], acc, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  };
  int kt = 0;
  for (; kt + kSkStages <= nk; kt += kSkStages) each_buffer([&](auto b) { step(b, kt + decltype(b)::value); });
  each_buffer([&](auto b) {
    if (kt + decltype(b)::value < nk) step(b, kt + decltype(b)::value);
  });
  wait_vmcnt<0>();  // every DMA landed before the workgroup's LDS is released

  const int row = 16 * wave + r;
  if (row < M) {
    const int col = tile_n * 16 + 4 * g;
    half4_t v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = epilogue<EPI>(acc[e], EPI != GD_EPI_NONE ? (float)bias[col + e] : 0.f);
    *reinterpret_cast<half4_t*>(C + (int64_t)row * ldc + col) = v;
  }
}

int launch_skinny(const half_t* A, const half_t* W, const half_t* bias, half_t* C, int M, int N, int K, int64_t lda,
                  int64_t ldc, int epi, hipStream_t stream) {
  const dim3 grid(N / 16), block(128);
#define GD_SKINNY(E) \
  hipLaunchKernelGGL((gemm_skinny_kernel<E>), grid, block, 0, stream, A, W, bias, C, M, N, K, lda, ldc)
  switch (epi) {
    case GD_EPI_NONE: GD_SKINNY(GD_EPI_NONE); break;
    case GD_EPI_BIAS: GD_SKINNY(GD_EPI_BIAS); break;
    case GD_EPI_BIAS_GELU: GD_SKINNY(GD_EPI_BIAS_GELU); break;
    default: GD_SKINNY(GD_EPI_BIAS_RELU); break;
  }
#undef GD_SKINNY
  GD_LAUNCH_CHECK();
  return GD_OK;
}

// Correctly rounded fp16 GELU of every table entry (host, double precision).
const std::vector<uint16_t>& gelu_table_host() {
  static const std::vector<uint16_t> tab = [] {
    std::vector<uint16_t> v(kGeluEntries);
    for (int sgn = 0; sgn < 2; ++sgn)
      for (int mag = 0; mag < kGeluHalf; ++mag) {
        const uint16_t bits = (uint16_t)((sgn << 15) | mag);
        half_t yh;
        std::memcpy(&yh, &bits, 2);
        const double y = (double)(float)yh;
        const double g = 0.5 * y * std::erfc(-y / std::sqrt(2.0));  // = 0.5 y (1 + erf(y / sqrt 2))
        const half_t gh = (half_t)g;  // round to nearest even
        std::memcpy(&v[sgn * kGeluHalf + mag], &gh, 2);
      }
    return v;
  }();
  return tab;
}

}  // namespace

int ensure_gelu_table(hipStream_t stream) {
  static std::mutex mu;
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
    set_error("the GELU table of device %d is filled on first use, which cannot happen during graph capture: "
              "run one GELU linear (or create the classifier) first", dev);
    return GD_ERR_UNSUPPORTED;
  }
  const std::vector<uint16_t>& tab = gelu_table_host();
  GD_HIP_CHECK(hipMemcpyToSymbol(HIP_SYMBOL(g_gelu_table), tab.data(), tab.size() * sizeof(uint16_t)));
  // the full table from the compact one, before any stream can read it
  hipLaunchKernelGGL(gelu_full_table_kernel, dim3(256), dim3(256), 0, stream);
  GD_LAUNCH_CHECK();
  GD_HIP_CHECK(hipStreamSynchronize(stream));
  ready[dev] = true;
  return GD_OK;
}

namespace {
// Compute units of the current device (cached per device).
int64_t gemm_cu_count() {
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
}  // namespace

namespace {
// Tile choice for up to 4,096 rows: a cost model fitted to a sweep of every
// tile kernel over 160 to 4,096 rows of the encoder's four products (N =
// 1024, 3072, 4096; K = 1024 and 4096; bias and GELU epilogues; one MI355X,
// each choice the measured fastest at every swept point).  A tile kernel
// that holds one workgroup per CU takes ceil(tiles / CUs) rounds of
// a + b K / 1024 (+ g with GELU) us; the 64 x 64 tiles run two workgroups
// per CU, each round after the first adding the fraction `share` of one
// (0.57 at K = 1024, 0.73 at K = 4096).  The 256 x 192 tiles fit N = 3072
// only, so the sweep fixes their cost at K = 1024 alone; their K term is
// scaled like the other 256-row tiles'.  Every kernel accumulates an
// element the same way, so the choice changes no bit.
struct TileCost {
  int bm, bn;
  float a, b, g;
};
constexpr TileCost kTileCosts[] = {
    {64, 64, 3.19f, 3.32f, 1.59f},    {128, 128, 1.53f, 9.37f, 3.39f}, {160, 128, 5.86f, 8.08f, 3.88f},
    {192, 128, 5.63f, 8.79f, 3.20f},  {256, 128, 6.88f, 10.18f, 4.83f}, {256, 192, 10.0f, 12.6f, 4.42f},
    {256, 256, 8.44f, 16.34f, 7.79f},
};

// Index into kTileCosts of the cheapest tile for an M x N x K product.
int cheapest_tile(int M, int N, int K, bool gelu, int64_t cus) {
  int best = 0;
  double best_us = 1e30;
  const double kk = K / 1024.0;
  for (int i = 0; i < (int)(sizeof kTileCosts / sizeof kTileCosts[0]); ++i) {
    const TileCost& t = kTileCosts[i];
    if (N % t.bn) continue;
    const int64_t tiles = (int64_t)((M + t.bm - 1) / t.bm) * (N / t.bn);
    const double rounds = (double)((tiles + cus - 1) / cus);
    const double per = t.a + t.b * kk + (gelu ? t.g : 0.0);
    double us = per * rounds;
    if (t.bm == 64) {
      const double share = K <= 1024 ? 0.57 : (K >= 4096 ? 0.73 : 0.57 + 0.16 * (K - 1024) / 3072.0);
      us = per * (1.0 + share * (rounds - 1.0));
    }
    if (us < best_us) best_us = us, best = i;
  }
  return best;
}
}  // namespace

int launch_linear(const void* a, const void* w, const void* bias, void* c, int64_t m, int64_t n, int64_t k, int64_t lda,
                  int64_t ldc, const int32_t* a_rows, int64_t a_row_count, int epilogue_kind, hipStream_t stream) {
  if (m == 0) return GD_OK;
  if (epilogue_kind == GD_EPI_BIAS_GELU) GD_RETURN_IF_ERROR(ensure_gelu_table(stream));
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
  // The DMA tile kernels address A and W by 32-bit element offsets; larger
  // operands take the register-staged kernel (same accumulation order).
  if ((int64_t)(M - 1) * lda + K >= (int64_t{1} << 31) || (int64_t)N * K >= (int64_t{1} << 31))
    return launch_tile<128, 128, false>(A, Wt, Bv, Cm, M, N, K, lda, ldc, nullptr, 0, epilogue_kind, stream);
  // At most 32 rows: 32 x 16 tiles, one MFMA chain per wave, eight stages in
  // flight.
  if (M <= 32 && N % 16 == 0 && K % kSkBK == 0)
    return launch_skinny(A, Wt, Bv, Cm, M, N, K, lda, ldc, epilogue_kind, stream);
  if (M <= 4096 && N % 128 == 0 && K % 64 == 0) {
    switch (cheapest_tile(M, N, K, epilogue_kind == GD_EPI_BIAS_GELU, gemm_cu_count())) {
      case 0: return launch_lds_tile<64, 64, 2, 64, 4, 4>(A, Wt, Bv, Cm, M, N, K, lda, ldc, epilogue_kind, stream);
      case 1: return launch_lds_tile<128, 128, 2, 64, 2>(A, Wt, Bv, Cm, M, N, K, lda, ldc, epilogue_kind, stream);
      case 2:
        if (epilogue_kind != GD_EPI_BIAS_GELU) return launch_lds_split160(A, Wt, Bv, Cm, M, N, K, lda, ldc, epilogue_kind, stream);
        return launch_lds_tile<160, 128, 1, 64, 3, 4>(A, Wt, Bv, Cm, M, N, K, lda, ldc, epilogue_kind, stream);
      case 3: return launch_lds_tile<192, 128, 2, 64, 3>(A, Wt, Bv, Cm, M, N, K, lda, ldc, epilogue_kind, stream);
      case 4: return launch_lds_tile<256, 128, 4, 64, 3>(A, Wt, Bv, Cm, M, N, K, lda, ldc, epilogue_kind, stream);
      case 5: return launch_lds_tile<256, 192, 4, 64, 2>(A, Wt, Bv, Cm, M, N, K, lda, ldc, epilogue_kind, stream);
      default: return launch_lds_tile<256, 256, 2, 64, 2>(A, Wt, Bv, Cm, M, N, K, lda, ldc, epilogue_kind, stream);
    }
  }
  if (M >= 2048 && N % 256 == 0) {
    // Whole rounds of 256 x 256 tiles (one tile per CU) over the first rows
    // and, when the rows left over fit one round of 128 x 128 tiles and would
    // cost the 256 x 256 launch a further round, those in a second launch: a
    // last round of a few large tiles is slower than one of many small ones
    // (FFN-up at 4,896 rows: 44 + 18.5 us against 71.5 us; with GELU, one
    // round of 320 x 256 tiles: 55.5 us).  Where the rest adds no round
    // (N = 3072 on 32,768 rows: 1,536 tiles, six rounds either way) the
    // second launch only adds its own ramp (212 against 199 us).  Every
    // kernel accumulates in the same order and reads the GELU table.
    const int64_t cus = gemm_cu_count();
    const int64_t m_tiles_round = cus / (N / 256);
    // GELU (FFN-up) on up to 320 rows per tile row: one round of 320 x 256
    // tiles where 256 x 256 tiles would need a second (FFN-up at 4,896 rows).
    if (epilogue_kind == GD_EPI_BIAS_GELU && M > m_tiles_round * 256 && M <= m_tiles_round * 320 && K % 64 == 0)
      return launch_lds_tile_gelu320(A, Wt, Bv, Cm, M, N, K, lda, ldc, stream);
    const int64_t full_rows = m_tiles_round > 0 ? M / (m_tiles_round * 256) * (m_tiles_round * 256) : 0;
    const int64_t rest = M - full_rows;
    auto rounds256 = [&](int64_t rows) { return ((rows + 255) / 256 * (N / 256) + cus - 1) / cus; };
    if (full_rows > 0 && rest > 0 && (rest + 127) / 128 * (N / 128) <= cus && rounds256(full_rows) < rounds256(M)) {
      const int st =
          launch_lds_tile<256, 256, 2, 64, 2>(A, Wt, Bv, Cm, (int)full_rows, N, K, lda, ldc, epilogue_kind, stream);
      if (st != GD_OK) return st;
      return launch_lds_tile<128, 128, 2, 64, 2>(A + full_rows * lda, Wt, Bv, Cm + full_rows * ldc, (int)rest, N, K,
                                                 lda, ldc, epilogue_kind, stream);
    }
  }
  if (M >= 2048) {
    // 256-row tiles: 256 x 256 (two 64-deep stages, 128 KiB of LDS), 256 x 192
    // (two stages, 112 KiB) or 256 x 128 (three stages, 144 KiB), whichever
    // finishes first: rounds of one tile per CU, each costing the tile's
    // measured time per round relative to a 256 x 128 tile (1.5, 1.35, 1; K =
    // 1024 and 4096 alike, from a sweep of every tile kernel over 4,896 to
    // 32,768 rows).  Ties keep the larger tile.
    const int64_t cus = gemm_cu_count();
    auto rounds = [&](int bm, int bn) { return (double)((((M + bm - 1) / bm) * (N / bn) + cus - 1) / cus); };
    // One round of 160 x 128 tiles (three stages, 108 KiB) where it fits:
    // out-proj and FFN-down on up to 5,120 packed rows run 248 tiles instead
    // of 208 larger ones (FFN-down at 4,896 rows 49.6 -> 47.0 us, out-proj
    // 16.2 -> 15.9 us with four waves; eight waves, rows split 96 / 64:
    // out-proj 15.2 us, FFN-down at 2,600 and 3,500 rows 3% less).
    if (epilogue_kind != GD_EPI_BIAS_GELU && N % 128 == 0 && (M + 159) / 160 * (N / 128) <= cus)
      return launch_lds_split160(A, Wt, Bv, Cm, M, N, K, lda, ldc, epilogue_kind, stream);
    int bm = 256, bn = 128;
    double best = rounds(256, 128);
    // 192 x 128 tiles (three stages, 120 KiB) fill a round that 256-row
    // tiles leave part idle (N = 1024 on 5,121 to 6,144 rows: 256 tiles or
    // fewer against 168 to 192), at about 0.8 of a 256 x 128 tile's time.
    if (rounds(192, 128) * 0.8 < best) {
      bm = 192;
      best = rounds(192, 128) * 0.8;
    }
    if (N % 192 == 0 && rounds(256, 192) * 1.35 <= best) {
      bm = 256, bn = 192;
      best = rounds(256, 192) * 1.35;
    }
    if (N % 256 == 0 && rounds(256, 256) * 1.5 <= best) {
      bm = 256, bn = 256;
      best = rounds(256, 256) * 1.5;
    }
    // With GELU, 320 x 256 tiles (two stages, 144 KiB) at about 1.95 of a
    // 256 x 128 tile: FFN-up on 8,193 to 10,240
    // rows takes two rounds of them against three of 256 x 256 (9,500 rows:
    // 105.3 -> 93.6 us).
    if (epilogue_kind == GD_EPI_BIAS_GELU && N % 256 == 0 && rounds(320, 256) * 1.95 < best)
      return launch_lds_tile_gelu320(A, Wt, Bv, Cm, M, N, K, lda, ldc, stream);
    if (bn == 256) return launch_lds_tile<256, 256, 2, 64, 2>(A, Wt, Bv, Cm, M, N, K, lda, ldc, epilogue_kind, stream);
    if (bn == 192) return launch_lds_tile<256, 192, 4, 64, 2>(A, Wt, Bv, Cm, M, N, K, lda, ldc, epilogue_kind, stream);
    if (bm == 192) return launch_lds_tile<192, 128, 2, 64, 3>(A, Wt, Bv, Cm, M, N, K, lda, ldc, epilogue_kind, stream);
    return launch_lds_tile<256, 128, 4, 64, 3>(A, Wt, Bv, Cm, M, N, K, lda, ldc, epilogue_kind, stream);
  }
  // Widths that are a multiple of 64 but not of 128: 64 x 64 DMA-pipelined
  // tiles of four waves with four 64-deep stages in flight (the
  // register-staged kernel keeps one K step in flight, which left a 160-row
  // K = 4096 product waiting on global latency for 55 us).
  if (N % 64 == 0 && K % 64 == 0)
    return launch_lds_tile<64, 64, 2, 64, 4, 4>(A, Wt, Bv, Cm, M, N, K, lda, ldc, epilogue_kind, stream);
  if (M >= 1024) return launch_tile<128, 128, false>(A, Wt, Bv, Cm, M, N, K, lda, ldc, a_rows, (int)a_row_count, epilogue_kind, stream);
  return launch_tile<64, 128, false>(A, Wt, Bv, Cm, M, N, K, lda, ldc, a_rows, (int)a_row_count, epilogue_kind, stream);
}


// ---------------------------------------------------------------------------
// gd_diag_mfma_forms: the two MFMA forms the GEMM kernels use for the same
// 16-product K slice, one 32 x 32 output tile per wave: d32 through one
// v_mfma_f32_32x32x16_f16, d16 through four v_mfma_f32_16x16x16_f16.  The
// skinny GEMM is bit-identical to the tile kernels only if these agree.
// A [t][32][16], W [t][32][16] fp16 (C = A W^T, as in gd_linear), C0 and the
// outputs [t][32][32] fp32, row-major.
// ---------------------------------------------------------------------------
namespace {
__global__ __launch_bounds__(64) void mfma_form32_kernel(const half_t* __restrict__ A, const half_t* __restrict__ W,
                                                        const float* __restrict__ C0, float* __restrict__ D) {
  const int64_t t = blockIdx.x;
  const int l = threadIdx.x;
  const half_t* a = A + t * 512;
  const half_t* w = W + t * 512;
  half8_t fa, fw;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    fa[i] = a[(l & 31) * 16 + 8 * (l >> 5) + i];
    fw[i] = w[(l & 31) * 16 + 8 * (l >> 5) + i];
  }
  float16_t c;
#pragma unroll
  for (int e = 0; e < 16; ++e) c[e] = C0[t * 1024 + (8 * (e >> 2) + 4 * (l >> 5) + (e & 3)) * 32 + (l & 31)];
  c = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa, fw, c, 0, 0, 0);
#pragma unroll
  for (int e = 0; e < 16; ++e) D[t * 1024 + (8 * (e >> 2) + 4 * (l >> 5) + (e & 3)) * 32 + (l & 31)] = c[e];
}

__global__ __launch_bounds__(64) void mfma_form16_kernel(const half_t* __restrict__ A, const half_t* __restrict__ W,
                                                        const float* __restrict__ C0, float* __restrict__ D) {
  const int64_t t = blockIdx.x;
  const int l = threadIdx.x;
  const half_t* a = A + t * 512;
  const half_t* w = W + t * 512;
#pragma unroll
  for (int rm = 0; rm < 2; ++rm)
#pragma unroll
    for (int cn = 0; cn < 2; ++cn) {
      half4_t fa, fw;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        fa[i] = a[(16 * rm + (l & 15)) * 16 + 4 * (l >> 4) + i];
        fw[i] = w[(16 * cn + (l & 15)) * 16 + 4 * (l >> 4) + i];
      }
      float4_t c;
#pragma unroll
      for (int e = 0; e < 4; ++e) c[e] = C0[t * 1024 + (16 * rm + 4 * (l >> 4) + e) * 32 + 16 * cn + (l & 15)];
      c = __builtin_amdgcn_mfma_f32_16x16x16f16(fa, fw, c, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) D[t * 1024 + (16 * rm + 4 * (l >> 4) + e) * 32 + 16 * cn + (l & 15)] = c[e];
    }
}
}  // namespace

int launch_mfma_forms(const void* a, const void* w, const float* c0, float* d32, float* d16, int64_t tiles,
                      hipStream_t stream) {
  if (tiles == 0) return GD_OK;
  hipLaunchKernelGGL(mfma_form32_kernel, dim3((unsigned)tiles), dim3(64), 0, stream, static_cast<const half_t*>(a),
                     static_cast<const half_t*>(w), c0, d32);
  GD_LAUNCH_CHECK();
  hipLaunchKernelGGL(mfma_form16_kernel, dim3((unsigned)tiles), dim3(64), 0, stream, static_cast<const half_t*>(a),
                     static_cast<const half_t*>(w), c0, d16);
  GD_LAUNCH_CHECK();
  return GD_OK;
}

}  // namespace gd
