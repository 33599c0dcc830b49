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
#include <cstdint>
#include <initializer_list>

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

// ---------------------------------------------------------------------------
// The general-index kernels on the matrix cores (D = 64, L a multiple of 16,
// L <= 512, P <= 65536).  A workgroup of 4 waves owns (b, h, 64 queries),
// wave w queries q0 + 16 w .. + 15, and takes the keys in blocks of 64: the
// relative bias gives each key block a workgroup of its own, the fused
// attention walks all of them.  25 KB of LDS per workgroup; the bias kernel's
// 86 VGPRs let five workgroups share a CU, the fused kernel's 127 (it also
// carries the softmax state and the output) four.  Time follows occupancy:
// the passes below are chains of LDS round trips and barriers.
// For a key block, every pass over 64 positions of the tables computes
// C2P = Q . posK[pass]^T (v_mfma_f32_16x16x32_f16, fp32) into an LDS table
// [query][position], or per 16-key block P2C = K . posQ[pass]^T into a table
// [key][position]; each score takes its two terms from the tables at its
// indices when they fall in the pass.  The c2p passes run before the p2c
// passes, so a score accumulates (x + c2p) + p2c, x = -0 for the bias and
// x = q.k for the fused attention: the reference's fp32 sum, term by term,
// whatever pass a term came from.  Indices outside [0, P) are clamped, as the
// per-query kernels do.
//
// Fused attention: scores (x + c2p + p2c) * scale (masked keys -65504) feed
// an online softmax per query row (running max seeded at -65504, the
// reference's seed), and P . V runs on the matrix cores with P split into
// fp16 hi + lo (V rows in LDS, read transposed by ds_read_b64_tr_b16); the
// output row is divided by the row's sum at the end.
// ---------------------------------------------------------------------------
constexpr int kGenPass = 64;               // table positions per pass
constexpr int kGenStride = kGenPass + 4;   // fp32 row stride: float4 stores of 8 lanes hit 32 distinct banks
// Column kGenPass of every table row holds -0, the term of a position outside
// the pass (x + -0 = x for every fp32 x, signed zeros included).
__device__ __forceinline__ int gen_col(int c) { return (unsigned)c < (unsigned)kGenPass ? c : kGenPass; }
constexpr int kGenKeyBlocks = 4;           // 16-key blocks per key block (64 keys)
// The table-rows buffer also holds the fused kernel's K rows and V rows of a key block.
static_assert(16 * kGenKeyBlocks == kGenPass, "a key block's K / V rows fill the table-rows buffer");

typedef __attribute__((address_space(3))) void gen_lds_void_t;
typedef __attribute__((address_space(3))) half_t gen_lds_half_t;
typedef short gen_short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) gen_short4_t gen_lds_short4_t;

__device__ __forceinline__ int gen_swz(int row, int chunk) { return row * 64 + ((chunk ^ ((row >> 1) & 7)) << 3); }

template <bool FUSED>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(FUSED ? 4 : 5, FUSED ? 4 : 5))) void general_mfma_kernel(
    const half_t* __restrict__ q, const half_t* __restrict__ k, const half_t* __restrict__ v,
    const half_t* __restrict__ pos_key, const half_t* __restrict__ pos_query, const int32_t* __restrict__ c2p_idx,
    const int32_t* __restrict__ p2c_idx, const half_t* __restrict__ key_mask, float scale, int H, int L, int P,
    half_t* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) float tab[64 * kGenStride];          // C2P [query][position]
  __shared__ __attribute__((aligned(16))) half_t rows[kGenPass * 64];          // a pass's table rows (fused: V rows)
  // Workgroup -> (b, h, query block qb, key block ky; the fused kernel takes
  // every key block).  Workgroups go to the 8 XCDs round-robin; with H a
  // multiple of 8, XCD x takes heads x H / 8 .. (x + 1) H / 8 - 1 only, so
  // its L2 holds just those heads' index tensors and position tables.
  constexpr int MAXKB = kGenKeyBlocks;
  const int nqb = (L + 63) / 64, nky = (L / 16 + MAXKB - 1) / MAXKB;
  const int nky_wg = FUSED ? 1 : nky;
  int h, qb, ky, b;
  {
    const int w = blockIdx.x;
    int r;
    if (H % 8 == 0) {
      const int hx = H / 8, l = w >> 3;
      h = (w & 7) * hx + l % hx;
      r = l / hx;
    } else {
      h = w % H;
      r = w / H;
    }
    qb = r % nqb;
    r /= nqb;
    ky = r % nky_wg;
    b = r / nky_wg;
  }
  const int bh = b * H + h;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lc = lane & 15, g = lane >> 4;
  const int qw = qb * 64 + 16 * wave;  // the wave's first query
  const bool active = qw < L;          // uniform
  const int qg = qw + lc;              // this lane's query in the score tile (keys 4 g .. 4 g + 3 of a block)
  const half_t* qbase = q + (int64_t)bh * L * 64;
  const half_t* kbase = k + (int64_t)bh * L * 64;
  const half_t* pkh = pos_key + (int64_t)h * P * 64;
  const half_t* pqh = pos_query + (int64_t)h * P * 64;
  const int32_t* c2ph = c2p_idx + (int64_t)h * L * L;
  const int32_t* p2ch = p2c_idx + (int64_t)h * L * L;
  const half_t* mrow = key_mask + (int64_t)b * L;
  const int qr = qg < L ? qg : L - 1;
  const half8_t qf0 = *reinterpret_cast<const half8_t*>(qbase + (qr * 64 + 8 * g));
  const half8_t qf1 = *reinterpret_cast<const half8_t*>(qbase + (qr * 64 + 32 + 8 * g));
  auto clampi = [&](int x) { return x < 0 ? 0 : (x >= P ? P - 1 : x); };
  auto unpack = [](const uint32_t (&w)[2], int j) -> int { return (int)((w[j >> 1] >> (16 * (j & 1))) & 0xFFFFu); };

  // Steps of a key block: the passes over the posK rows that hold any c2p
  // index of the key block (passes c_lo .. c_lo + nc - 1), then the passes
  // over the posQ rows that hold any of its p2c indices (p_lo .. p_lo + npp
  // - 1); pass p covers table rows [64 p, + 64) (rows past P repeat row
  // P - 1).  A pass holding no index of the block adds nothing, so it is not
  // run (relative-position indices of a 64 x 64 tile span at most 127 rows:
  // 2 or 3 passes of each table instead of all of them).  The fused kernel's
  // last step brings the key block's V rows.  A step's rows are read into
  // registers during the step before.
  __shared__ int pass_range[4][4];  // per wave: least / greatest c2p and p2c index
  int c_lo = 0, nc = 0, p_lo = 0, npp = 0;
  constexpr int kPieces = kGenPass * 8 / 256;  // 16-byte pieces per thread
  half8_t pre[kPieces];
  auto fetch_rows = [&](int step, int ky_) {
#pragma unroll
    for (int it = 0; it < kPieces; ++it) {
      const int i = t + 256 * it;
      const int row = i >> 3, ch = i & 7;
      if (step < nc + npp) {
        const int prow0 = (step < nc ? c_lo + step : p_lo + step - nc) * kGenPass + row;
        const half_t* src = (step < nc ? pkh : pqh) + (prow0 < P ? prow0 : P - 1) * 64;
        pre[it] = *reinterpret_cast<const half8_t*>(src + ch * 8);
      } else {
        // V rows of keys past L are zeros (their probabilities are 0 too)
        const int key = 16 * MAXKB * ky_ + row;
        pre[it] = (half8_t){0, 0, 0, 0, 0, 0, 0, 0};
        if (key < L) pre[it] = *reinterpret_cast<const half8_t*>(v + (int64_t)bh * L * 64 + (key * 64 + ch * 8));
      }
    }
  };

  // fused: running max (per query row, the same in the row's four lanes),
  // this lane's part of the row sum, and O^T (lane: query lc, d 16 dt + 4 g + i)
  float m_run = -65504.f, l_run = 0.f;
  float4_t o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = (float4_t){0.f, 0.f, 0.f, 0.f};

  if (t < 64) tab[t * kGenStride + kGenPass] = -0.0f;  // visible after the first step's barriers
  for (int kyi = 0; kyi < (FUSED ? nky : 1); ++kyi) {  // uniform
    const int kyb = FUSED ? kyi : ky;
    const int kb0 = MAXKB * kyb;  // first 16-key block of this key block
    const int nkb = L / 16 - kb0 < MAXKB ? L / 16 - kb0 : MAXKB;
    // This lane's indices, clamped and packed two per register: c2p of keys
    // 16 kb + 4 g + j at query qg, p2c of query qg at those keys.
    uint32_t c2pk[MAXKB][2], p2ck[MAXKB][2];
    int cmn = P, cmx = -1, pmn = P, pmx = -1;  // this lane's index range (valid scores only)
#pragma unroll
    // L is a multiple of 16, so a wave's queries all exist or none does: `ok`
    // is uniform.  Blocks past nkb and waves past L load the indices of block
    // nkb - 1 / query lc, in bounds and never used.
    for (int kb = 0; kb < MAXKB; ++kb) {
      const bool ok = active && kb < nkb;
      const int kbc = kb < nkb ? kb : nkb - 1, qc = active ? qg : lc;
      int pi[4];
      const int4 ci = *reinterpret_cast<const int4*>(c2ph + (qc * L + 16 * (kb0 + kbc) + 4 * g));
#pragma unroll
      for (int j = 0; j < 4; ++j) pi[j] = p2ch[(16 * (kb0 + kbc) + 4 * g + j) * L + qc];
      const int c[4] = {clampi(ci.x), clampi(ci.y), clampi(ci.z), clampi(ci.w)};
      const int pc[4] = {clampi(pi[0]), clampi(pi[1]), clampi(pi[2]), clampi(pi[3])};
      c2pk[kb][0] = (uint32_t)c[0] | ((uint32_t)c[1] << 16);
      c2pk[kb][1] = (uint32_t)c[2] | ((uint32_t)c[3] << 16);
      p2ck[kb][0] = (uint32_t)pc[0] | ((uint32_t)pc[1] << 16);
      p2ck[kb][1] = (uint32_t)pc[2] | ((uint32_t)pc[3] << 16);
      if (ok) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          cmn = min(cmn, c[j]), cmx = max(cmx, c[j]);
          pmn = min(pmn, pc[j]), pmx = max(pmx, pc[j]);
        }
      }
    }
    // The workgroup's index range: wave reductions, then the four waves'
    // through LDS (the previous key block read pass_range before its steps).
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      cmn = min(cmn, __shfl_xor(cmn, off, 64)), cmx = max(cmx, __shfl_xor(cmx, off, 64));
      pmn = min(pmn, __shfl_xor(pmn, off, 64)), pmx = max(pmx, __shfl_xor(pmx, off, 64));
    }
    if (lane == 0) {
      pass_range[wave][0] = cmn, pass_range[wave][1] = cmx;
      pass_range[wave][2] = pmn, pass_range[wave][3] = pmx;
    }
    __syncthreads();
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      cmn = min(cmn, pass_range[w][0]), cmx = max(cmx, pass_range[w][1]);
      pmn = min(pmn, pass_range[w][2]), pmx = max(pmx, pass_range[w][3]);
    }
    // (wave 0's queries exist and nkb >= 1, so both ranges are non-empty)
    c_lo = __builtin_amdgcn_readfirstlane(cmn / kGenPass);
    nc = __builtin_amdgcn_readfirstlane(cmx / kGenPass) - c_lo + 1;
    p_lo = __builtin_amdgcn_readfirstlane(pmn / kGenPass);
    npp = __builtin_amdgcn_readfirstlane(pmx / kGenPass) - p_lo + 1;
    const int nsteps = nc + npp + (FUSED ? 1 : 0);
    fetch_rows(0, kyb);  // lands during the K loads and q.k
    // K of the key block (keys past L clamped to L - 1).  Each wave keeps
    // the fragments of its p2c keys (16 kb + lc, kb = 4 kg + wave) in
    // registers: the bias kernel loads them from global memory; the fused
    // kernel, whose q.k needs every key in every wave, stages the key block's
    // K rows in the table-rows buffer first (the previous key block's last
    // reads of that buffer, its V rows, came before this block's pass_range
    // barrier; the first step's barrier follows these reads).
    half8_t kp[MAXKB / 4][2];
    float acc[MAXKB][4];
    if constexpr (FUSED) {
#pragma unroll
      for (int it = 0; it < 16 * MAXKB * 8 / 256; ++it) {
        const int i = t + 256 * it;
        const int row = i >> 3, ch = i & 7;
        const int key = 16 * kb0 + row < L ? 16 * kb0 + row : L - 1;
        *reinterpret_cast<half8_t*>(rows + gen_swz(row, ch)) =
            *reinterpret_cast<const half8_t*>(kbase + (key * 64 + ch * 8));
      }
      __syncthreads();  // K rows visible
      // q.k of this wave's queries (lane: query lc, keys 16 kb + 4 g + i)
#pragma unroll
      for (int kb = 0; kb < MAXKB; ++kb) {
        const half8_t kf0 = *reinterpret_cast<const half8_t*>(rows + gen_swz(16 * kb + lc, g));
        const half8_t kf1 = *reinterpret_cast<const half8_t*>(rows + gen_swz(16 * kb + lc, 4 + g));
        float4_t r = {0.f, 0.f, 0.f, 0.f};
        r = mfma16x16x32(kf0, qf0, r);
        r = mfma16x16x32(kf1, qf1, r);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[kb][j] = r[j];
      }
#pragma unroll
      for (int kg = 0; kg < MAXKB / 4; ++kg) {
        kp[kg][0] = *reinterpret_cast<const half8_t*>(rows + gen_swz(16 * (4 * kg + wave) + lc, g));
        kp[kg][1] = *reinterpret_cast<const half8_t*>(rows + gen_swz(16 * (4 * kg + wave) + lc, 4 + g));
      }
    } else {
#pragma unroll
      for (int kg = 0; kg < MAXKB / 4; ++kg) {
        const int key = 16 * (kb0 + 4 * kg + wave) + lc < L ? 16 * (kb0 + 4 * kg + wave) + lc : L - 1;
        kp[kg][0] = *reinterpret_cast<const half8_t*>(kbase + (key * 64 + 8 * g));
        kp[kg][1] = *reinterpret_cast<const half8_t*>(kbase + (key * 64 + 32 + 8 * g));
      }
#pragma unroll
      for (int kb = 0; kb < MAXKB; ++kb)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[kb][j] = -0.0f;
    }

    float* const p2c64 = tab;  // p2c steps: P2C of 64 keys [key][kGenStride] in the C2P table's space
    for (int step = 0; step < nc + npp; ++step) {  // uniform
      __syncthreads();  // the previous step is done with `rows` and the tables
#pragma unroll
      for (int it = 0; it < kPieces; ++it) {
        const int i = t + 256 * it;
        *reinterpret_cast<half8_t*>(rows + gen_swz(i >> 3, i & 7)) = pre[it];
      }
      __syncthreads();
      if (step + 1 < nsteps) fetch_rows(step + 1, kyb);  // lands during this step
      // The packed indices stay packed across steps: unpacking them once,
      // outside the loop, would take 32 more registers.
#pragma unroll
      for (int kb = 0; kb < MAXKB; ++kb) {
        asm volatile("" : "+v"(c2pk[kb][0]), "+v"(c2pk[kb][1]), "+v"(p2ck[kb][0]), "+v"(p2ck[kb][1]));
      }
      const int base = (step < nc ? c_lo + step : p_lo + step - nc) * kGenPass;
      if (step < nc) {
        // ---- c2p: C2P of this wave's queries, gathered by the wave itself ----
        if (active) {
#pragma unroll
          for (int tp = 0; tp < kGenPass / 16; ++tp) {
            const half8_t a0 = *reinterpret_cast<const half8_t*>(rows + gen_swz(16 * tp + lc, g));
            const half8_t a1 = *reinterpret_cast<const half8_t*>(rows + gen_swz(16 * tp + lc, 4 + g));
            float4_t r = {0.f, 0.f, 0.f, 0.f};
            r = mfma16x16x32(a0, qf0, r);
            r = mfma16x16x32(a1, qf1, r);  // lane: query lc, positions 16 tp + 4 g + i
            *reinterpret_cast<float4_t*>(tab + (16 * wave + lc) * kGenStride + 16 * tp + 4 * g) = r;
          }
          wave_lds_sync();
          // Every score gathers a term; one whose position lies outside this
          // pass reads the row's -0 column, which leaves the sum unchanged.
          // (Blocks past nkb gather too, at index 0: their scores are never used.)
          const float* const trow = tab + (16 * wave + lc) * kGenStride;
#pragma unroll
          for (int kb = 0; kb < MAXKB; ++kb)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[kb][j] += trow[gen_col(unpack(c2pk[kb], j) - base)];
        }
      } else {
        // ---- p2c: P2C of 64 keys at a time (wave w: key block 4 kg + w) ----
#pragma unroll
        for (int kg = 0; kg < MAXKB / 4; ++kg) {
          if (4 * kg >= nkb) continue;  // uniform
          {
            // (blocks past nkb hold clamped keys; their P2C rows are never read)
            const half8_t kf0 = kp[kg][0], kf1 = kp[kg][1];
#pragma unroll
            for (int tp = 0; tp < kGenPass / 16; ++tp) {
              const half8_t a0 = *reinterpret_cast<const half8_t*>(rows + gen_swz(16 * tp + lc, g));
              const half8_t a1 = *reinterpret_cast<const half8_t*>(rows + gen_swz(16 * tp + lc, 4 + g));
              float4_t r = {0.f, 0.f, 0.f, 0.f};
              r = mfma16x16x32(a0, kf0, r);
              r = mfma16x16x32(a1, kf1, r);  // lane: key lc, positions 16 tp + 4 g + i
              *reinterpret_cast<float4_t*>(p2c64 + (16 * wave + lc) * kGenStride + 16 * tp + 4 * g) = r;
            }
          }
          __syncthreads();
          if (active) {
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
              for (int j = 0; j < 4; ++j)
                acc[4 * kg + u][j] += p2c64[(16 * u + 4 * g + j) * kGenStride + gen_col(unpack(p2ck[4 * kg + u], j) - base)];
          }
          __syncthreads();
        }
      }
    }

    if constexpr (!FUSED) {
      // ---- scores: (c2p + p2c) * scale, masked keys -65504 ----
      if (active) {  // (uniform: every lane of the wave takes part in the row swaps)
        half_t* orow = out + (int64_t)bh * L * L + qg * L;
        // Lane (g, query lc) holds keys 4 g .. 4 g + 3 of each 16-key block.
        // Per group of four blocks a 4 x 4 transpose across the wave's four
        // 16-lane rows (v_permlane32_swap, then v_permlane16_swap) leaves row
        // g with all 16 keys of block 4 m + g, stored as one 32-byte piece.
#pragma unroll
        for (int m = 0; m < MAXKB / 4; ++m) {
          if (4 * m >= nkb) continue;  // uniform
          uint32_t x[4][2];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int kb = 4 * m + u, kbc = kb < nkb ? kb : nkb - 1;  // blocks past nkb: in bounds, never stored
            const half4_t mk = *reinterpret_cast<const half4_t*>(mrow + 16 * (kb0 + kbc) + 4 * g);
            half4_t sv;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const float sc = acc[kb][j] * scale;
              sv[j] = (float)mk[j] < -60000.f ? (half_t)-65504.f : (half_t)sc;
            }
            const uint2 w = __builtin_bit_cast(uint2, sv);
            x[u][0] = w.x, x[u][1] = w.y;
          }
#pragma unroll
          for (int d = 0; d < 2; ++d) {
            const auto s02 = __builtin_amdgcn_permlane32_swap(x[0][d], x[2][d], false, false);
            const auto s13 = __builtin_amdgcn_permlane32_swap(x[1][d], x[3][d], false, false);
            const uint32_t z0 = s02[0], z2 = s02[1], z1 = s13[0], z3 = s13[1];
            const auto s01 = __builtin_amdgcn_permlane16_swap(z0, z1, false, false);
            const auto s23 = __builtin_amdgcn_permlane16_swap(z2, z3, false, false);
            x[0][d] = s01[0], x[1][d] = s01[1], x[2][d] = s23[0], x[3][d] = s23[1];
          }
          if (4 * m + g < nkb) {
            half_t* dst = orow + 16 * (kb0 + 4 * m + g);
            *reinterpret_cast<uint4*>(dst) = uint4{x[0][0], x[0][1], x[1][0], x[1][1]};
            *reinterpret_cast<uint4*>(dst + 8) = uint4{x[2][0], x[2][1], x[3][0], x[3][1]};
          }
        }
      }
    } else {
      // ---- online softmax over this key block, then P . V ----
      constexpr float kLog2e = 1.4426950408889634f;
      float bmax = m_run;
#pragma unroll
      for (int kb = 0; kb < MAXKB; ++kb) {
        if (kb >= nkb) continue;  // uniform
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int key = 16 * (kb0 + kb) + 4 * g + j;
          const float sc = (float)mrow[key] < -60000.f ? -65504.f : acc[kb][j] * scale;
          acc[kb][j] = sc;
          bmax = fmaxf(bmax, sc);
        }
      }
      bmax = rows_max(bmax);
      // exp(s - m) = 2^(s log2e - m log2e); the rounding of m log2e scales a
      // whole row alike and cancels in the normalisation.
      const float alpha = __builtin_amdgcn_exp2f(m_run * kLog2e - bmax * kLog2e);
      m_run = bmax;
      const float m_l2 = bmax * kLog2e;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
#pragma unroll
      for (int kb = 0; kb < MAXKB; ++kb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float e = kb < nkb ? __builtin_amdgcn_exp2f(fmaf(acc[kb][j], kLog2e, -m_l2)) : 0.f;
          acc[kb][j] = e;
          l_run += e;
        }
      // V step: the key block's V rows into `rows` (every wave's p2c reads
      // of `rows` ended at the last step's closing barrier)
#pragma unroll
      for (int it = 0; it < kPieces; ++it) {
        const int i = t + 256 * it;
        *reinterpret_cast<half8_t*>(rows + gen_swz(i >> 3, i & 7)) = pre[it];
      }
      __syncthreads();
      if (active) {
        // ds_read_b64_tr_b16: in each 16-lane group, source lane s names 4
        // consecutive halfs and lane j receives element j % 4 of source lanes
        // j / 4, 4 + j / 4, 8 + j / 4, 12 + j / 4.  Source lane lc of group g
        // names V[16 T + 4 g + lc / 4][16 dt + 4 (lc % 4) ..], so lane (g, lc)
        // receives V[16 T + 4 g + i][16 dt + lc], i = 0..3 (from 16 rows on,
        // tile T + 1): with V as the A operand and P^T as the B operand the
        // product lane holds O[query lc][16 dt + 4 g + i].  The swizzle term
        // (row >> 1) & 7 of those rows is (2 g + lc / 8) & 7.
        gen_lds_half_t* const rows3 = (gen_lds_half_t*)(gen_lds_void_t*)rows;
        const int tr_sw = (2 * g + (lc >> 3)) & 7;
        const int tr_lane = (4 * g + (lc >> 2)) * 64 + 4 * (lc & 1);
        const int tr_c = (lc >> 1) & 1;
#pragma unroll
        for (int T = 0; T < MAXKB; T += 2) {
          if (T >= nkb) continue;  // uniform; a tile T + 1 past nkb has P = 0 and zero V rows
          half8_t pa, pl;
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
              const float x0 = acc[T + u][i], x1 = acc[T + u][i + 1];
              const half2_t hi = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(x0, x1));
              pa[4 * u + i] = hi[0];
              pa[4 * u + i + 1] = hi[1];
              pl[4 * u + i] = (half_t)(x0 - (float)hi[0]);
              pl[4 * u + i + 1] = (half_t)(x1 - (float)hi[1]);
            }
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) {
            const gen_lds_half_t* a = rows3 + 16 * T * 64 + tr_lane + (((2 * dt + tr_c) ^ tr_sw) << 3);
            const gen_short4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((gen_lds_short4_t*)a);
            const gen_short4_t v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((gen_lds_short4_t*)(a + 16 * 64));
            const half4_t h0 = __builtin_bit_cast(half4_t, v0), h1 = __builtin_bit_cast(half4_t, v1);
            half8_t vb;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              vb[i] = h0[i];
              vb[4 + i] = h1[i];
            }
            o[dt] = mfma16x16x32(vb, pa, o[dt]);
            o[dt] = mfma16x16x32(vb, pl, o[dt]);
          }
        }
      }
      // The next key block writes pass_range and `rows` only after barriers
      // that every wave reaches after its V reads here.
    }
  }
  if constexpr (FUSED) {
    if (active && qg < L) {
      const float inv = 1.0f / rows_sum(l_run);
      half_t* orow = out + (((int64_t)b * L + qg) * H + h) * 64;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        half4_t ov;
#pragma unroll
        for (int i = 0; i < 4; ++i) ov[i] = (half_t)(o[dt][i] * inv);
        *reinterpret_cast<half4_t*>(orow + 16 * dt + 4 * g) = ov;
      }
    }
  }
}

__global__ void relative_index_table_kernel(int32_t* __restrict__ out, int n, int bucket_size, int max_position) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < 2 * n - 1) out[i] = relative_index(i - (n - 1), bucket_size, max_position);
}

// The matrix-core kernels read q, k, v and the table rows in 16-byte pieces,
// the c2p indices and (the bias kernel) the key mask four at a time, and
// store 8- or 16-byte pieces of the output; both entry points hold every
// operand to 16-byte alignment, as the header states.
bool general_mfma_ok(int64_t D, int64_t L, int64_t P, const int32_t* error_flag,
                     std::initializer_list<const void*> ptrs) {
  if (D != 64 || L % 16 != 0 || L > 512 || P > 65536 || error_flag != nullptr) return false;
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return false;
  return true;
}

}  // namespace

int launch_relative_bias_general(const void* q, const void* k, const void* pos_key, const void* pos_query,
                                 const int32_t* c2p, const int32_t* p2c, const void* key_mask, float scale, int64_t B,
                                 int64_t H, int64_t L, int64_t D, int64_t P, void* out, int32_t* error_flag,
                                 hipStream_t stream) {
  if (B * H * L == 0) return GD_OK;
  // Indices travel packed in 16 bits, so the tables hold at most 65536 rows.
  if (general_mfma_ok(D, L, P, error_flag, {q, k, pos_key, pos_query, c2p, p2c, key_mask, out})) {
    const dim3 grid((unsigned)(B * H * ((L + 63) / 64) * ((L / 16 + kGenKeyBlocks - 1) / kGenKeyBlocks)));
    hipLaunchKernelGGL(general_mfma_kernel<false>, grid, dim3(256), 0, stream, static_cast<const half_t*>(q),
                       static_cast<const half_t*>(k), nullptr, static_cast<const half_t*>(pos_key),
                       static_cast<const half_t*>(pos_query), c2p, p2c, static_cast<const half_t*>(key_mask), scale,
                       (int)H, (int)L, (int)P, static_cast<half_t*>(out));
    GD_LAUNCH_CHECK();
    return GD_OK;
  }
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
  // Indices travel packed in 16 bits, so the tables hold at most 65536 rows.
  if (general_mfma_ok(D, L, P, error_flag, {q, k, v, pos_key, pos_query, c2p, p2c, key_mask, out})) {
    const dim3 grid((unsigned)(B * H * ((L + 63) / 64)));
    hipLaunchKernelGGL(general_mfma_kernel<true>, grid, dim3(256), 0, stream, static_cast<const half_t*>(q),
                       static_cast<const half_t*>(k), static_cast<const half_t*>(v),
                       static_cast<const half_t*>(pos_key), static_cast<const half_t*>(pos_query), c2p, p2c,
                       static_cast<const half_t*>(key_mask), scale, (int)H, (int)L, (int)P,
                       static_cast<half_t*>(out));
    GD_LAUNCH_CHECK();
    return GD_OK;
  }
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
