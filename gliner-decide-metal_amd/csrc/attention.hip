// Disentangled attention of the DeBERTa-v3 encoder.
//
// Reference:
//   default graph  DeBERTa.swift:322-395 (relative bias from c2pRaw/p2cRaw
//                  gathers, additive key mask, MLX fused SDPA) and the index
//                  math DeBERTa.swift:498-551;
//   Metal kernels  FusedKernels.swift:13-81 (fused attention) and :83-123
//                  (relative bias), launched at :160-258.
//
// ---------------------------------------------------------------------------
// deberta_attention_kernel (the hot path)
// ---------------------------------------------------------------------------
// One workgroup = (batch b, head h, 64 queries), 4 waves of 16 queries each.
// Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_16x16x32_f16,
// so every lane ends up owning ONE query column (q = lane % 16) and 4
// consecutive keys per 16-key tile: row reductions of the softmax are
// in-register plus two cross-lane steps, and the probabilities are already in
// the A-operand layout of the P.V MFMA (the contraction index may be any
// bijection shared by both operands, so no LDS round trip for P).
//
// The relative bias uses the band structure of idx(q,k) = clip(bucket(q-k) +
// 256, 0, 511), which depends on q - k only and is monotone in it:
//   c2p  For the wave's 16 queries and ALL keys, the indices needed form one
//        contiguous window [idx(q0-L+1), idx(q0+15)]; its width is ~L+15 in
//        the linear zone but the log buckets compress it (<= 271 at L = 256),
//        so C2P = posK[window] . Q^T costs ~1.06x the direct dot products.
//        It is computed once per wave on MFMA and parked in LDS as fp16 --
//        exactly the reference's fp16 c2pRaw.
//   p2c  For one 16-key tile and the wave's 16 queries the window has <= 31
//        positions (2 MFMA column tiles): P2C = K_tile . posQ[window]^T, fp16
//        into a small per-wave LDS tile (the reference's fp16 p2cRaw).
//   Each score element then gathers its two terms from LDS by idx and applies
//   the reference rounding chain fp16(fp16(c2p + p2c) / fp16(sqrt(3D))).
// Keys stream through LDS in chunks of 64 (shared by the 4 waves); for the
// context output V is streamed again, transposed into LDS.
// ---------------------------------------------------------------------------
#include <cmath>
#include <cstdlib>

#include "gd_common.hpp"
#include "gd_kernels.hpp"

namespace gd {
namespace {

constexpr int kQT = 64;       // queries per workgroup
constexpr int kKC = 64;       // keys per LDS chunk
constexpr int kD = 64;        // head dim
constexpr int kP2CStride = 34;  // halfs per row of the per-wave p2c tile (32 + pad)
constexpr int kVtStride = 68;   // halfs per row of the transposed V chunk (64 + pad)

// Largest c2p window (positions) for a 16-query wave at sequence length L.
// Filled on the host (exact) and checked against the kernel's LDS capacity.
constexpr int c2p_cap_for(int maxt) { return maxt <= 4 ? 80 : maxt <= 8 ? 144 : maxt <= 16 ? 288 : 416; }

template <int MAXT>
struct AttnSmem {
  static constexpr int kC2PCap = c2p_cap_for(MAXT);  // multiple of 16
  static constexpr int kC2PStride = kC2PCap + 2;
  int16_t idx_tab[2 * 16 * MAXT];
  __attribute__((aligned(16))) half_t kv[kD * kVtStride];  // K chunk (64 x 64 swizzled) or V^T chunk
  half_t c2p[4][16 * kC2PStride];
  half_t p2c[4][16 * kP2CStride];
};

__device__ __forceinline__ int kswz(int row, int chunk) { return row * kD + ((chunk ^ (row & 7)) << 3); }

template <int MAXT, int OUT>
__global__ __launch_bounds__(256) void deberta_attention_kernel(
    const half_t* __restrict__ Q, const half_t* __restrict__ K, const half_t* __restrict__ V, int64_t qsb, int64_t qsh,
    int64_t qsl, int64_t ksb, int64_t ksh, int64_t ksl, int64_t vsb, int64_t vsh, int64_t vsl,
    const half_t* __restrict__ PK, const half_t* __restrict__ PQ, int64_t pksh, int64_t pksp, int64_t pqsh,
    int64_t pqsp, const half_t* __restrict__ mask, int mask_kind, int B, int H, int L, int P, int bucket_size,
    float scale_qk, float scale16, half_t* __restrict__ out, int64_t ldo) {
  using Smem = AttnSmem<MAXT>;
  __shared__ Smem sm;
  constexpr int CS = Smem::kC2PStride;

  const int ntq = (L + kQT - 1) / kQT;
  const int nblk = B * H * ntq;
  int bid = blockIdx.x;
  if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);  // keep one (b,h) on one XCD
  const int qt = bid % ntq;
  const int bh = bid / ntq;
  const int h = bh % H;
  const int b = bh / H;

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int lc = lane & 15;  // column (query) of the MFMA output
  const int g = lane >> 4;   // lane group: k-chunk of operands, row group of outputs
  const int q0 = qt * kQT;
  const int qw = q0 + 16 * wave;
  const bool active = qw < L;
  const int nt = L >> 4;  // 16-key tiles

  // ---- relative index table for r in [-(L-1), L-1] ----
  for (int i = t; i < 2 * L - 1; i += 256) sm.idx_tab[i] = (int16_t)relative_index(i - (L - 1), bucket_size, P);
  __syncthreads();
  auto idx_of = [&](int r) -> int { return sm.idx_tab[r + L - 1]; };

  const half_t* Qb = Q + (int64_t)b * qsb + (int64_t)h * qsh;
  const half_t* Kb = K + (int64_t)b * ksb + (int64_t)h * ksh;
  const half_t* PKh = PK + (int64_t)h * pksh;
  const half_t* PQh = PQ + (int64_t)h * pqsh;
  half_t* c2p_w = sm.c2p[wave];
  half_t* p2c_w = sm.p2c[wave];

  // ---- Q fragments (B operand of K Q^T): Q[qw + lc][8g .. 8g+7] and [32 + 8g ..] ----
  half8_t qf0 = {}, qf1 = {};
  int pc_lo = 0;
  if (active) {
    const half_t* qrow = Qb + (int64_t)(qw + lc) * qsl;
    qf0 = *reinterpret_cast<const half8_t*>(qrow + 8 * g);
    qf1 = *reinterpret_cast<const half8_t*>(qrow + 32 + 8 * g);
    // ---- c2p window for this wave: C2P^T[p][q] = posK[p] . Q[q] ----
    pc_lo = idx_of(qw - (L - 1));
    const int pc_hi = idx_of(qw + 15);
    const int ntw = (pc_hi - pc_lo + 16) >> 4;
    for (int tw = 0; tw < ntw; ++tw) {
      int p = pc_lo + 16 * tw + lc;
      p = p < P ? p : P - 1;
      const half_t* prow = PKh + (int64_t)p * pksp;
      const half8_t a0 = *reinterpret_cast<const half8_t*>(prow + 8 * g);
      const half8_t a1 = *reinterpret_cast<const half8_t*>(prow + 32 + 8 * g);
      float4_t c = {0.f, 0.f, 0.f, 0.f};
      c = mfma16x16x32(a0, qf0, c);
      c = mfma16x16x32(a1, qf1, c);
      // lane holds positions 16tw + 4g + i for query lc
      half_t* dst = c2p_w + lc * CS + 16 * tw + 4 * g;
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[i] = (half_t)c[i];
    }
  }

  // ---- scores: S^T tiles + bias gather, kept in registers ----
  float sc[MAXT][4];
#pragma unroll
  for (int T = 0; T < MAXT; ++T)
#pragma unroll
    for (int i = 0; i < 4; ++i) sc[T][i] = -INFINITY;

  const half_t* maskb = mask + (int64_t)b * L;
#pragma unroll
  for (int c = 0; c < MAXT / 4; ++c) {
    const int kc = c * kKC;
    if (kc >= L) break;  // uniform across the workgroup
    // cooperative K chunk load (64 keys x 8 chunks of 16 B, 2 per thread)
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int piece = t + 256 * it;
      const int row = piece >> 3, ch = piece & 7;
      if (kc + row < L)
        *reinterpret_cast<half8_t*>(sm.kv + kswz(row, ch)) =
            *reinterpret_cast<const half8_t*>(Kb + (int64_t)(kc + row) * ksl + 8 * ch);
    }
    __syncthreads();
    if (active) {
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const int T = 4 * c + tt;
        if (T < nt) {
          const int k0 = 16 * T;
          const half8_t ka0 = *reinterpret_cast<const half8_t*>(sm.kv + kswz(16 * tt + lc, g));
          const half8_t ka1 = *reinterpret_cast<const half8_t*>(sm.kv + kswz(16 * tt + lc, 4 + g));
          float4_t s = {0.f, 0.f, 0.f, 0.f};
          s = mfma16x16x32(ka0, qf0, s);
          s = mfma16x16x32(ka1, qf1, s);
          // p2c window for keys k0..k0+15 x queries qw..qw+15
          const int pp_lo = idx_of(qw - k0 - 15);
          const int pp_hi = idx_of(qw - k0 + 15);
          const int nj = (pp_hi - pp_lo + 16) >> 4;  // 1 or 2
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            if (j < nj) {
              int p = pp_lo + 16 * j + lc;
              p = p < P ? p : P - 1;
              const half_t* prow = PQh + (int64_t)p * pqsp;
              const half8_t b0 = *reinterpret_cast<const half8_t*>(prow + 8 * g);
              const half8_t b1 = *reinterpret_cast<const half8_t*>(prow + 32 + 8 * g);
              float4_t r = {0.f, 0.f, 0.f, 0.f};
              r = mfma16x16x32(ka0, b0, r);
              r = mfma16x16x32(ka1, b1, r);
              // lane holds keys 4g+i, position 16j + lc
#pragma unroll
              for (int i = 0; i < 4; ++i) p2c_w[(4 * g + i) * kP2CStride + 16 * j + lc] = (half_t)r[i];
            }
          }
          wave_lds_sync();
          const half4_t mv = *reinterpret_cast<const half4_t*>(maskb + k0 + 4 * g);
          const int q = qw + lc;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int k = k0 + 4 * g + i;
            const int id = idx_of(q - k);
            const float c2p = (float)c2p_w[lc * CS + (id - pc_lo)];
            const float p2c = (float)p2c_w[(4 * g + i) * kP2CStride + (id - pp_lo)];
            const float bias16 = round_f16(round_f16(c2p + p2c) / scale16);
            const float m = (float)mv[i];
            const bool valid = mask_kind == GD_MASK_ATTENTION ? (m > 0.f) : !(m < -60000.f);
            if (OUT == GD_ATTN_OUT_BIAS) {
              sc[T][i] = round_f16(bias16 + (valid ? 0.f : -65504.f));
            } else {
              sc[T][i] = valid ? s[i] * scale_qk + bias16 : -INFINITY;
            }
          }
          wave_lds_sync();
        }
      }
    }
    __syncthreads();
  }

  if (!active && OUT != GD_ATTN_OUT_CONTEXT) return;  // no further barriers in these modes

  const int q = qw + lc;
  if (OUT == GD_ATTN_OUT_BIAS) {
    half_t* orow = out + (((int64_t)b * H + h) * L + q) * L;
#pragma unroll
    for (int T = 0; T < MAXT; ++T)
      if (T < nt) {
        half4_t v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (half_t)sc[T][i];
        *reinterpret_cast<half4_t*>(orow + 16 * T + 4 * g) = v;
      }
    return;
  }

  // ---- softmax over keys for query q (lane column), across the 4 lane groups ----
  float mx = -INFINITY;
#pragma unroll
  for (int T = 0; T < MAXT; ++T)
#pragma unroll
    for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[T][i]);
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  const float mref = mx == -INFINITY ? 0.f : mx;
  constexpr float kLog2e = 1.4426950408889634f;
  float sum = 0.f;
#pragma unroll
  for (int T = 0; T < MAXT; ++T)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float e = exp2f((sc[T][i] - mref) * kLog2e);  // exp2(-inf) = 0 for masked / absent keys
      sc[T][i] = e;
      sum += e;
    }
  sum += __shfl_xor(sum, 16, 64);
  sum += __shfl_xor(sum, 32, 64);
  const float inv = sum > 0.f ? 1.0f / sum : 0.f;

  if (OUT == GD_ATTN_OUT_PROBS) {
    half_t* orow = out + (((int64_t)b * H + h) * L + q) * L;
#pragma unroll
    for (int T = 0; T < MAXT; ++T)
      if (T < nt) {
        half4_t v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (half_t)(sc[T][i] * inv);
        *reinterpret_cast<half4_t*>(orow + 16 * T + 4 * g) = v;
      }
    return;
  }

  // ---- context: O = P V with P as the A operand (keys permuted consistently) ----
  float4_t o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = (float4_t){0.f, 0.f, 0.f, 0.f};
  const half_t* Vb = V + (int64_t)b * vsb + (int64_t)h * vsh;
#pragma unroll
  for (int c = 0; c < MAXT / 4; ++c) {
    const int kc = c * kKC;
    if (kc >= L) break;
    // V chunk -> LDS transposed: vt[d][key]
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int piece = t + 256 * it;
      const int row = piece >> 3, ch = piece & 7;
      half8_t v = {};
      if (kc + row < L) v = *reinterpret_cast<const half8_t*>(Vb + (int64_t)(kc + row) * vsl + 8 * ch);
#pragma unroll
      for (int e = 0; e < 8; ++e) sm.kv[(8 * ch + e) * kVtStride + row] = v[e];
    }
    __syncthreads();
    if (active) {
#pragma unroll
      for (int tt = 0; tt < 4; tt += 2) {
        const int T = 4 * c + tt;
        if (T < nt) {
          // P = P_hi + P_lo, both fp16: two MFMAs make P.V exact to ~2^-22
          // relative instead of rounding the probabilities to fp16 first.
          half8_t pa, pl;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p0 = sc[T][i] * inv;
            const float p1 = (T + 1 < nt) ? sc[T + 1][i] * inv : 0.f;
            pa[i] = (half_t)p0;
            pa[4 + i] = (half_t)p1;
            pl[i] = (half_t)(p0 - (float)pa[i]);
            pl[4 + i] = (half_t)(p1 - (float)pa[4 + i]);
          }
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) {
            const half_t* vrow = sm.kv + (16 * dt + lc) * kVtStride;
            const half4_t v0 = *reinterpret_cast<const half4_t*>(vrow + 16 * tt + 4 * g);
            const half4_t v1 = *reinterpret_cast<const half4_t*>(vrow + 16 * (tt + 1) + 4 * g);
            half8_t vb;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              vb[i] = v0[i];
              vb[4 + i] = v1[i];
            }
            o[dt] = mfma16x16x32(pa, vb, o[dt]);
            o[dt] = mfma16x16x32(pl, vb, o[dt]);
          }
        }
      }
    }
    __syncthreads();
  }
  if (!active) return;
  // lane holds O[qw + 4g + i][16 dt + lc]
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    half_t* orow = out + ((int64_t)b * L + (qw + 4 * g + i)) * ldo + (int64_t)h * kD;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) orow[16 * dt + lc] = (half_t)o[dt][i];
  }
}

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

template <int MAXT>
int launch_attention_maxt(const AttentionArgs& a, hipStream_t stream) {
  const int ntq = (int)((a.L + kQT - 1) / kQT);
  const dim3 grid((unsigned)(a.B * a.H * ntq)), block(256);
  auto hq = static_cast<const half_t*>(a.q);
  auto hk = static_cast<const half_t*>(a.k);
  auto hv = static_cast<const half_t*>(a.v);
  auto hpk = static_cast<const half_t*>(a.pk);
  auto hpq = static_cast<const half_t*>(a.pq);
  auto hm = static_cast<const half_t*>(a.mask);
  auto ho = static_cast<half_t*>(a.out);
#define GD_ATTN_LAUNCH(OUTK)                                                                                       \
  hipLaunchKernelGGL((deberta_attention_kernel<MAXT, OUTK>), grid, block, 0, stream, hq, hk, hv, a.qsb, a.qsh,      \
                     a.qsl, a.ksb, a.ksh, a.ksl, a.vsb, a.vsh, a.vsl, hpk, hpq, a.pksh, a.pksp, a.pqsh, a.pqsp,    \
                     hm, a.mask_kind, (int)a.B, (int)a.H, (int)a.L, (int)a.P, a.bucket_size, a.scale_qk,          \
                     a.scale16, ho, a.ldo)
  switch (a.output) {
    case GD_ATTN_OUT_PROBS:
      GD_ATTN_LAUNCH(GD_ATTN_OUT_PROBS);
      break;
    case GD_ATTN_OUT_CONTEXT:
      GD_ATTN_LAUNCH(GD_ATTN_OUT_CONTEXT);
      break;
    default:
      GD_ATTN_LAUNCH(GD_ATTN_OUT_BIAS);
      break;
  }
#undef GD_ATTN_LAUNCH
  GD_LAUNCH_CHECK();
  return GD_OK;
}

// Host-side band width: the largest c2p window any wave needs at length L.
int max_c2p_window(int L, int bucket_size, int max_position) {
  auto idx = [&](int r) {
    const int mid = bucket_size / 2;
    const int a = r < 0 ? -r : r;
    int bucket = r;
    if (a > mid) {
      const double x = std::log((double)a / mid) / std::log((double)(max_position - 1) / mid) * (mid - 1);
      const int lp = (int)std::ceil(x) + mid;
      bucket = r < 0 ? -lp : lp;
    }
    int v = bucket + bucket_size;
    return v < 0 ? 0 : (v > 2 * bucket_size - 1 ? 2 * bucket_size - 1 : v);
  };
  int worst = 0;
  for (int qw = 0; qw < L; qw += 16) {
    const int w = idx(qw + 15) - idx(qw - (L - 1)) + 1;
    worst = w > worst ? w : worst;
  }
  return (worst + 15) / 16 * 16;
}

}  // namespace

int launch_deberta_attention(const AttentionArgs& a, hipStream_t stream) {
  // GD_ATTN_VARIANT=1 selects the first (per-wave streaming) kernel for A/B
  // comparisons; the staged kernel is the default.
  static const int variant = [] {
    const char* e = std::getenv("GD_ATTN_VARIANT");
    return e ? std::atoi(e) : 0;
  }();
  if (variant == 0) return launch_deberta_attention2(a, stream);
  const int window = max_c2p_window((int)a.L, a.bucket_size, (int)a.P);
  if (a.L <= 64) {
    if (window > c2p_cap_for(4)) return fail(GD_ERR_UNSUPPORTED, "c2p window exceeds LDS capacity");
    return launch_attention_maxt<4>(a, stream);
  }
  if (a.L <= 128) {
    if (window > c2p_cap_for(8)) return fail(GD_ERR_UNSUPPORTED, "c2p window exceeds LDS capacity");
    return launch_attention_maxt<8>(a, stream);
  }
  if (a.L <= 256) {
    if (window > c2p_cap_for(16)) return fail(GD_ERR_UNSUPPORTED, "c2p window exceeds LDS capacity");
    return launch_attention_maxt<16>(a, stream);
  }
  if (window > c2p_cap_for(32)) return fail(GD_ERR_UNSUPPORTED, "c2p window exceeds LDS capacity");
  return launch_attention_maxt<32>(a, stream);
}

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
