// Disentangled attention of the DeBERTa-v3 encoder (the hot path).
//
// Reference: DeBERTa.swift:322-395 (relative bias from the fp16 c2pRaw/p2cRaw
// gathers, additive key mask, SDPA) with the index math of :498-551.
//
// One work item = (batch b, head h, 128 queries), run by a workgroup of 8
// waves, each owning 16 consecutive queries.  The LDS holds one
// workgroup per CU; up to L = 256 the grid has one workgroup per CU, each
// looping over items and fetching the next item's first stage while it
// finishes the current one.  Keys stream through LDS in chunks of 64.  The
// pairs (q, k) of a chunk have q - k in [bot, bot + 190], bot = q0 - kc - 63,
// so a chunk reads
//     K rows        64 x 128 B
//     posK window  192 x 128 B   (relative keys, for c2p)
//     posQ window  192 x 128 B   (relative queries, for p2c)
// where window row j holds table row idx(bot + j): the stages gather table
// rows through the index table, so inside the window the relative index is
// the plain distance q - k - bot for every pair, in the log-bucket zone as in
// the linear one, and every gather below is at a closed-form offset.  The
// next chunk's window is this one's shifted by 64 distances, so the windows
// live in two 256-row rings (distance d at ring row (d - q0 + 64) mod 256)
// and a chunk's stage brings only its K rows (one of two buffers) and the
// 64 window rows new to it; an item's first stage brings the whole window.
// Stages go out with global_load_lds_dwordx4 (16 B per lane straight into
// LDS, each lane from its own table row; the XOR swizzle of the 128-byte rows
// is applied on the global side) while the chunk before is computed.  Inside
// a chunk nothing touches global memory:
//   c2p  per wave: C2P = Q . posK[window]^T over <= 80 positions (5 MFMA
//        column tiles, v_mfma_f32_16x16x32_f16), rounded to fp16 (the
//        reference's c2pRaw) into a per-wave LDS tile;
//   per 16-key tile: S^T = K Q^T (2 MFMAs) and P2C^T = posQ[window] . K^T over
//        <= 31 positions (4 MFMAs), fp16 into a per-wave LDS tile; each score
//        gathers its two terms by idx and applies the reference rounding
//        chain fp16(fp16(c2p + p2c) / fp16(sqrt(3D))).
// Scores stay in registers (a lane owns one query column and 4 keys per
// tile), the softmax reduces in registers plus two cross-lane steps, and the
// outputs leave through LDS as 16-byte row segments: P rows (probabilities),
// the SDPA additive mask (bias), or the context P.V (V^T chunks in LDS, P as
// the MFMA A operand split into fp16 hi + lo parts).
//
// This header holds the kernel template; deberta_attention.hip holds the
// per-forward helper kernels (row extents, item schedule, packed rows) and
// the relative index table, and each attention_sm_*.hip instantiates one
// score mode.
#pragma once

#include <atomic>
#include <climits>
#include <cmath>
#include <mutex>
#include <type_traits>
#include "gd_common.hpp"
#include "gd_kernels.hpp"

namespace gd {

namespace {

constexpr int kThreads = 512;
constexpr int kWaves = 8;
constexpr int kQT = 128;           // queries per workgroup
constexpr int kKC = 64;            // keys per chunk
constexpr int kD = 64;             // head dim
constexpr int kWin = 192;          // relative-table rows per chunk window (>= 191)
constexpr int kC2PCols = 80;       // per-wave c2p window (<= 79 positions)
// Row strides of the per-wave c2p and p2c tiles, chosen against gfx950's LDS
// as the bank-conflict counter shows it for these patterns: 32 banks of 4
// bytes, 8-byte accesses served 16 lanes per cycle, 2-byte reads 32 lanes per
// cycle (two lanes in one dword do not conflict).
// c2p tile [80 positions][16 queries] in rows of 20 halfs: a lane's MFMA
// output (one position, four consecutive queries) is one aligned 8-byte
// store, conflict-free, and a score's four terms (query lc at positions
// 63 - 16 tt + lc - 4g - i) are four aligned 2-byte reads with at most two
// lanes on one bank.  (Rows by query would make the four terms one 8-byte
// read, but starting at any half: unaligned LDS reads stall.)
constexpr int kC2PTStride = 20;
// p2c tile (16 keys x 32 window positions) row-major by key in rows of 44
// halfs: a lane's MFMA output (one key, four consecutive positions) is one
// 8-byte store, and a score's four terms (keys 4g + i at positions
// 15 + lc - 4g - i) are four 2-byte reads 43 halfs apart; both conflict-free.
constexpr int kP2TStride = 44;
constexpr int kP2CRows = 47;       // fp32 chains: kr + p <= 15 + 31

// LDS map of `stages` (halfs): K buffers 0 and 1, the posK and posQ rings,
// and the V region (V rows 0 .. 255 for the P.V pass; free otherwise).  After
// the score loop the rings hold the next item's first stage (persistent
// workgroups); without a next item they take V rows 256 .. 511.
constexpr int kKBuf = kKC * kD;                   // 4096: one chunk's K rows
constexpr int kRingRows = 256;
constexpr int kRing = kRingRows * kD;             // 16384
constexpr int kVRowsA = 256;                      // V rows in the V region
constexpr int kOffPK = 2 * kKBuf;
constexpr int kOffPQ = kOffPK + kRing;
constexpr int kOffV = kOffPQ + kRing;
constexpr int kStagesLen = kOffV + kVRowsA * kD;  // 57344 halfs = 112 KiB
// The kernel-bias and fused chains keep c2p and p2c in fp32 (the Metal
// kernels never round them): per wave and key tile, c2p [16 queries][33]
// over the tile's 32 positions (33-float rows spread a wave's gathers over
// the banks) and p2c skewed, value (key row kr, position p) at row kr + p,
// column kr, in rows of 16 floats whose 16-byte block index is XORed with
// bits 2..3 of the row: a score's four keys 4g .. 4g+3 share kr + p =
// 15 + lc, so its four p2c terms are one conflict-free 16-byte read.
constexpr int kC2PF32Stride = 33;
constexpr int kScratchWave16 = kC2PCols * kC2PTStride + 16 * kP2TStride;    // halfs
constexpr int kScratchWave32 = (16 * kC2PF32Stride + kP2CRows * 16) * 2;    // halfs
constexpr int kScratchWave = kScratchWave16 > kScratchWave32 ? kScratchWave16 : kScratchWave32;
static_assert(16 * 72 <= kScratchWave, "context staging fits a wave's scratch");
static_assert((16 * kC2PF32Stride * 4) % 16 == 0 && (kScratchWave * 2) % 16 == 0, "fp32 p2c tile alignment");

// The relative index table holds idx(r) for every r in [-kRelSpan, kRelSpan]
// (bucket size 256, 512 positions) at entry r + kRelSpan.
constexpr int kRelSpan = 511;

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) half_t lds_half_t;
typedef short short4_t __attribute__((ext_vector_type(4)));


// 16-byte direct-to-LDS load (global_load_lds_dwordx4: lane l's 16 bytes land
// at M0 + 16 l), issued as inline assembly.  The compiler cannot tell which
// LDS buffer the builtin form writes once stage pointers are merged across
// the unrolled chunks, so it would drain every load in flight (vmcnt(0))
// before each later LDS read and serialise the stage pipeline; here the
// pipeline orders these loads itself (vmcnt(0) + barrier before a stage is
// read).  M0 is not used by anything else in this kernel.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void load_lds16(const half_t* g, lds_half_t* lds_block) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_block);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m0) : "memory", "m0");
}
// The same with a wave-uniform base address and a 32-bit byte offset per lane.
__device__ __forceinline__ void load_lds16(const half_t* sbase, uint32_t voff, lds_half_t* lds_block) {
  // (readfirstlane returns int: each half goes through uint32_t so that the
  // low half is not sign-extended into the high one)
  const uint64_t a = (uint64_t)(uintptr_t)sbase;
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a);
  sbase = (const half_t*)(uintptr_t)(((uint64_t)hi << 32) | lo);
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_block);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(m0)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// 128-byte rows; the 16-byte chunk index is XORed with bits 1..3 of the row.
// gfx950's LDS serves a ds_read_b128 16 lanes at a time over 64 banks
// (256 B): 16 consecutive rows at the same logical chunk then land on 16
// distinct (row parity, chunk) bank groups -- conflict-free.
__device__ __forceinline__ int swz(int row, int chunk) { return row * kD + ((chunk ^ ((row >> 1) & 7)) << 3); }

// Workgroups loop over items up to L = 256 (16 key tiles).
template <int MAXT>
constexpr bool attention_persistent() {
  return MAXT <= 16;
}

// SM selects the score chain (AttentionScore): the bias term (the default
// graph's fp16 chain, or the Metal kernels' fp32 c2p + p2c) and how it meets
// q.k (SDPA with an additive mask, the explicit fp16 chain, or the fused
// kernel's single fp32 sum).
template <int MAXT, int OUT, int SM>
__global__ __launch_bounds__(kThreads) void deberta_attention_kernel(
    const half_t* __restrict__ Q, const half_t* __restrict__ K, const half_t* __restrict__ V, int qsb, int qsh,
    int qsl, int ksb, int ksh, int ksl, int vsb, int vsh, int vsl, const half_t* __restrict__ PK,
    const half_t* __restrict__ PQ, int pksh, int pksp, int pqsh, int pqsp, const half_t* __restrict__ mask,
    int mask_kind, const int* __restrict__ row_len, const int* __restrict__ row_off, const int* __restrict__ q_len,
    const int* __restrict__ sched,
    int n_sched, int B, int H, int L, int P, int bucket_size, float scale_qk, float scale16, float scale_rel,
    const int16_t* __restrict__ rel_idx, half_t* __restrict__ out, int ldo) {
  // fp32 c2p / p2c per key tile (the Metal kernels' arithmetic)
  constexpr bool B32 = SM == kScoreKernelBias || SM == kScoreKernelBiasExplicit || SM == kScoreFused;
  // explicit-score chain: fp16 content score, fp16 P (DeBERTa.swift:397-409)
  constexpr bool GENC = SM == kScoreExplicit || SM == kScoreKernelBiasExplicit;
  // Two stage buffers and the per-wave scratch.  The stage DMA is inline
  // assembly the compiler does not track, so its reads of a stage never wait
  // for the next stage's loads in flight; the kernel orders them itself
  // (vmcnt + barrier before a stage is read).
  __shared__ __attribute__((aligned(1024))) half_t stages[kStagesLen];
  __shared__ __attribute__((aligned(1024))) half_t scratch_lds[kWaves * kScratchWave];
  __shared__ int16_t idx_tab[2 * 16 * MAXT];
  __shared__ __attribute__((aligned(16))) float mask_add[16 * MAXT];
  // per wave w (keys 64w .. 64w + 63): last valid key + 1 among its keys, or
  // 0, plus 1 << 16 when all 64 keys are valid
  __shared__ __attribute__((aligned(16))) int key_last[kWaves];

  // The stage buffers as LDS pointers: the DMA and the transposing reads
  // address them through these (no generic-to-LDS casts of computed pointers).
  lds_half_t* const stages3 = (lds_half_t*)(lds_void_t*)stages;
  constexpr bool kPersistent = attention_persistent<MAXT>();
  const int ntq = (L + kQT - 1) / kQT;
  const int nblk = B * H * ntq;
  const int t = threadIdx.x;
  const int lane = t & 63;
  // Wave-uniform values live in scalar registers: branches on them are scalar
  // and their address arithmetic runs once per wave, not per lane.
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  // The wave's 16-query group: groups 0-3 go to waves 0, 3, 5 and 6, then
  // 1, 2, 4, 7.  Waves w and w + 4 share a SIMD (the HW_ID register read on
  // the device), so up to four active groups sit on distinct SIMDs in this
  // order as in wave order; this one measured 0.5% faster on the packed step.
  const int qgrp = (0x73261540 >> (4 * wave)) & 7;
  const int lc = lane & 15;  // MFMA output column: the lane's query
  const int g = lane >> 4;   // lane group
  const float inv_scale16 = 1.0f / scale16;  // correctly rounded fp32 reciprocal
  half_t* c2p_w = scratch_lds + wave * kScratchWave;
  half_t* p2c_w = c2p_w + kC2PCols * kC2PTStride;  // [16 keys][kP2TStride]
  float* const c2pf = reinterpret_cast<float*>(c2p_w);  // fp32 chains
  float* const p2cf = c2pf + 16 * kC2PF32Stride;

  // ---- stage loads: lane l of 1 KiB block `blk` writes physical chunk l%8 of
  // row 8*blk + l/8, so it fetches the logical chunk that swz() puts there.
  // Every block this wave loads has the parity of the wave index.  Window row
  // j of a chunk with lowest distance bot = q0 - kc - 63 is table row
  // idx(bot + j), with the distance clamped to [-(L - 1), L - 1] (rows of
  // distances past it are never gathered).  The table offsets are 32-bit
  // byte offsets from the head's first row (checked by the launcher). ----
  const int blk_row = lane >> 3;
  const int blk_chunk = (lane & 7) ^ (((wave & 1) << 2) | (lane >> 4));
  // Table rows of 8-row block blk of a window starting at distance bot: the
  // lane's row of each table, into ring rows ring0 + 8 blk .. + 7 (ring0 a
  // multiple of 64, so the block's swizzle is that of rows 8 blk ..).
  auto stage_block = [&](const half_t* PKh, const half_t* PQh, int bot, int blk, int ring0, auto&& idx_of) {
    int r = bot + 8 * blk + blk_row;
    r = r < -(L - 1) ? -(L - 1) : (r > L - 1 ? L - 1 : r);
    const int prow = idx_of(r);
    const int off = (ring0 + 8 * blk) * kD;
    load_lds16(PKh, (uint32_t)((prow * pksp + blk_chunk * 8) * 2), stages3 + kOffPK + off);
    load_lds16(PQh, (uint32_t)((prow * pqsp + blk_chunk * 8) * 2), stages3 + kOffPQ + off);
  };
  // K rows kc .. kc + 63 into K buffer kb: 8 blocks of 8 rows, one per wave;
  // rows from klim on repeat row klim - 1.
  auto stage_k = [&](const half_t* Kb, int kc, int klim, int kb) {
    int key = kc + wave * 8 + blk_row;
    key = key < klim ? key : klim - 1;
    load_lds16(Kb + (int64_t)key * ksl + blk_chunk * 8, stages3 + kb * kKBuf + wave * 512);
  };
  // An item's first stage (chunk 0, window distances bot .. bot + 191 at
  // ring rows 0 .. 191): kStageOps DMA instructions per wave.
  auto issue_stage0 = [&](const half_t* Kb, const half_t* PKh, const half_t* PQh, int bot, int klim, auto&& idx_of) {
    stage_k(Kb, 0, klim, 0);
#pragma unroll
    for (int j = 0; j < kWin / 8 / kWaves; ++j) stage_block(PKh, PQh, bot, wave + kWaves * j, 0, idx_of);
  };
  constexpr int kStageOps = 1 + 2 * (kWin / 8 / kWaves);
  // idx(r) computed (the first stage, issued before the LDS index table exists)
  auto rel_arith = [&](int r) -> int { return relative_index(r, 256, 512); };
  // idx(r) from the LDS index table
  auto rel_lds = [&](int r) -> int { return idx_tab[r + L - 1]; };

  // ---- work items: (b, h, 128-query tile).  Up to L = 256 the grid holds
  // at most one workgroup per CU (the LDS allows no more) and workgroup w
  // takes items w, w + gridDim.x, ...; beyond, the scores fill the registers
  // and every workgroup takes one item.  Item ids map so that a (b, h)'s query tiles share an
  // XCD.  Each item's first stage and per-thread set-up reads are issued
  // while the previous item finishes (last chunk, softmax, P.V, stores), into
  // the stage buffer that item no longer needs. ----
  // `len` is the item's row extent: positions from len on take no part (keys
  // past it are neither read nor weighted, queries past it are not computed);
  // L without a row-extent array.  `klim` = max(len, 1) bounds row reads.
  // `row0` is the token row of (b, 0) with packed rows (row_off[b]), else -1.
  // `qlen` (<= len) bounds the queries computed and stored: q_len[b] when
  // given (only the rows a later step reads), else len.
  struct Item {
    int b, h, qt, len, klim, row0, qlen;
  };
  // Q / K / V of (b, h): row 0 of the batch row's slice.
  auto slice_base = [&](const half_t* X, const int b, const int h, const int row0, int sb, int sh, int sl) {
    return X + (row0 >= 0 ? (int64_t)row0 * sl : (int64_t)b * sb) + (int64_t)h * sh;
  };
  // Remap: item w + j gridDim.x (workgroup w on XCD w % 8, round j) becomes
  // local index l = w / 8 + j G (G = gridDim.x / 8) of XCD w % 8's contiguous
  // share, so the two query tiles of a (b, h) (l = 2m, 2m + 1 at L = 256) run
  // side by side on one XCD and share their K, V and table reads through its
  // L2.  On odd rounds l is swapped with its partner (l ^ 1): a workgroup's
  // successive items alternate between the pair's query tiles, which differ
  // in cost under row extents (when G and the share are even, the pairs stay
  // within a round).
  const bool swap_rounds = ((nblk >> 3) & 1) == 0 && ((gridDim.x >> 3) & 1) == 0 && gridDim.x >= 8;
  // With a schedule (row extents; built per forward by
  // attention_schedule_kernel) item slot s holds bh * ntq + qt, or -1 for an
  // empty slot, which runs as a query tile past every row's extent.
  const int n_items = sched != nullptr ? n_sched : nblk;
  auto decode = [&](int item) -> Item {
    int bid = item;
    bool empty = false;
    if (sched != nullptr) {
      bid = __builtin_amdgcn_readfirstlane(sched[item]);
      empty = bid < 0;
      bid = empty ? 0 : bid;
    } else if ((nblk & 7) == 0) {
      int l = bid >> 3;
      if (swap_rounds) l ^= (l / (int)(gridDim.x >> 3)) & 1;
      bid = (bid & 7) * (nblk >> 3) + l;
    }
    const int bh = bid / ntq;
    const int b = __builtin_amdgcn_readfirstlane(bh / H);
    int len = L;
    if (row_len != nullptr) {
      len = __builtin_amdgcn_readfirstlane(row_len[b]);
      len = len < 0 ? 0 : (len > L ? L : len);
    }
    const int row0 = row_off != nullptr ? __builtin_amdgcn_readfirstlane(row_off[b]) : -1;
    int qlen = len;
    if (q_len != nullptr) {
      qlen = __builtin_amdgcn_readfirstlane(q_len[b]);
      qlen = qlen < 0 ? 0 : (qlen > len ? len : qlen);
    }
    return Item{b, __builtin_amdgcn_readfirstlane(bh % H), empty ? ntq : __builtin_amdgcn_readfirstlane(bid % ntq), len,
                len > 0 ? len : 1, row0, qlen};
  };
  // First stage of an item (chunk 0: bot = q0 - 63).
  auto stage0_of = [&](const Item& it, auto&& idx_of) {
    issue_stage0(slice_base(K, it.b, it.h, it.row0, ksb, ksh, ksl), PK + (int64_t)it.h * pksh,
                 PQ + (int64_t)it.h * pqsh, it.qt * kQT - (kKC - 1), it.klim, idx_of);
  };
  // Per-thread set-up reads of an item: its key-mask entry and the Q
  // fragments.
  static_assert(2 * kThreads >= 2 * 16 * MAXT - 1 && kThreads >= 16 * MAXT, "one pass of set-up reads");
  struct Setup {
    half8_t qf0, qf1;  // Q[qw + lc][8g..] and [32 + 8g..] (B operand of K Q^T)
    half_t mval;
  };
  // The global loads are unconditional (clamped rows; values of rows past
  // the sequence are never used).  An item's set-up reads are issued before
  // its stage DMA: any vmcnt wait the compiler places among them (it does not
  // count the DMA, which is inline assembly) then cannot wait for that DMA.
  auto setup_of = [&](const Item& it) -> Setup {
    Setup su;
    const int q0 = it.qt * kQT, qw = q0 + 16 * qgrp;
    su.mval = mask[(int64_t)it.b * L + (t < L ? t : L - 1)];
    const int qr = qw + lc < it.klim ? qw + lc : it.klim - 1;
    const half_t* qrow = slice_base(Q, it.b, it.h, it.row0, qsb, qsh, qsl) + (int64_t)qr * qsl;
    su.qf0 = *reinterpret_cast<const half8_t*>(qrow + 8 * g);
    su.qf1 = *reinterpret_cast<const half8_t*>(qrow + 32 + 8 * g);
    return su;
  };

  int item = blockIdx.x;
  Item cur = decode(item);
  stage0_of(cur, rel_arith);
  // The index table, the same for every item, is built once.
  const int n_idx = 2 * L - 1;
  const int16_t id0 = t < n_idx ? rel_idx[t - (L - 1) + kRelSpan] : (int16_t)0;
  const int16_t id1 = t + kThreads < n_idx ? rel_idx[t + kThreads - (L - 1) + kRelSpan] : (int16_t)0;
  if (t < n_idx) idx_tab[t] = id0;
  if (t + kThreads < n_idx) idx_tab[t + kThreads] = id1;
  stage_barrier();  // the index table is complete (setup_of reads it)
  Setup cs = setup_of(cur);

  for (;;) {
    const int next = item + (int)gridDim.x;
    const bool has_next = kPersistent && next < n_items;  // uniform
    Item nit = cur;  // decoded once the chunk loop is done
    bool next_staged = false, next_setup = false;

    [&]() {
      // Lane-derived values of the item body are computed afresh per item
      // (an opaque copy of the lane index), not hoisted out of the item loop
      // where they would hold registers through every chunk.
      int lane_item = lane;
      asm volatile("" : "+v"(lane_item));
      const int lane = lane_item;
      const int lc = lane & 15;
      const int g = lane >> 4;
      // Swizzled offsets of this lane's two 16-byte chunks (g and 4 + g) in
      // row 16m + lc of a staged table: the XOR term depends on the row only
      // through lc, so a 16-aligned tile row base is a plain (uniform) offset.
      const int swz_lo = swz(lc, g);
      const int swz_hi = swz(lc, 4 + g);
      const int b = cur.b, h = cur.h;
      const int q0 = cur.qt * kQT;
      const int qw = q0 + 16 * qgrp;
      // Key tiles and chunks of this item: up to its row extent.  An item
      // whose queries all lie past the extent computes nothing; it runs one
      // chunk step (its first stage is already in flight) and loads no V.
      const bool live = q0 < cur.qlen;
      // Key tiles and chunks: set after chunk 0's barrier, once the key mask
      // has been reduced (the initial values only keep chunk 0 running).
      int nt = live ? (cur.len + 15) >> 4 : 0;
      int nchunks = live ? (nt + 3) >> 2 : 1;
      const int klim = cur.klim;
      const bool active = qw < cur.qlen;
      const half_t* Kb = slice_base(K, b, h, cur.row0, ksb, ksh, ksl);
      const half_t* PKh = PK + (int64_t)h * pksh;
      const half_t* PQh = PQ + (int64_t)h * pqsh;
      const half_t* Vb = slice_base(V, b, h, cur.row0, vsb, vsh, vsl);
      const half8_t qf0 = cs.qf0, qf1 = cs.qf1;
      // The key mask of batch row b as an additive term: 0 for a valid key,
      // -inf (probabilities) or -65504 (the SDPA mask output) for a masked
      // one; made visible by chunk 0's barrier.
      bool valid = false;
      if (t < L) {
        const float m = (float)cs.mval;
        valid = mask_kind == GD_MASK_ATTENTION ? (m > 0.f) : !(m < -60000.f);
        mask_add[t] = valid ? 0.f : (OUT == GD_ATTN_OUT_BIAS ? -65504.f : -INFINITY);
      }
      // Keys past the row's last valid one get probability exactly 0, so the
      // probabilities and the context stop there (the bias output keeps
      // every key: a masked key's bias is fp16(bias - 65504)).  A batch row
      // with no valid key keeps the reference's degenerate softmax over every
      // key (the masked scores themselves, below).  Each wave publishes the
      // extent of its keys' valid ones and whether all 64 are valid (chunk
      // `wave` then needs no mask term); read after chunk 0's barrier.
      {
        const uint64_t bal = __ballot(valid);
        if (lane == 0)
          key_last[wave] = (bal != 0 ? 64 * wave + 64 - __builtin_clzll(bal) : 0) | (~bal == 0 ? 1 << 16 : 0);
      }
      bool all_masked = false;  // uniform: set after chunk 0's barrier
      int chunk_valid = 0;      // uniform: bit c set when every key of chunk c is valid

      // ---- V for the P.V pass: rows [row_lo, row_hi) of the (b, h) slice
      // land row-major and swizzled like K at rows 0.. of an LDS buffer, by
      // DMA (placement: after the chunk loop).  Rows past the sequence repeat
      // row klim - 1; their probabilities are exactly 0. ----
      auto v_rows = [&]() { return ((16 * nt + 31) >> 5) << 5; };  // the P.V tile pairs reach this far
      auto issue_v = [&](lds_half_t* dst, int row_lo, int row_hi) {
        for (int blk = wave; 8 * blk < row_hi - row_lo; blk += kWaves) {  // uniform
          int key = row_lo + 8 * blk + blk_row;
          key = key < klim ? key : klim - 1;
          load_lds16(Vb + (int64_t)key * vsl + blk_chunk * 8, dst + blk * 512);
        }
      };

      float sc[MAXT][4];  // tiles at or past nt take no part in the softmax (probability 0)

#pragma unroll
      for (int c = 0; c < MAXT / 4; ++c) {
        if (c >= nchunks) break;  // uniform
        wait_vmcnt<0>();
        __syncthreads();  // stage c landed everywhere; every wave is done with stage c - 1
        if (c == 0) {
          const int4 a0 = *reinterpret_cast<const int4*>(key_last);
          const int4 a1 = *reinterpret_cast<const int4*>(key_last + 4);
          chunk_valid = __builtin_amdgcn_readfirstlane(
              ((a0.x >> 16) & 1) | ((a0.y >> 15) & 2) | ((a0.z >> 14) & 4) | ((a0.w >> 13) & 8) |
              ((a1.x >> 12) & 16) | ((a1.y >> 11) & 32) | ((a1.z >> 10) & 64) | ((a1.w >> 9) & 128));
          if constexpr (OUT != GD_ATTN_OUT_BIAS) {
            const int kext = __builtin_amdgcn_readfirstlane(
                max(max(max(a0.x & 0xffff, a0.y & 0xffff), max(a0.z & 0xffff, a0.w & 0xffff)),
                    max(max(a1.x & 0xffff, a1.y & 0xffff), max(a1.z & 0xffff, a1.w & 0xffff))));
            all_masked = kext == 0;
            const int klen = all_masked || kext > cur.len ? cur.len : kext;
            nt = live ? (klen + 15) >> 4 : 0;
            nchunks = live && nt > 0 ? (nt + 3) >> 2 : 1;
          }
        }
        // Chunk c + 1's stage: its K rows into K buffer (c + 1) & 1 and the 64
        // window rows new to it (distances bot_(c+1) .. + 63) into ring rows
        // (192 - 64 c) mod 256 .. + 63, the rows chunk c does not read (every
        // wave is done with chunk c - 1, which read them last).
        if (c + 1 < nchunks) {
          stage_k(Kb, (c + 1) * kKC, klim, (c + 1) & 1);
          stage_block(PKh, PQh, q0 - (c + 1) * kKC - (kKC - 1), wave, (kRingRows - kKC * (c + 1)) & (kRingRows - 1),
                      rel_lds);
        } else if constexpr (OUT == GD_ATTN_OUT_CONTEXT) {  // V rows into the V region
          issue_v(stages3 + kOffV, 0, v_rows() < kVRowsA ? v_rows() : kVRowsA);
        }
        const half_t* Ks = stages + (c & 1) * kKBuf;
        const half_t* PKs = stages + kOffPK;
        const half_t* PQs = stages + kOffPQ;
        // ring row of chunk c's window row j (16-aligned j: the block's rows
        // stay contiguous, and its swizzle is that of rows 0 .. 15)
        auto rr = [&](int j) -> int { return ((j - kKC * c) & (kRingRows - 1)) * kD; };
        const int kc = c * kKC;
        // The chunk's work for this wave, in compile-time variants whose bodies
        // have no branches, so the scheduler can overlap the tiles freely.
        // Window row of the pair (q, k) is q - k - bot (bot = q0 - kc - 63):
        // every offset below is closed-form and 16-aligned and the gathers
        // are contiguous.  FULL: all 64 keys of the chunk exist.  ALLM: the
        // item's batch row has no valid key.
        auto chunk = [&](auto full_c, auto allm_c, auto nomask_c) {
          constexpr bool FULL = decltype(full_c)::value;
          constexpr bool ALLM = decltype(allm_c)::value;
          // NOMASK: every key of the chunk is valid (its mask term is 0)
          constexpr bool NOMASK = decltype(nomask_c)::value;
          // c2p for this wave's 16 queries and the chunk's keys: window rows
          // [16 qgrp, 16 qgrp + 80) (distances qw - kc - 63 .. qw - kc + 16)
          const int crow0 = 16 * qgrp;
          if constexpr (!B32) {  // the fp32 chains compute c2p per key tile instead
#pragma unroll
          for (int tw = 0; tw < kC2PCols / 16; ++tw) {
            {
              const half8_t a0 = *reinterpret_cast<const half8_t*>(PKs + rr(crow0 + 16 * tw) + swz_lo);
              const half8_t a1 = *reinterpret_cast<const half8_t*>(PKs + rr(crow0 + 16 * tw) + swz_hi);
              // C2P = Q . posK^T: lane holds (query 4g + i, position 16 tw + lc)
              float4_t r = {0.f, 0.f, 0.f, 0.f};
              r = mfma16x16x32(qf0, a0, r);
              r = mfma16x16x32(qf1, a1, r);
              *reinterpret_cast<half4_t*>(c2p_w + (16 * tw + lc) * kC2PTStride + 4 * g) =
                  __builtin_convertvector(r, half4_t);
            }
          }
          }

          // Per 16-key tile tt: S^T = K Q^T (scores) and P2C over the 32 window
          // rows [prow0, prow0 + 32) the tile needs (prow0 = 16 (qgrp - tt) +
          // 48) into p2c_w.  Tiles are software-pipelined: tile tt's gathers are
          // issued before tile tt+1's MFMAs and p2c stores (the LDS executes a
          // wave's accesses in order, so one p2c buffer suffices), and tile tt is
          // combined while those are in flight.
          float4_t s_t[4];
          half8_t fk[2][2], fq[2][4];  // per tile parity: K rows (chunks g, 4+g), posQ rows (j = 0, 1)
          // Operand fragments of tile tt (LDS reads only; issued a tile ahead).
          // Tile tt's posQ rows [prow0 + 16, prow0 + 32) are tile tt-1's rows
          // [prow0', prow0' + 16) (prow0 = prow0' - 16): kept from its fragments.
          auto prep_load = [&](int tt) {
            const int par = tt & 1;
            const int prow0 = 16 * (qgrp - tt) + 48;
            fk[par][0] = *reinterpret_cast<const half8_t*>(Ks + 16 * tt * kD + swz_lo);
            fk[par][1] = *reinterpret_cast<const half8_t*>(Ks + 16 * tt * kD + swz_hi);
            fq[par][0] = *reinterpret_cast<const half8_t*>(PQs + rr(prow0) + swz_lo);
            fq[par][1] = *reinterpret_cast<const half8_t*>(PQs + rr(prow0) + swz_hi);
            if (tt == 0) {
              fq[par][2] = *reinterpret_cast<const half8_t*>(PQs + rr(prow0 + 16) + swz_lo);
              fq[par][3] = *reinterpret_cast<const half8_t*>(PQs + rr(prow0 + 16) + swz_hi);
            } else {
              fq[par][2] = fq[par ^ 1][0];
              fq[par][3] = fq[par ^ 1][1];
            }
          };
          // Scores and p2c of tile tt from its fragments.
          auto prep_compute = [&](int tt) {
            const int par = tt & 1;
            float4_t sv = {0.f, 0.f, 0.f, 0.f};
            sv = mfma16x16x32(fk[par][0], qf0, sv);
            s_t[tt] = mfma16x16x32(fk[par][1], qf1, sv);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              float4_t r = {0.f, 0.f, 0.f, 0.f};
              if constexpr (B32) {
                // P2C = K . posQ^T: lane holds (kr = 4g + i, p = 16 j + lc),
                // stored at row kr + p, column kr
                r = mfma16x16x32(fk[par][0], fq[par][2 * j], r);
                r = mfma16x16x32(fk[par][1], fq[par][2 * j + 1], r);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                  const int row = 4 * g + i + 16 * j + lc;
                  p2cf[row * 16 + ((g ^ ((row >> 2) & 3)) << 2) + i] = r[i];
                }
              } else {
                // P2C^T = posQ . K^T: lane holds (p = 16 j + 4g + i, key lc),
                // one 8-byte store of four fp16 values
                r = mfma16x16x32(fq[par][2 * j], fk[par][0], r);
                r = mfma16x16x32(fq[par][2 * j + 1], fk[par][1], r);
                *reinterpret_cast<half4_t*>(p2c_w + lc * kP2TStride + 16 * j + 4 * g) =
                    __builtin_convertvector(r, half4_t);
              }
            }
            if constexpr (B32) {
              // C2P^T = posK[the tile's 32 window rows] . Q^T, the same window
              // rows as the p2c fragments; lane holds (row 16 j + 4 g + i,
              // query lc).
              const int prow0 = 16 * (qgrp - tt) + 48;
#pragma unroll
              for (int j = 0; j < 2; ++j) {
                const half8_t a0 = *reinterpret_cast<const half8_t*>(PKs + rr(prow0 + 16 * j) + swz_lo);
                const half8_t a1 = *reinterpret_cast<const half8_t*>(PKs + rr(prow0 + 16 * j) + swz_hi);
                float4_t r = {0.f, 0.f, 0.f, 0.f};
                r = mfma16x16x32(a0, qf0, r);
                r = mfma16x16x32(a1, qf1, r);
#pragma unroll
                for (int i = 0; i < 4; ++i) c2pf[lc * kC2PF32Stride + 16 * j + 4 * g + i] = r[i];
              }
            }
          };
          prep_load(0);
          prep_compute(0);
#pragma unroll
          for (int tt = 0; tt < 4; ++tt) {
            const int T = 4 * c + tt;
            if constexpr (!FULL) {
              if (T >= nt) break;  // uniform
            }
            const int k0 = 16 * T;
            const bool next = tt + 1 < 4 && (FULL || T + 1 < nt);
            if (next) prep_load(tt + 1);  // fragment reads overlap this tile's gathers
            wave_lds_sync();  // tile tt's p2c stores (and the chunk's c2p) precede its gathers
            // Gather the two terms of score (q = qw + lc, k = k0 + 4g + i) at
            // window row q - k - bot: the c2p terms at tile position 63 - 16 tt
            // + lc - 4 g - i of query lc, the p2c terms at tile position 15 + lc
            // - 4 g - i of keys 4 g + i.
            float4_t madd = {0.f, 0.f, 0.f, 0.f};
            if constexpr (!NOMASK) madd = *reinterpret_cast<const float4_t*>(mask_add + k0 + 4 * g);
            half4_t c2p = {}, p2c = {};  // (the fp32 chains use c2p32 / p2c32 only)
            float4_t c2p32, p2c32;
            if constexpr (B32) {
              const float* cp = c2pf + lc * kC2PF32Stride + 15 + lc - 4 * g;
#pragma unroll
              for (int i = 0; i < 4; ++i) c2p32[i] = cp[-i];
              const int row = 15 + lc;
              p2c32 = *reinterpret_cast<const float4_t*>(p2cf + row * 16 + ((g ^ ((row >> 2) & 3)) << 2));
            } else {
              const half_t* cp = c2p_w + (63 - 16 * tt + lc - 4 * g) * kC2PTStride + lc;
#pragma unroll
              for (int i = 0; i < 4; ++i) c2p[i] = cp[-i * kC2PTStride];
              const half_t* pt = p2c_w + 4 * g * (kP2TStride - 1) + 15 + lc;
#pragma unroll
              for (int i = 0; i < 4; ++i) p2c[i] = pt[i * (kP2TStride - 1)];
            }
            wave_lds_sync();  // these gathers precede the next tile's p2c stores
            if (next) prep_compute(tt + 1);
            // fp16(c2p + p2c) is the fp16 add (two packed adds); the division by
            // fp16(sqrt(3D)) is a multiply by its fp32 reciprocal, which rounds to
            // the same fp16 value for every finite fp16 numerator (checked
            // exhaustively).
            // The fp32 chains: the relative-bias kernel's fp16((c2p + p2c) *
            // scale) with masked keys := -65504 (FusedKernels.swift:113-119),
            // or the fused kernel's (q.k + c2p + p2c) * scale (:47-56).
            const half4_t sum16 = c2p + p2c;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float v;
              if constexpr (ALLM) {
                // Every key masked: the reference's scores with the mask term
                // itself instead of -inf.  The fused kernel and the explicit
                // chain's `where` set every score to -65504 (uniform
                // weights); SDPA adds the kernel bias (-65504 on every key)
                // or fp16(bias + -65504) in fp32; the kernel-bias explicit
                // chain adds the bias in fp16.
                if constexpr (SM == kScoreFused || SM == kScoreExplicit) {
                  v = -65504.f;
                } else if constexpr (SM == kScoreKernelBias) {
                  v = fmaf(s_t[tt][i], scale_qk, -65504.f);
                } else if constexpr (SM == kScoreKernelBiasExplicit) {
                  v = round_f16(round_f16(round_f16(s_t[tt][i]) * inv_scale16) - 65504.f);
                } else {
                  v = fmaf(s_t[tt][i], scale_qk, round_f16(round_f16((float)sum16[i] * inv_scale16) - 65504.f));
                }
              } else if constexpr (SM == kScoreFused) {
                v = ((s_t[tt][i] + c2p32[i]) + p2c32[i]) * scale_rel;
                if constexpr (!NOMASK) v += madd[i];
              } else {
                float bias16;
                if constexpr (B32)
                  bias16 = round_f16((c2p32[i] + p2c32[i]) * scale_rel);
                else
                  bias16 = round_f16((float)sum16[i] * inv_scale16);
                if constexpr (OUT == GD_ATTN_OUT_BIAS) {
                  // (an unmasked key still takes the add: fp16(-0 + 0) = +0)
                  if constexpr (B32)
                    v = madd[i] != 0.f ? -65504.f : bias16;
                  else
                    v = round_f16(bias16 + madd[i]);
                } else if constexpr (GENC) {
                  // fp16(fp16(q.k) / fp16(sqrt(3D))) (the reciprocal multiply
                  // rounds like the divide for every fp16 numerator), then the
                  // fp16 add of the bias
                  const float content = round_f16(round_f16(s_t[tt][i]) * inv_scale16);
                  v = round_f16(content + bias16);
                  if constexpr (!NOMASK) v += madd[i];
                } else {
                  v = fmaf(s_t[tt][i], scale_qk, bias16);
                  if constexpr (!NOMASK) v += madd[i];
                }
              }
              sc[T][i] = v;
            }
          }
          if constexpr (!FULL) {  // key tiles of this chunk past the extent: probability 0
#pragma unroll
            for (int tt = 0; tt < 4; ++tt)
              if (4 * c + tt >= nt)
#pragma unroll
                for (int i = 0; i < 4; ++i) sc[4 * c + tt][i] = -INFINITY;
          }
          wave_lds_sync();  // the last gathers precede the next chunk's c2p / p2c stores
        };
        if (active) {
          if (all_masked)
            chunk(std::false_type{}, std::true_type{}, std::false_type{});
          else if (kc + kKC > 16 * nt)
            chunk(std::false_type{}, std::false_type{}, std::false_type{});
          else if ((chunk_valid >> c) & 1)
            chunk(std::true_type{}, std::false_type{}, std::true_type{});
          else
            chunk(std::true_type{}, std::false_type{}, std::false_type{});
        }
      }
      // The stage buffers are free from here on, except for V rows in flight
      // (context; waited for before the P.V pass) and the next item's stage.
      stage_barrier();
      // The next item's first stage goes to K buffer 0 and the rings now.  V
      // rows [0, kVRowsA) are in the V region (loaded during the last chunk);
      // rows from kVRowsA on (L > 256: no next item) go to the posK ring now.
      lds_half_t* const v_lo = stages3 + kOffV;   // V rows [0, kVRowsA)
      lds_half_t* const v_hi = stages3 + kOffPK;  // V rows [kVRowsA, v_rows)
      static_assert(MAXT * 16 <= kVRowsA || !kPersistent, "V rows past the V region need the rings");
      static_assert(MAXT * 16 - kVRowsA <= kRingRows, "V rows fit the V region and one ring");
      if constexpr (OUT == GD_ATTN_OUT_CONTEXT) {
        if (MAXT * 16 > kVRowsA && v_rows() > kVRowsA) issue_v(v_hi, kVRowsA, v_rows());  // no next item here
      }
      if (has_next) {  // after every V row; the set-up reads before the stage DMA (see setup_of)
        nit = decode(next);
        cs = setup_of(nit);  // (the item's own set-up values are dead by now)
        next_setup = true;
        stage0_of(nit, rel_lds);
        next_staged = true;
      }

      // The softmax runs over whole chunks: key tiles of the last chunk past
      // the extent hold -inf (set by the chunk), tiles of later chunks are
      // set to probability 0 here.
      float inv_sum = 0.f;
      if (OUT != GD_ATTN_OUT_BIAS) {
        float mx = -INFINITY;
#pragma unroll
        for (int c = 0; c < MAXT / 4; ++c)
          if (c < nchunks)  // uniform
#pragma unroll
            for (int T = 4 * c; T < 4 * c + 4; ++T)
#pragma unroll
              for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[T][i]);
        mx = rows_max(mx);
        const float mref = mx == -INFINITY ? 0.f : mx;
        constexpr float kLog2e = 1.4426950408889634f;
        // exp(s - m) = 2^(s log2e - m log2e) as one fma per score; the rounding
        // of m log2e scales the whole row alike and cancels in the normalisation.
        const float mref_l2 = mref * kLog2e;
        float sum = 0.f;
#pragma unroll
        for (int c = 0; c < MAXT / 4; ++c) {
          if (c < nchunks) {  // uniform
#pragma unroll
            for (int T = 4 * c; T < 4 * c + 4; ++T)
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const float e = __builtin_amdgcn_exp2f(fmaf(sc[T][i], kLog2e, -mref_l2));  // v_exp_f32; exp2(-inf) = 0
                sc[T][i] = e;
                sum += e;
              }
          } else {  // past the key extent: probability 0
#pragma unroll
            for (int T = 4 * c; T < 4 * c + 4; ++T)
#pragma unroll
              for (int i = 0; i < 4; ++i) sc[T][i] = 0.f;
          }
        }
        sum = rows_sum(sum);
        inv_sum = sum > 0.f ? 1.0f / sum : 0.f;
        // The context path scales O once at the end instead of every
        // probability, except on the explicit chain, whose P.V multiplies the
        // fp16 probabilities (DeBERTa.swift:407-408).
        if (OUT == GD_ATTN_OUT_PROBS || GENC) {
#pragma unroll
          for (int T = 0; T < MAXT; ++T)
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[T][i] *= inv_sum;
        }
      }
      if (OUT == GD_ATTN_OUT_PROBS || OUT == GD_ATTN_OUT_BIAS) {
        // Stage this wave's 16 rows x L in LDS (rows padded by 16 bytes so the
        // 8-byte column stores of a wave hit distinct banks), then write
        // 16-byte row segments.  Rows 0-7 and 8-15 of wave w go to 8-row
        // slots 2w and 2w + 1, which fill the V region (with a next item,
        // whose first stage occupies K buffer 0 and the rings) or all of
        // `stages` (without), then the scratch buffer.
        const int rs = L + 8;
        constexpr int kSlot = 8 * (16 * MAXT + 8);
        constexpr int kOffA = kPersistent ? kOffV : 0;
        constexpr int kSlotsA = (kStagesLen - kOffA) / kSlot;
        static_assert(kSlotsA + kWaves * kScratchWave / kSlot >= 2 * kWaves, "probability staging");
        auto slot = [&](int sl) -> half_t* {
          return sl < kSlotsA ? stages + kOffA + sl * kSlot : scratch_lds + (sl - kSlotsA) * kSlot;
        };
        half_t* const rows_lo = slot(2 * wave);      // rows 0-7
        half_t* const rows_hi = slot(2 * wave + 1);  // rows 8-15
        if (active) {
          half_t* const wrow = (lc < 8 ? rows_lo : rows_hi) + (lc & 7) * rs + 4 * g;
#pragma unroll
          for (int T = 0; T < MAXT; ++T)
            if (16 * T < L) {  // tiles past the key extent hold 0 (probabilities) or the bias of every key
              half4_t v;
#pragma unroll
              for (int i = 0; i < 4; ++i) v[i] = (half_t)sc[T][i];
              *reinterpret_cast<half4_t*>(wrow + 16 * T) = v;
            }
          wave_lds_sync();
          // Pass it covers rows kRowsPass it + lane / kPieces, 16-byte piece
          // lane % kPieces of each (pieces from L / 8 on are past the row and
          // not stored; their LDS reads stay in this wave's staging rows).
          // Every LDS read is issued before the first store.  The stores are
          // non-temporal: the [B, H, L, L] output would otherwise evict the
          // relative tables, which every item re-reads, from the L2.
          constexpr int kPieces = 2 * MAXT;
          constexpr int kRowsPass = 64 / kPieces;
          constexpr int kPasses = 16 / kRowsPass;
          const int pr = lane / kPieces, cpos = lane % kPieces;
          half8_t seg[kPasses];
#pragma unroll
          for (int it = 0; it < kPasses; ++it)  // rows of pass it: all below 8 or all from 8 on
            seg[it] = *reinterpret_cast<const half8_t*>((kRowsPass * (it + 1) <= 8 ? rows_lo : rows_hi) +
                                                        ((kRowsPass * it + pr) & 7) * rs + cpos * 8);
          half_t* const orow = out + (((int64_t)b * H + h) * L + qw + pr) * L + cpos * 8;
          if (cpos < L / 8) {
#pragma unroll
            for (int it = 0; it < kPasses; ++it)
              __builtin_nontemporal_store(seg[it], reinterpret_cast<half8_t*>(orow + (int64_t)kRowsPass * it * L));
          }
        }
        return;
      }

      // ---- context: O = P V with V row-major in LDS, P (hi + lo) as the A operand ----
      // The B operand (keys x d) is read with ds_read_b64_tr_b16: in each
      // 16-lane group, source lane s names 4 consecutive halfs and output lane
      // j receives element j % 4 of source lanes j / 4, 4 + j / 4, 8 + j / 4,
      // 12 + j / 4.  Source lane lc of group g names V[r0 + lc / 4][16 dt +
      // 4 (lc % 4) ..] with r0 = 16 T + 4 g, so lane (g, lc) receives
      // V[16 T + 4 g + i][16 dt + lc], i = 0..3: the B fragment of the keys
      // that pa holds for tile T (and, from r0 + 16, for tile T + 1).  The
      // swizzle term (row >> 1) & 7 of those rows is (2 g + lc / 8) & 7 for
      // every 16-aligned tile base.  The next item's stage (the last kStageOps
      // DMA instructions, issued after the V rows) may stay in flight.
      if (next_staged)
        wait_vmcnt<kStageOps>();
      else
        wait_vmcnt<0>();
      stage_barrier();  // every wave's V rows have landed
      if (!active) return;
      float4_t o[4];
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) o[dt] = (float4_t){0.f, 0.f, 0.f, 0.f};
      typedef __attribute__((address_space(3))) short4_t lds_short4_t;
      const int tr_sw = (2 * g + (lc >> 3)) & 7;
      const int tr_lane = (4 * g + (lc >> 2)) * kD + 4 * (lc & 1);  // row and half offset of this source lane
      const int tr_c = (lc >> 1) & 1;                                // 16-byte chunk within the 32-byte d slice
#pragma unroll
      for (int c = 0; c < MAXT / 4; ++c) {
        if (c >= nchunks) break;
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) {
          const int T = 4 * c + 2 * pr;
          if (T >= nt) break;  // uniform; nt is at most one past the last pair's first tile
          const int row0 = 16 * T;
          const lds_half_t* vsrc = row0 < kVRowsA ? v_lo + row0 * kD : v_hi + (row0 - kVRowsA) * kD;
          // Unnormalised P of key tiles T, T + 1 as the A operand, split into
          // fp16 hi (truncated) + lo (the exact fp32 remainder, rounded).  Tiles
          // at or past nt hold 0.
          // On the explicit chain the operand is P rounded to fp16 (the
          // reference's fp16 probabilities), with no low part.
          half8_t pa, pl;
#pragma unroll
          for (int i = 0; i < 4; i += 2) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              const float x0 = sc[T + u][i], x1 = sc[T + u][i + 1];
              if constexpr (GENC) {
                pa[4 * u + i] = (half_t)x0;
                pa[4 * u + i + 1] = (half_t)x1;
              } else {
                const half2_t hi = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(x0, x1));
                pa[4 * u + i] = hi[0];
                pa[4 * u + i + 1] = hi[1];
                pl[4 * u + i] = (half_t)(x0 - (float)hi[0]);
                pl[4 * u + i + 1] = (half_t)(x1 - (float)hi[1]);
              }
            }
          }
          half8_t vb[4];
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) {
            const lds_half_t* a = vsrc + tr_lane + (((2 * dt + tr_c) ^ tr_sw) << 3);
            const short4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)a);
            const short4_t v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(a + 16 * kD));
            const half4_t h0 = __builtin_bit_cast(half4_t, v0), h1 = __builtin_bit_cast(half4_t, v1);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              vb[dt][i] = h0[i];
              vb[dt][4 + i] = h1[i];
            }
          }
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) o[dt] = mfma16x16x32(pa, vb[dt], o[dt]);
          if constexpr (!GENC) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) o[dt] = mfma16x16x32(pl, vb[dt], o[dt]);
          }
        }
      }
      // lane holds O[qw + 4g + i][16 dt + lc]: stage 16 x 64 in LDS, write 128-byte rows
      // (the softmax sum of query row r sits in lanes with lc = r)
      half_t* ot = scratch_lds + wave * kScratchWave;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float inv_row = GENC ? 1.0f : __shfl(inv_sum, 4 * g + i, 64);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) ot[(4 * g + i) * 72 + 16 * dt + lc] = (half_t)(o[dt][i] * inv_row);
      }
      wave_lds_sync();
      {
        const int r = lane >> 3, cpos = lane & 7;  // 8 rows x 8 pieces per pass
#pragma unroll
        for (int pass = 0; pass < 2; ++pass) {
          const int row = r + 8 * pass;
          // packed rows: rows past the extent belong to the next batch row;
          // rows from qlen on are not computed
          if ((cur.row0 < 0 && q_len == nullptr) || qw + row < cur.qlen)
            *reinterpret_cast<half8_t*>(out + ((cur.row0 >= 0 ? (int64_t)cur.row0 : (int64_t)b * L) + qw + row) * ldo +
                                        (int64_t)h * kD + cpos * 8) =
                *reinterpret_cast<const half8_t*>(ot + row * 72 + cpos * 8);
        }
      }
    }();

    if (!has_next) break;
    if (!next_setup) cs = setup_of(nit);
    cur = nit;
    item = next;
  }
}

template <int SM, int MAXT>
int launch_attention_maxt(const AttentionArgs& a, hipStream_t stream) {
  const int ntq = (int)((a.L + kQT - 1) / kQT);
  const int64_t items = a.B * a.H * ntq;
  const int64_t cus = attention_persistent<MAXT>() ? device_cu_count() : items;
  const dim3 grid((unsigned)(items < cus ? items : cus)), block(kThreads);
  auto hq = static_cast<const half_t*>(a.q);
  auto hk = static_cast<const half_t*>(a.k);
  auto hv = static_cast<const half_t*>(a.v);
  auto hpk = static_cast<const half_t*>(a.pk);
  auto hpq = static_cast<const half_t*>(a.pq);
  auto hm = static_cast<const half_t*>(a.mask);
  auto ho = static_cast<half_t*>(a.out);
  // element strides in 32 bits (checked by launch_deberta_attention)
#define GD_ATTN2(OUTK)                                                                                            \
  hipLaunchKernelGGL((deberta_attention_kernel<MAXT, OUTK, SM>), grid, block, 0, stream, hq, hk, hv, (int)a.qsb, \
                     (int)a.qsh, (int)a.qsl, (int)a.ksb, (int)a.ksh, (int)a.ksl, (int)a.vsb, (int)a.vsh, (int)a.vsl, \
                     hpk, hpq, (int)a.pksh, (int)a.pksp, (int)a.pqsh, (int)a.pqsp, hm, a.mask_kind, a.row_len,      \
                     a.row_off, a.q_len, a.sched, a.n_sched, (int)a.B, (int)a.H, (int)a.L, (int)a.P, a.bucket_size, \
                     a.scale_qk, a.scale16, a.scale_rel, a.rel_idx, ho, (int)a.ldo)
  switch (a.output) {
    case GD_ATTN_OUT_PROBS:
      GD_ATTN2(GD_ATTN_OUT_PROBS);
      break;
    case GD_ATTN_OUT_CONTEXT:
      GD_ATTN2(GD_ATTN_OUT_CONTEXT);
      break;
    default:
      // the bias output exists on the chains that add a bias of their own
      if constexpr (SM == kScoreDefault || SM == kScoreKernelBias) {
        GD_ATTN2(GD_ATTN_OUT_BIAS);
      } else {
        return fail(GD_ERR_INVALID_ARGUMENT, "attention: no bias output on this score chain");
      }
      break;
  }
#undef GD_ATTN2
  GD_LAUNCH_CHECK();
  return GD_OK;
}

template <int SM>
int launch_attention_sm(const AttentionArgs& a, hipStream_t stream) {
  if (a.rel_idx == nullptr) return fail(GD_ERR_INVALID_ARGUMENT, "attention: no relative index table");
  if (a.L <= 64) return launch_attention_maxt<SM, 4>(a, stream);
  if (a.L <= 128) return launch_attention_maxt<SM, 8>(a, stream);
  if (a.L <= 256) return launch_attention_maxt<SM, 16>(a, stream);
  return launch_attention_maxt<SM, 32>(a, stream);
}

}  // namespace
}  // namespace gd
