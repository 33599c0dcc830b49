// Internal launchers (C++), called by the C-ABI layer and the classifier
// context after argument validation.  All return a gd_status.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace gd {

// Compute units of the current device (cached per device).
int device_cu_count();

// Streaming reference kernel (gd_stream_probe_add): c = a + b, n fp16.
int launch_stream_probe_add(const void* a, const void* b, void* c, int64_t n, hipStream_t stream);

// gd_diag_mfma_forms: 32 x 32 x 16 and 16 x 16 x 16 MFMA forms on the same tiles.
int launch_mfma_forms(const void* a, const void* w, const float* c0, float* d32, float* d16, int64_t tiles,
                      hipStream_t stream);

int launch_residual_layer_norm(const void* x, const void* residual, const void* gamma, const void* beta, void* out,
                               int64_t rows, int64_t cols, float eps, uint32_t flags, hipStream_t stream);

// row_map (optional, device int32 [tokens]): output row t embeds token
// row_map[t] of ids / mask, which hold `sources` tokens (packed rows).
int launch_embedding_layer_norm(const int32_t* ids, const void* mask, const void* table, const void* gamma,
                                const void* beta, void* out, int64_t tokens, int64_t cols, int64_t vocab, float eps,
                                int32_t* error_flag, hipStream_t stream, const int32_t* row_map = nullptr,
                                int64_t sources = 0);

// Fills the per-device GELU table used by the GELU epilogue (first call per
// device; refuses while `stream` is capturing a graph).
int ensure_gelu_table(hipStream_t stream);
// Fills the device's relative index table used by launch_deberta_attention
// (first call per device; not allowed during graph capture).
int ensure_relative_index_table(hipStream_t stream);

int launch_linear(const void* a, const void* w, const void* bias, void* c, int64_t m, int64_t n, int64_t k, int64_t lda,
                  int64_t ldc, const int32_t* a_rows, int64_t a_row_count, int epilogue_kind, hipStream_t stream);

// Score chains of the attention kernel (which reference graph it reproduces).
enum AttentionScore {
  kScoreDefault = 0,             // default bias chain + SDPA (DeBERTa.swift:374-394)
  kScoreExplicit = 1,            // default bias + explicit-score chain (useFastAttention=false, :397-409)
  kScoreKernelBias = 2,          // relative-bias Metal kernel's bias + SDPA with it as the mask (:357-372, 383-385)
  kScoreKernelBiasExplicit = 3,  // the same bias + explicit-score chain without where (:397-405)
  kScoreFused = 4,               // fused-attention Metal kernel (useFusedAttentionKernel, :337-354)
};

struct AttentionArgs {
  const void* q;
  const void* k;
  const void* v;
  int64_t qsb, qsh, qsl, ksb, ksh, ksl, vsb, vsh, vsl;
  const void* pk;
  const void* pq;
  int64_t pksh, pksp, pqsh, pqsp;
  const void* mask;
  int mask_kind;
  int64_t B, H, L, P;
  int bucket_size;
  float scale_qk;  // 1 / sqrt(3 D) in fp32 (applied to q.k)
  float scale16;   // fp16(sqrt(3 D)) (divides the relative bias)
  int output;      // GD_ATTN_OUT_*
  void* out;
  int64_t ldo;
  // Optional row extents [B] (context output only): keys at or past row_len[b]
  // are not read, queries at or past it are not computed (their output rows
  // hold copies or are left as they were).
  const int32_t* row_len = nullptr;
  // Optional packed rows [B] (context output, with row_len): token (b, l) of
  // Q, K, V and the output is row row_off[b] + l (the batch strides unused);
  // output rows at or past row_len[b] are not written.
  const int32_t* row_off = nullptr;
  // Optional query extents [B] (with row_len): queries at or past
  // min(q_len[b], row_len[b]) are neither computed nor stored.
  const int32_t* q_len = nullptr;
  // Optional item schedule (with row_len; launch_attention_schedule):
  // n_sched = attention_schedule_slots(B, H, L) entries.
  const int32_t* sched = nullptr;
  int n_sched = 0;
  // Score chain (AttentionScore) and, for the kernel-bias and fused chains,
  // the scale the Metal kernels multiply (c2p + p2c) or (q.k + c2p + p2c)
  // by (FusedKernels.swift:53,116).
  int score = kScoreDefault;
  float scale_rel = 0.f;
  // Device address of the relative index table (set by
  // launch_deberta_attention).
  const int16_t* rel_idx = nullptr;
};

// Per-score-mode launchers (one translation unit each).
int launch_attention_default(const AttentionArgs& args, hipStream_t stream);
int launch_attention_explicit(const AttentionArgs& args, hipStream_t stream);
int launch_attention_kernel_bias(const AttentionArgs& args, hipStream_t stream);
int launch_attention_fused(const AttentionArgs& args, hipStream_t stream);
// The relative index table's device address on the current device (filled
// on first use, as ensure_relative_index_table).
int relative_index_table_device(const int16_t** out, hipStream_t stream);

// Slots of the persistent attention's item schedule for (B, H, L), 0 when
// that launch takes no schedule (L > 256, or more than 2048 (b, h) pairs).
int attention_schedule_slots(int64_t B, int64_t H, int64_t L);
// Builds the schedule from the row extents (one workgroup; once per forward).
int launch_attention_schedule(const int32_t* row_len, int64_t B, int64_t H, int64_t L, int32_t* sched,
                              hipStream_t stream);

int launch_deberta_attention(const AttentionArgs& args, hipStream_t stream);

// Row extents for the attention: out[b] = max(last l with mask[b, l] > 0,
// last position read by a marker slot of row b with marker_mask > 0
// (position 0 for an out-of-range index)) + 1, or 0.
int launch_row_extent(const void* mask, const int32_t* markers, const float* marker_mask, int64_t B, int64_t L,
                      int64_t slots, int32_t* out, hipStream_t stream);

// Query extents: out[b] = last position read by a marker slot of row b with
// marker_mask > 0 (position 0 for an out-of-range index) + 1, or 0.
int launch_query_extent(const int32_t* markers, const float* marker_mask, int64_t B, int64_t L, int64_t slots,
                        int32_t* out, hipStream_t stream);

// Packed rows from the extents: row_off[b] = sum of row_len[0, b) (B + 1
// entries) and row_map[row_off[b] + l] = b * L + l for l < row_len[b], for
// packed rows below `total`.  exact: a sum other than `total` raises the
// error flag; otherwise `total` is a capacity (a larger sum raises it) and
// the rows past the sum map to token 0.
int launch_pack_rows(const int32_t* row_len, int64_t B, int64_t L, int64_t total, bool exact, int32_t* row_off,
                     int32_t* row_map, int32_t* error_flag, hipStream_t stream);

int launch_relative_bias_general(const void* q, const void* k, const void* pos_key, const void* pos_query,
                                 const int32_t* c2p, const int32_t* p2c, const void* key_mask, float scale, int64_t B,
                                 int64_t H, int64_t L, int64_t D, int64_t P, void* out, int32_t* error_flag,
                                 hipStream_t stream);

int launch_fused_attention_general(const void* q, const void* k, const void* v, const void* pos_key,
                                   const void* pos_query, const int32_t* c2p, const int32_t* p2c, const void* key_mask,
                                   float scale, int64_t B, int64_t H, int64_t L, int64_t D, int64_t P, void* out,
                                   int32_t* error_flag, hipStream_t stream);

int launch_relative_index_table(int32_t* out, int n, int bucket_size, int max_position, hipStream_t stream);

// Classifier head helpers (head.hip).
// rows_out[b, s] = token row of marker s of batch row b: b * seq_len +
// position, or row_off[b] + position with packed rows (row_off optional).
int launch_marker_rows(const int32_t* marker_indices, int32_t* rows_out, int64_t batch, int64_t seq_len,
                       int64_t markers_per_row, int32_t* error_flag, hipStream_t stream,
                       const int32_t* row_off = nullptr);
// dst[i, :] = src[rows[i], :] for i < n (rows clamped to [0, src_rows)),
// `cols` fp16 columns, rows of `cols` elements.
int launch_gather_rows(const void* src, const int32_t* rows, int64_t n, int64_t src_rows, int64_t cols, void* dst,
                       hipStream_t stream);
int launch_head_output(const void* inner, const void* w2, const void* b2, const float* marker_mask, void* logits,
                       int64_t rows, int64_t width, hipStream_t stream);

}  // namespace gd
