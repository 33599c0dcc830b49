/*
 * gliner_decide.h -- C-ABI of the MI355X (gfx950) GLiNER-Decide encoder path.
 *
 * This is the boundary that replaces the reference's MLX/Metal operator
 * surface.  Every entry point names the reference interface it stands in for
 * (file:line in shantanugoel/gliner-decide-metal).
 *
 * Conventions
 *  - Tensors are caller-owned DEVICE pointers (hipMalloc'd or equivalent),
 *    row-major, fp16 unless stated ("f16" = IEEE binary16 as uint16 storage).
 *  - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *    Calls enqueue work and return without synchronising; outputs are ready
 *    when the stream reaches that point.
 *  - Every function returns a gd_status (0 = GD_OK).  On failure nothing is
 *    enqueued and gd_last_error() returns a message (thread-local).  Shape
 *    misuse that the reference traps on with `precondition`
 *    (FusedKernels.swift:176-182, 229-232, 269-272) is reported here as
 *    GD_ERR_SHAPE / GD_ERR_INVALID_ARGUMENT instead.
 *  - Standalone kernels allocate nothing.  The classifier context allocates
 *    its weights at creation and its activation workspace on first use of a
 *    larger shape (gd_classifier_reserve pre-allocates it).
 *  - Thread safety: one context may be used from one thread at a time;
 *    distinct contexts and the standalone kernels are reentrant per stream.
 */
#ifndef GLINER_DECIDE_H_
#define GLINER_DECIDE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The library is built with hidden visibility; everything declared here is
 * exported. */
#if defined(__GNUC__)
#pragma GCC visibility push(default)
#endif

#define GD_ABI_VERSION 1

/* Status codes (replace Swift `precondition` traps and WeightStoreError,
 * Weights.swift:4-19). */
typedef enum gd_status {
  GD_OK = 0,
  GD_ERR_INVALID_ARGUMENT = -1, /* null pointer, bad flag, bad scalar           */
  GD_ERR_SHAPE = -2,            /* unsupported / inconsistent dimensions        */
  GD_ERR_UNSUPPORTED = -3,      /* valid request this build does not implement  */
  GD_ERR_HIP = -4,              /* HIP runtime or launch failure                */
  GD_ERR_MISSING_WEIGHT = -5,   /* WeightStoreError.missingWeight               */
  GD_ERR_WEIGHT_SHAPE = -6,     /* WeightStoreError.invalidShape                */
  GD_ERR_WEIGHT_DTYPE = -7,     /* dtype check of WeightStore.array             */
  GD_ERR_IO = -8,               /* file open / parse failure                    */
  GD_ERR_OUT_OF_MEMORY = -9,
  GD_ERR_DEVICE_INDEX = -10     /* a device-side index was out of range         */
} gd_status;

/* Element types for weight-store entries (safetensors dtype names). */
typedef enum gd_dtype {
  GD_F16 = 0,
  GD_F32 = 1,
  GD_BF16 = 2,
  GD_I32 = 3,
  GD_I64 = 4
} gd_dtype;

const char* gd_last_error(void);
int gd_abi_version(void);
const char* gd_build_info(void);

/* ------------------------------------------------------------------------ *
 * Configuration -- DeBERTaV2Configuration (Configuration.swift:3-48)
 * ------------------------------------------------------------------------ */
typedef struct gd_config {
  int32_t hidden_size;            /* 1024 */
  int32_t intermediate_size;      /* 4096 */
  int32_t num_hidden_layers;      /* 24   */
  int32_t num_attention_heads;    /* 16   */
  float layer_norm_eps;           /* 1e-7 */
  int32_t position_buckets;       /* 256  */
  int32_t max_relative_positions; /* -1 in the config; the graph uses 512 (DeBERTa.swift:505) */
  int32_t pad_token_id;           /* 0    */
  int32_t vocab_size;             /* 128011 for the real checkpoint (DeBERTa.swift:199-202) */
  int32_t classifier_hidden;      /* 2048 (classifier.0: 1024 -> 2048) */
} gd_config;

/* DeBERTaV2Configuration.default (Configuration.swift:38-48). */
void gd_config_default(gd_config* config);

/* ------------------------------------------------------------------------ *
 * Fused kernels -- FusedKernels (FusedKernels.swift:7-286) and the default
 * graph ops they sit beside in GLiNERDecideClassifier.forward.
 * ------------------------------------------------------------------------ */

/* Flags for gd_residual_layer_norm. */
#define GD_LN_SUM_F16 1u /* round x + residual to fp16 before the norm: the default
                            graph `norm(x + residual)` (DeBERTa.swift:463).  Without it
                            the sum stays fp32 as in the Metal kernel
                            (FusedKernels.swift:137-152). */

/* out[r, :] = LayerNorm(x[r, :] + residual[r, :]) * gamma + beta, biased
 * variance, rsqrt(var + eps); fp16 I/O, fp32 arithmetic.  `residual` may be
 * NULL (plain LayerNorm, LayerNormWeight.callAsFunction, DeBERTa.swift:94-106).
 * `out` may alias `x` or `residual`.  cols must be a positive multiple of 8.
 * Replaces FusedKernels.residualLayerNorm (FusedKernels.swift:261-286). */
int gd_residual_layer_norm(const void* x, const void* residual, const void* gamma, const void* beta,
                           void* out, int64_t rows, int64_t cols, float eps, uint32_t flags,
                           void* stream);

/* Embedding stage (DeBERTa.swift:285-292): out[b, l, :] =
 * LayerNorm(table[ids[b, l], :]) * gamma + beta, times attention_mask[b, l]
 * (fp16).  ids outside [0, vocab) read row 0 and, when error_flag is not
 * NULL, set *error_flag (device int32) to 1.  hidden % 8 == 0. */
int gd_embedding_layer_norm(const int32_t* ids, const void* attention_mask, const void* table,
                            const void* gamma, const void* beta, void* out, int64_t batch,
                            int64_t seq_len, int64_t hidden, int64_t vocab, float eps,
                            int32_t* error_flag, void* stream);

/* Linear epilogues for gd_linear. */
typedef enum gd_epilogue {
  GD_EPI_NONE = 0,      /* C = A W^T                                   */
  GD_EPI_BIAS = 1,      /* C = A W^T + b  (addMM, DeBERTa.swift:69-71) */
  GD_EPI_BIAS_GELU = 2, /* C = gelu(fp16(A W^T + b)), exact erf GELU (MLXNN.gelu, DeBERTa.swift:421) */
  GD_EPI_BIAS_RELU = 3  /* C = relu(fp16(A W^T + b)) (MLXNN.relu, DeBERTa.swift:437) */
} gd_epilogue;

/* C[m, n] = epilogue(sum_k A[m, k] * W[n, k] (+ bias[n])), fp16 in/out, fp32
 * accumulation on MFMA.  W is [n, k] row-major (PyTorch Linear layout, as the
 * checkpoint stores it).  lda/ldc in elements.  Requires k % 64 == 0,
 * n % 128 == 0, lda % 8 == 0, ldc % 8 == 0, a, w and c 16-byte aligned.
 * When a_rows is not NULL, row m
 * of A is A[a_rows[m], :] (row gather; used for the marker gather,
 * DeBERTa.swift:431-436); gathered indices are clamped into [0, a_row_count).
 * The first GD_EPI_BIAS_GELU call on a device fills that device's GELU table
 * (a synchronous 72 KiB upload); made on a stream that is capturing a graph it
 * returns GD_ERR_UNSUPPORTED instead, so a caller that captures makes one
 * GELU call (or creates a classifier) on the device beforehand.
 * Replaces LinearWeight / FusedProjectionWeight addMM (DeBERTa.swift:60-92). */
int gd_linear(const void* a, const void* w, const void* bias, void* c, int64_t m, int64_t n,
              int64_t k, int64_t lda, int64_t ldc, const int32_t* a_rows, int64_t a_row_count,
              int32_t epilogue, void* stream);

/* Key-mask conventions for the attention kernels. */
#define GD_MASK_ATTENTION 0 /* fp16 attention mask [B, L]; key valid iff > 0 (DeBERTa.swift:329) */
#define GD_MASK_ADDITIVE 1  /* fp16 additive key mask [B, L]; key masked iff < -60000
                               (FusedKernels.swift:54,117) */

/* Relative-position bias with general index tensors, FusedKernels semantics:
 * out[b,h,q,k] = (q_bhq . pos_key[h, c2p[h,q,k]] + k_bhk . pos_query[h, p2c[h,k,q]]) * scale
 * in fp32, masked keys := -65504, fp16 output [B, H, L, L].
 * q, k: [B, H, L, D]; pos_key/pos_query: [H, P, D]; c2p/p2c: int32 [H, L, L];
 * key_mask: fp16 additive [B, L].
 * c2p_indices = p2c_indices = NULL selects the closed-form indices the
 * classifier builds (c2p[h,q,k] = p2c[h,k,q] = clip(bucket(q - k) + 256, 0,
 * 511), DeBERTa.swift:498-519) and runs them on the MFMA attention kernel
 * (D = 64, P = 512, L a multiple of 16 in [16, 512]).  Index tensors run on
 * the matrix cores too when D = 64, L is a multiple of 16 up to 512,
 * P <= 65536 and every operand is 16-byte aligned; otherwise on per-query
 * kernels.  Indices outside [0, P) read the nearest table row.
 * Replaces FusedKernels.relativeBias (FusedKernels.swift:83-123, 214-258). */
int gd_relative_bias(const void* q, const void* k, const void* pos_key, const void* pos_query,
                     const int32_t* c2p_indices, const int32_t* p2c_indices, const void* key_mask,
                     float scale, int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                     int64_t positions, void* out, void* stream);

/* Fully fused attention with general index tensors, FusedKernels semantics:
 * score = (q.k + q.pos_key[c2p] + k.pos_query[p2c]) * scale (fp32), masked
 * keys := -65504, softmax, out[b, q, h, :] = sum_k w v  -> [B, L, H, D] fp16.
 * NULL index tensors select the closed-form indices, as for
 * gd_relative_bias, on the MFMA attention kernel; index tensors take the
 * matrix cores under gd_relative_bias's conditions.
 * Replaces FusedKernels.fusedAttention (FusedKernels.swift:13-81, 160-210). */
int gd_fused_attention(const void* q, const void* k, const void* v, const void* pos_key,
                       const void* pos_query, const int32_t* c2p_indices,
                       const int32_t* p2c_indices, const void* key_mask, float scale,
                       int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                       int64_t positions, void* out, void* stream);

/* Strided view of a [B, H, L, D] tensor with contiguous D: element
 * (b, h, l, d) at base + b*stride_b + h*stride_h + l*stride_l + d. */
typedef struct gd_bhld {
  const void* data;
  int64_t stride_b, stride_h, stride_l;
} gd_bhld;

/* Strided view of a relative table [H, P, D] with contiguous D: element
 * (h, p, d) at base + h*stride_h + p*stride_p + d. */
typedef struct gd_table {
  const void* data;
  int64_t stride_h, stride_p;
} gd_table;

/* Outputs of gd_deberta_attention. */
#define GD_ATTN_OUT_PROBS 0   /* probabilities P [B, H, L, L] fp16 */
#define GD_ATTN_OUT_CONTEXT 1 /* context P.V as [B, L, H*D] fp16 (ldo = H*D) */
#define GD_ATTN_OUT_BIAS 2    /* the SDPA additive mask fp16(bias + key mask) [B, H, L, L] */

/* Score chains of gd_deberta_attention, OR'ed into `output` (one of them;
 * DEFAULT when none).  Each reproduces one graph of
 * GLiNERDecideClassifier.forward (DeBERTa.swift:322-410):
 *  DEFAULT   the default relative bias and SDPA with bias + key mask (:374-394)
 *  EXPLICIT  useFastAttention = false: fp16(fp16(q.k) / fp16(sqrt(3D))), the
 *            fp16 add of the default bias, masked keys := -65504, fp16
 *            probabilities, fp16(P.V) (:397-409)
 *  KERNEL_BIAS  useCustomRelativeKernel: bias = fp16((c2p + p2c) / sqrt(3D))
 *            with c2p, p2c in fp32 and masked keys := -65504
 *            (FusedKernels.swift:83-123), the whole SDPA mask (:383-385);
 *            with GD_ATTN_OUT_BIAS the output is that bias
 *  KERNEL_BIAS_EXPLICIT  useCustomRelativeKernel with useFastAttention =
 *            false: that bias added to the fp16 content score, no where
 *            (:397-405)
 *  FUSED     useFusedAttentionKernel: (q.k + c2p + p2c) / sqrt(3D) in fp32,
 *            masked keys excluded, softmax, P.V (FusedKernels.swift:13-81)
 * GD_ATTN_OUT_BIAS exists for DEFAULT and KERNEL_BIAS only. */
#define GD_ATTN_SCORE_DEFAULT 0x000
#define GD_ATTN_SCORE_EXPLICIT 0x100
#define GD_ATTN_SCORE_KERNEL_BIAS 0x200
#define GD_ATTN_SCORE_KERNEL_BIAS_EXPLICIT 0x300
#define GD_ATTN_SCORE_FUSED 0x400

/* Default-graph disentangled attention with closed-form log-bucket indices
 * (DeBERTa.swift:322-395, 498-551), one fused MFMA kernel:
 *   idx(q,k)  = clip(bucket(q - k) + 256, 0, 511)
 *   c2p       = fp16(q_q . pos_key[idx])           (c2pRaw, :374-375)
 *   p2c       = fp16(k_k . pos_query[idx])         (p2cRaw, :376-378)
 *   bias      = fp16(fp16(c2p + p2c) / fp16(sqrt(3 D)))   (:379)
 *   P         = softmax_k(q.k / sqrt(3 D) + bias) over valid keys only
 *               (key-only mask; padded query rows attend to valid keys)
 *   context   = P . V                              (SDPA, :386-394)
 * head_dim must be 64, seq_len a multiple of 16 in [16, 512], positions 512,
 * bucket_size 256; element strides below 2^31.  The first call on a device
 * fills that device's relative index table (a small kernel and a stream
 * synchronisation); made on a stream that is capturing a graph it returns
 * GD_ERR_UNSUPPORTED instead, so a caller that captures makes one attention
 * call (or creates a classifier) on the device beforehand.
 * `output` = GD_ATTN_OUT_* | GD_ATTN_SCORE_*.  Replaces the attention stage
 * of GLiNERDecideClassifier.forward (:322-410) under each of its flags. */
int gd_deberta_attention(gd_bhld q, gd_bhld k, gd_bhld v, gd_table pos_key, gd_table pos_query,
                         const void* mask, int32_t mask_kind, int64_t batch, int64_t heads,
                         int64_t seq_len, int64_t head_dim, int64_t positions,
                         int32_t bucket_size, int32_t output, void* out, int64_t ldo,
                         void* stream);

/* Writes the kernel's relative index idx(r) = clip(bucket(r) + bucket_size,
 * 0, 2*bucket_size-1) for r in [-(n-1), n-1] to out[r + n - 1] (device int32,
 * 2n-1 entries).  Exposes the device bucket math for parity tests
 * (makeRelativePositions, DeBERTa.swift:521-551). */
int gd_relative_index_table(int32_t* out, int32_t n, int32_t bucket_size, int32_t max_position,
                            void* stream);

/* ------------------------------------------------------------------------ *
 * Weight store -- WeightStore (Weights.swift:23-58)
 * ------------------------------------------------------------------------ */
typedef struct gd_weight_store gd_weight_store;

int gd_weight_store_create(gd_weight_store** store);
void gd_weight_store_destroy(gd_weight_store* store);
/* Adds (copies) one host tensor under `key`. */
int gd_weight_store_add(gd_weight_store* store, const char* key, const void* host_data,
                        int32_t dtype, const int64_t* shape, int32_t ndim);
/* Loads every tensor of a safetensors file (MLX loadArrays, Weights.swift:26-28). */
int gd_weight_store_load_safetensors(gd_weight_store* store, const char* path);
int64_t gd_weight_store_count(const gd_weight_store* store);
/* Looks up `key` (WeightStore.array's lookup, Weights.swift:35-57, without
 * the shape/dtype checks): writes its dtype (gd_dtype), rank (<= 8) and
 * shape (shape[0..ndim)), and a pointer to the store's host bytes, valid
 * until the store is destroyed or the key is replaced.  GD_ERR_MISSING_WEIGHT
 * when absent. */
int gd_weight_store_get(const gd_weight_store* store, const char* key, int32_t* dtype, int64_t* shape,
                        int32_t* ndim, const void** host_data, int64_t* nbytes);

/* ------------------------------------------------------------------------ *
 * Classifier context -- GLiNERDecideClassifier (DeBERTa.swift:156-447)
 * ------------------------------------------------------------------------ */
typedef struct gd_classifier gd_classifier;

/* Constructor flags mirroring GLiNERDecideClassifier.init (DeBERTa.swift:188-196). */
#define GD_USE_FUSED_KERNELS 1u    /* useFusedKernels: residual LN keeps x + residual in fp32 */
#define GD_USE_COMPILED_GRAPH 2u   /* useCompiledGraph: capture each shape's forward in a hipGraph */
#define GD_USE_GENERIC_ATTENTION 4u /* useFastAttention = false: the explicit-score path (:397-409) */
#define GD_USE_CUSTOM_RELATIVE_KERNEL 16u /* useCustomRelativeKernel: the relative-bias Metal kernel's
                                             bias (:357-372); residual LNs as GD_USE_FUSED_KERNELS */
#define GD_USE_FUSED_ATTENTION_KERNEL 32u /* useFusedAttentionKernel: the fused-attention Metal kernel
                                             (:337-354); residual LNs as GD_USE_FUSED_KERNELS */
/* No counterpart in the reference.  By default classify computes each row's
 * attention only up to its extent: the larger of (last position with
 * attention_mask > 0) + 1 and (last position a marker slot with
 * marker_mask > 0 reads) + 1.  Positions past the extent are masked keys and
 * feed no position before it, so the logits are the same; their hidden
 * states are not computed.  Likewise the last layer, whose only reader is
 * the classifier, computes its attention queries up to each row's last
 * marker and the rest of the layer on the marker rows alone (the logits
 * are bit-identical).  GD_FULL_ROWS computes every position of every layer,
 * as the reference's graph does (encode and layer_forward always do). */
#define GD_FULL_ROWS 8u

/* Loads and checks the weights (key names and shapes of
 * DeBERTa.swift:127-149, 199-208, 228-229), uploads them to the current
 * device, normalises the relative table and precomputes the per-layer
 * relative query/key projections (DeBERTa.swift:204-241). */
int gd_classifier_create(gd_classifier** out, const gd_weight_store* store, const gd_config* config,
                         uint32_t flags, void* stream);
void gd_classifier_destroy(gd_classifier* model);

/* Pre-allocates activation memory for batches up to max_batch x max_seq_len
 * with up to max_heads x max_options markers.  What is kept is the two
 * products: any later call with B*L <= max_batch*max_seq_len tokens and
 * B*Hh*O <= max_batch*max_heads*max_options markers fits without growing it
 * (growing it drops the captured graphs). */
int gd_classifier_reserve(gd_classifier* model, int64_t max_batch, int64_t max_seq_len,
                          int64_t max_heads, int64_t max_options);

/* classify (DeBERTa.swift:244-272) -> forward (:274-447).
 * input_ids int32 [B, L]; attention_mask fp16 [B, L] (1 = real token);
 * marker_indices int32 [B, Hh, O] (positions in [0, L)); marker_mask fp32
 * [B, Hh, O]; logits_out fp16 [B, Hh, O] (unused slots -10000).
 * seq_len must be a multiple of 16 in [16, 512] (the L32..L512 buckets). */
int gd_classifier_classify(gd_classifier* model, const int32_t* input_ids, const void* attention_mask,
                           const int32_t* marker_indices, const float* marker_mask, int64_t batch,
                           int64_t seq_len, int64_t max_heads, int64_t max_options, void* logits_out,
                           void* stream);

/* classify on packed rows.  No counterpart in the reference (it pads every
 * row to the bucket); the logits are those of gd_classifier_classify.  Row b's
 * extent is the larger of (last l with attention_mask[b, l] > 0) + 1 and
 * (last position read by a marker slot of row b with marker_mask > 0) + 1 (an
 * out-of-range marker reads position 0); only the extents' tokens run through
 * the embedding, the GEMMs and the LayerNorms, batch row after batch row.
 * total_tokens must equal the sum of the extents (0 <= total_tokens <= B * L):
 * the caller's tokenizer knows it; a different value sets the device error
 * flag (gd_classifier_check_device_errors reports GD_ERR_DEVICE_INDEX) and
 * leaves the logits undefined.  Same shapes and rules as gd_classifier_classify
 * otherwise; with GD_USE_COMPILED_GRAPH each shape is captured once per token
 * capacity (total_tokens rounded up to a multiple of 256, at most B * L), and
 * that graph serves every total up to the capacity. */
int gd_classifier_classify_packed(gd_classifier* model, const int32_t* input_ids, const void* attention_mask,
                                  const int32_t* marker_indices, const float* marker_mask, int64_t batch,
                                  int64_t seq_len, int64_t max_heads, int64_t max_options, int64_t total_tokens,
                                  void* logits_out, void* stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory at call time (code under hipGraph capture, tight serving loops,
 * harnesses that forbid hipMalloc): classify with the activation workspace in
 * the library's static device array instead of the context's workspace.  It
 * calls no hipMalloc / hipFree and captures no graph.  total_tokens = -1 runs
 * every row at B x L tokens (as gd_classifier_classify); total_tokens >= 0
 * runs packed rows (as gd_classifier_classify_packed, same rule for the
 * total).  The logits equal those of those entry points.
 * Limit: the call's buffers must fit the 48 MiB array -- at hidden 1024 /
 * intermediate 4096 / classifier 2048 that is up to 2048 tokens (B*L, or the
 * packed total) with up to 1024 marker slots (B*Hh*O); larger calls return
 * GD_ERR_SHAPE.  The array (one per GPU, held from the library's first use on
 * that GPU until the process ends) is shared by every context on that GPU
 * and keeps the last call's contents.  Calls on one GPU are ordered: each
 * waits, on its stream, for the work of the call made before it (a per-GPU
 * event), so calls from two streams, threads or contexts run one after the
 * other in the order they were made.  A call made during graph capture
 * records no such wait: replays of that graph race with other calls on the
 * same GPU unless the caller orders them.  The call captures cleanly once
 * the context exists (its tables are filled at creation). */
int gd_classifier_classify_static(gd_classifier* model, const int32_t* input_ids, const void* attention_mask,
                                  const int32_t* marker_indices, const float* marker_mask, int64_t batch,
                                  int64_t seq_len, int64_t max_heads, int64_t max_options, int64_t total_tokens,
                                  void* logits_out, void* stream);

/* Encoder only: writes the final hidden states [B, L, hidden] fp16 after
 * `num_layers` layers (num_layers < 0 = all). */
int gd_classifier_encode(gd_classifier* model, const int32_t* input_ids, const void* attention_mask,
                         int64_t batch, int64_t seq_len, int32_t num_layers, void* hidden_out,
                         void* stream);

/* One encoder layer (DeBERTa.swift:296-428) on caller hidden states:
 * hidden_out = layer_<layer_index>(hidden_in) for [B, L, hidden] fp16 with
 * the fp16 attention mask [B, L].  hidden_out may alias hidden_in; both are
 * 16-byte aligned (the layer reads and writes them in place: no staging). */
int gd_classifier_layer_forward(gd_classifier* model, int32_t layer_index, const void* hidden_in,
                                const void* attention_mask, int64_t batch, int64_t seq_len,
                                void* hidden_out, void* stream);

/* Per-stage profile (classify(collectProfile: true), DeBERTa.swift:466-496):
 * runs classify with an event pair around every stage, synchronises, and
 * writes up to `capacity` (name, milliseconds) records.  Names are
 * "embedding", "layer_<i>_attention_projection", "layer_<i>_attention",
 * "layer_<i>_attention_output", "layer_<i>_feed_forward", "classifier". */
typedef struct gd_profile_event {
  char name[48];
  double milliseconds;
} gd_profile_event;

int gd_classifier_classify_profiled(gd_classifier* model, const int32_t* input_ids,
                                    const void* attention_mask, const int32_t* marker_indices,
                                    const float* marker_mask, int64_t batch, int64_t seq_len,
                                    int64_t max_heads, int64_t max_options, void* logits_out,
                                    gd_profile_event* events, int32_t capacity, int32_t* count,
                                    void* stream);

/* Reads and clears the context's device error flag (synchronises `stream`).
 * Returns GD_ERR_DEVICE_INDEX if an input id or marker index was out of
 * range in any call since the last check, GD_OK otherwise. */
int gd_classifier_check_device_errors(gd_classifier* model, void* stream);

/* Device memory held by the context (weights + tables + workspace), bytes. */
int64_t gd_classifier_device_bytes(const gd_classifier* model);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif

#ifdef __cplusplus
}
#endif

#endif /* GLINER_DECIDE_H_ */
