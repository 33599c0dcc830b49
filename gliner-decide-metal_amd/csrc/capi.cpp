// extern "C" entry points of include/gliner_decide.h: argument validation
// (the reference's `precondition` checks become status codes) and dispatch
// to the launchers / classifier context.
#include <cmath>
#include <cstring>
#include <new>
#include <stdexcept>

#include "gd_common.hpp"
#include "gd_kernels.hpp"
#include "model.hpp"
#include "weights.hpp"
#include "gliner_decide_diag.h"

struct gd_weight_store {
  gd::WeightStore impl;
};
struct gd_classifier {
  gd::Classifier impl;
};

namespace gd {

namespace {
thread_local std::string g_last_error;
}

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
}
const char* last_error() { return g_last_error.c_str(); }
void clear_error() { g_last_error.clear(); }

namespace {

inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }
inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace
}  // namespace gd

using namespace gd;

extern "C" {

const char* gd_last_error(void) { return last_error(); }
int gd_abi_version(void) { return GD_ABI_VERSION; }
const char* gd_build_info(void) {
  return "gliner-decide-mi355x: gfx950 HIP kernels (MFMA f16, wave64); ABI " "1";
}

void gd_config_default(gd_config* c) {
  if (!c) return;
  c->hidden_size = 1024;
  c->intermediate_size = 4096;
  c->num_hidden_layers = 24;
  c->num_attention_heads = 16;
  c->layer_norm_eps = 1e-7f;
  c->position_buckets = 256;
  c->max_relative_positions = -1;
  c->pad_token_id = 0;
  c->vocab_size = 128011;
  c->classifier_hidden = 2048;
}

int gd_residual_layer_norm(const void* x, const void* residual, const void* gamma, const void* beta, void* out,
                           int64_t rows, int64_t cols, float eps, uint32_t flags, void* stream) {
  clear_error();
  GD_CHECK_SHAPE(rows >= 0, "rows must be >= 0 (got %lld)", (long long)rows);
  GD_CHECK_SHAPE(cols > 0 && cols % 8 == 0, "cols must be a positive multiple of 8 (got %lld)", (long long)cols);
  GD_CHECK_ARG(eps > 0.f && std::isfinite(eps), "eps must be positive and finite");
  GD_CHECK_ARG((flags & ~GD_LN_SUM_F16) == 0, "unknown flags 0x%x", flags);
  if (rows == 0) return GD_OK;  // nothing to do; empty tensors may carry null pointers
  GD_CHECK_ARG(x && gamma && beta && out, "null tensor pointer");
  return launch_residual_layer_norm(x, residual, gamma, beta, out, rows, cols, eps, flags, as_stream(stream));
}

int gd_embedding_layer_norm(const int32_t* ids, const void* attention_mask, const void* table, const void* gamma,
                            const void* beta, void* out, int64_t batch, int64_t seq_len, int64_t hidden,
                            int64_t vocab, float eps, int32_t* error_flag, void* stream) {
  clear_error();
  GD_CHECK_SHAPE(batch >= 0 && seq_len >= 0, "negative batch or sequence length");
  GD_CHECK_SHAPE(hidden > 0 && hidden % 8 == 0, "hidden must be a positive multiple of 8 (got %lld)",
                 (long long)hidden);
  GD_CHECK_SHAPE(vocab > 0, "vocab must be positive");
  GD_CHECK_ARG(eps > 0.f && std::isfinite(eps), "eps must be positive and finite");
  if (batch * seq_len == 0) return GD_OK;
  GD_CHECK_ARG(ids && attention_mask && table && gamma && beta && out, "null tensor pointer");
  return launch_embedding_layer_norm(ids, attention_mask, table, gamma, beta, out, batch * seq_len, hidden, vocab, eps,
                                     error_flag, as_stream(stream));
}

int gd_linear(const void* a, const void* w, const void* bias, void* c, int64_t m, int64_t n, int64_t k, int64_t lda,
              int64_t ldc, const int32_t* a_rows, int64_t a_row_count, int32_t epilogue, void* stream) {
  clear_error();
  GD_CHECK_ARG(m == 0 || (a && w && c), "null tensor pointer");
  GD_CHECK_ARG(epilogue >= GD_EPI_NONE && epilogue <= GD_EPI_BIAS_RELU, "unknown epilogue %d", epilogue);
  GD_CHECK_ARG(epilogue == GD_EPI_NONE || bias, "epilogue %d needs a bias", epilogue);
  GD_CHECK_SHAPE(m >= 0 && m <= 0x7fffffff, "m out of range (%lld)", (long long)m);
  GD_CHECK_SHAPE(n > 0 && n % 128 == 0 && n <= 0x7fffffff, "n must be a positive multiple of 128 (got %lld)",
                 (long long)n);
  GD_CHECK_SHAPE(k > 0 && k % 64 == 0 && k <= 0x7fffffff, "k must be a positive multiple of 64 (got %lld)",
                 (long long)k);
  GD_CHECK_SHAPE(lda >= k && lda % 8 == 0, "lda must be >= k and a multiple of 8");
  GD_CHECK_SHAPE(ldc >= n && ldc % 8 == 0, "ldc must be >= n and a multiple of 8");
  GD_CHECK_ARG(aligned(a, 16) && aligned(w, 16), "a and w must be 16-byte aligned");
  GD_CHECK_ARG(aligned(c, 16), "c must be 16-byte aligned");
  GD_CHECK_SHAPE(!a_rows || (a_row_count > 0 && a_row_count <= 0x7fffffff), "a_row_count must be positive with a_rows");
  return launch_linear(a, w, bias, c, m, n, k, lda, ldc, a_rows, a_rows ? a_row_count : m, epilogue,
                       as_stream(stream));
}

namespace {

// Checks a closed-form-index attention call and launches it (shared by
// gd_deberta_attention and the closed-form paths of gd_relative_bias /
// gd_fused_attention).
int deberta_attention_checked(gd_bhld q, gd_bhld k, gd_bhld v, gd_table pos_key, gd_table pos_query,
                              const void* mask, int32_t mask_kind, int64_t batch, int64_t heads, int64_t seq_len,
                              int64_t head_dim, int64_t positions, int32_t bucket_size, int32_t output, int score,
                              float scale_rel, void* out, int64_t ldo, hipStream_t stream) {
  GD_CHECK_ARG(q.data && k.data && pos_key.data && pos_query.data && mask && out, "null tensor pointer");
  GD_CHECK_ARG(output == GD_ATTN_OUT_PROBS || output == GD_ATTN_OUT_CONTEXT || output == GD_ATTN_OUT_BIAS,
               "unknown output kind %d", output);
  GD_CHECK_ARG(score >= kScoreDefault && score <= kScoreFused, "unknown score chain %d", score);
  GD_CHECK_ARG(output != GD_ATTN_OUT_BIAS || score == kScoreDefault || score == kScoreKernelBias,
               "the bias output exists for the default and the kernel-bias score chains only");
  GD_CHECK_ARG(output != GD_ATTN_OUT_CONTEXT || v.data, "context output needs v");
  GD_CHECK_ARG(mask_kind == GD_MASK_ATTENTION || mask_kind == GD_MASK_ADDITIVE, "unknown mask kind %d", mask_kind);
  GD_CHECK_SHAPE(head_dim == 64, "head_dim must be 64 (got %lld)", (long long)head_dim);
  GD_CHECK_SHAPE(seq_len >= 16 && seq_len <= 512 && seq_len % 16 == 0,
                 "seq_len must be a multiple of 16 in [16, 512] (got %lld)", (long long)seq_len);
  GD_CHECK_SHAPE(positions == 512 && bucket_size == 256, "positions must be 512 and bucket_size 256");
  GD_CHECK_SHAPE(batch >= 0 && heads > 0 && batch * heads * ((seq_len + 63) / 64) <= 0x7fffffff, "bad batch/heads");
  const gd_bhld* views[3] = {&q, &k, &v};
  for (int i = 0; i < (output == GD_ATTN_OUT_CONTEXT ? 3 : 2); ++i) {
    const gd_bhld* t = views[i];
    GD_CHECK_ARG(aligned(t->data, 16) && t->stride_b % 8 == 0 && t->stride_h % 8 == 0 && t->stride_l % 8 == 0,
                 "q/k/v must be 16-byte aligned with strides that are multiples of 8 elements");
  }
  GD_CHECK_ARG(aligned(pos_key.data, 16) && aligned(pos_query.data, 16) && pos_key.stride_h % 8 == 0 &&
                   pos_key.stride_p % 8 == 0 && pos_query.stride_h % 8 == 0 && pos_query.stride_p % 8 == 0,
               "relative tables must be 16-byte aligned with strides that are multiples of 8 elements");
  GD_CHECK_ARG(aligned(mask, 8), "mask must be 8-byte aligned");
  if (output == GD_ATTN_OUT_CONTEXT) {
    GD_CHECK_ARG(ldo >= heads * head_dim, "ldo must be >= heads * head_dim");
  }
  if (batch == 0) return GD_OK;
  AttentionArgs a{};
  a.q = q.data;
  a.k = k.data;
  a.v = v.data ? v.data : q.data;
  a.qsb = q.stride_b;
  a.qsh = q.stride_h;
  a.qsl = q.stride_l;
  a.ksb = k.stride_b;
  a.ksh = k.stride_h;
  a.ksl = k.stride_l;
  a.vsb = v.stride_b;
  a.vsh = v.stride_h;
  a.vsl = v.stride_l;
  a.pk = pos_key.data;
  a.pq = pos_query.data;
  a.pksh = pos_key.stride_h;
  a.pksp = pos_key.stride_p;
  a.pqsh = pos_query.stride_h;
  a.pqsp = pos_query.stride_p;
  a.mask = mask;
  a.mask_kind = mask_kind;
  a.B = batch;
  a.H = heads;
  a.L = seq_len;
  a.P = positions;
  a.bucket_size = bucket_size;
  a.scale_qk = 1.0f / std::sqrt((float)(3 * head_dim));
  a.scale16 = (float)(_Float16)std::sqrt((float)(3 * head_dim));
  a.output = output;
  a.score = score;
  a.scale_rel = scale_rel;
  a.out = out;
  a.ldo = ldo;
  return launch_deberta_attention(a, stream);
}

}  // namespace

int gd_relative_bias(const void* q, const void* k, const void* pos_key, const void* pos_query,
                     const int32_t* c2p_indices, const int32_t* p2c_indices, const void* key_mask, float scale,
                     int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim, int64_t positions, void* out,
                     void* stream) {
  clear_error();
  GD_CHECK_ARG(q && k && pos_key && pos_query && key_mask && out, "null tensor pointer");
  GD_CHECK_ARG((c2p_indices == nullptr) == (p2c_indices == nullptr),
               "give both index tensors, or neither for the closed-form indices");
  GD_CHECK_SHAPE(batch >= 0 && heads > 0 && seq_len > 0 && head_dim > 0 && positions > 0,
                 "dimensions must be positive");
  if (c2p_indices == nullptr) {
    // Closed-form indices (the ones the classifier builds, DeBERTa.swift:498-519):
    // the MFMA attention kernel's kernel-bias chain with the bias output.
    const int64_t HLD = heads * seq_len * head_dim, LD = seq_len * head_dim;
    return deberta_attention_checked(gd_bhld{q, HLD, LD, head_dim}, gd_bhld{k, HLD, LD, head_dim}, gd_bhld{},
                                     gd_table{pos_key, positions * head_dim, head_dim},
                                     gd_table{pos_query, positions * head_dim, head_dim}, key_mask, GD_MASK_ADDITIVE,
                                     batch, heads, seq_len, head_dim, positions, 256, GD_ATTN_OUT_BIAS,
                                     kScoreKernelBias, scale, out, seq_len, as_stream(stream));
  }
  GD_CHECK_SHAPE(head_dim <= 4096, "head_dim too large");
  GD_CHECK_SHAPE(batch * heads * seq_len <= 0x7fffffff, "too many rows");
  return launch_relative_bias_general(q, k, pos_key, pos_query, c2p_indices, p2c_indices, key_mask, scale, batch,
                                      heads, seq_len, head_dim, positions, out, nullptr, as_stream(stream));
}

int gd_fused_attention(const void* q, const void* k, const void* v, const void* pos_key, const void* pos_query,
                       const int32_t* c2p_indices, const int32_t* p2c_indices, const void* key_mask, float scale,
                       int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim, int64_t positions, void* out,
                       void* stream) {
  clear_error();
  GD_CHECK_ARG(q && k && v && pos_key && pos_query && key_mask && out, "null tensor pointer");
  GD_CHECK_ARG((c2p_indices == nullptr) == (p2c_indices == nullptr),
               "give both index tensors, or neither for the closed-form indices");
  GD_CHECK_SHAPE(batch >= 0 && heads > 0 && seq_len > 0 && head_dim > 0 && positions > 0,
                 "dimensions must be positive");
  if (c2p_indices == nullptr) {
    // Closed-form indices: the MFMA attention kernel's fused chain; its
    // context rows [B, L, H*D] are the [B, L, H, D] output.
    const int64_t HLD = heads * seq_len * head_dim, LD = seq_len * head_dim;
    return deberta_attention_checked(gd_bhld{q, HLD, LD, head_dim}, gd_bhld{k, HLD, LD, head_dim},
                                     gd_bhld{v, HLD, LD, head_dim}, gd_table{pos_key, positions * head_dim, head_dim},
                                     gd_table{pos_query, positions * head_dim, head_dim}, key_mask, GD_MASK_ADDITIVE,
                                     batch, heads, seq_len, head_dim, positions, 256, GD_ATTN_OUT_CONTEXT,
                                     kScoreFused, scale, out, heads * head_dim, as_stream(stream));
  }
  GD_CHECK_SHAPE((head_dim + seq_len) * 4 <= 64 * 1024, "seq_len + head_dim exceed the kernel's LDS budget");
  GD_CHECK_SHAPE(batch * heads * seq_len <= 0x7fffffff, "too many rows");
  return launch_fused_attention_general(q, k, v, pos_key, pos_query, c2p_indices, p2c_indices, key_mask, scale, batch,
                                        heads, seq_len, head_dim, positions, out, nullptr, as_stream(stream));
}

int gd_deberta_attention(gd_bhld q, gd_bhld k, gd_bhld v, gd_table pos_key, gd_table pos_query, const void* mask,
                         int32_t mask_kind, int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                         int64_t positions, int32_t bucket_size, int32_t output, void* out, int64_t ldo,
                         void* stream) {
  clear_error();
  const int32_t kind = output & 0xff, score = (output >> 8) & 0xff;
  GD_CHECK_ARG((output & ~0xffff) == 0, "unknown output bits 0x%x", output);
  // the Metal kernels' scale: 1 / sqrt(3 D) in fp32 (DeBERTa.swift:347,366)
  const float scale_rel = head_dim > 0 ? 1.0f / std::sqrt((float)(3 * head_dim)) : 0.f;
  return deberta_attention_checked(q, k, v, pos_key, pos_query, mask, mask_kind, batch, heads, seq_len, head_dim,
                                   positions, bucket_size, kind, score, scale_rel, out, ldo, as_stream(stream));
}

int gd_stream_probe_add(const void* a, const void* b, void* c, int64_t n, void* stream) {
  clear_error();
  GD_CHECK_ARG(n == 0 || (a && b && c), "null tensor pointer");
  GD_CHECK_SHAPE(n >= 0 && n % 32 == 0, "n must be a non-negative multiple of 32");
  GD_CHECK_ARG(aligned(a, 16) && aligned(b, 16) && aligned(c, 16), "pointers must be 16-byte aligned");
  return launch_stream_probe_add(a, b, c, n, as_stream(stream));
}

int gd_diag_mfma_forms(const void* a, const void* w, const float* c0, float* d32, float* d16, int64_t tiles,
                       void* stream) {
  clear_error();
  GD_CHECK_ARG(tiles == 0 || (a && w && c0 && d32 && d16), "null tensor pointer");
  GD_CHECK_SHAPE(tiles >= 0 && tiles <= (int64_t{1} << 20), "tiles must be in [0, 2^20]");
  return launch_mfma_forms(a, w, c0, d32, d16, tiles, as_stream(stream));
}

int gd_relative_index_table(int32_t* out, int32_t n, int32_t bucket_size, int32_t max_position, void* stream) {
  clear_error();
  GD_CHECK_ARG(out, "null output");
  GD_CHECK_SHAPE(n > 0 && n <= 512, "n must be in [1, 512]");
  GD_CHECK_ARG(bucket_size == 256 && max_position == 512, "only bucket_size 256 / max_position 512 are supported");
  return launch_relative_index_table(out, n, bucket_size, max_position, as_stream(stream));
}

int gd_weight_store_create(gd_weight_store** store) {
  clear_error();
  GD_CHECK_ARG(store, "null output pointer");
  *store = new (std::nothrow) gd_weight_store();
  if (!*store) return fail(GD_ERR_OUT_OF_MEMORY, "allocation failed");
  return GD_OK;
}

void gd_weight_store_destroy(gd_weight_store* store) { delete store; }

int gd_weight_store_add(gd_weight_store* store, const char* key, const void* host_data, int32_t dtype,
                        const int64_t* shape, int32_t ndim) {
  clear_error();
  GD_CHECK_ARG(store && key, "null store or key");
  try {
    return store->impl.add(key, host_data, dtype, shape, ndim);
  } catch (const std::bad_alloc&) {
    return fail(GD_ERR_OUT_OF_MEMORY, "host allocation failed");
  } catch (const std::exception& e) {
    set_error("weight store: %s", e.what());
    return GD_ERR_INVALID_ARGUMENT;
  }
}

int gd_weight_store_load_safetensors(gd_weight_store* store, const char* path) {
  clear_error();
  GD_CHECK_ARG(store && path, "null store or path");
  try {
    return store->impl.load_safetensors(path);
  } catch (const std::bad_alloc&) {
    return fail(GD_ERR_OUT_OF_MEMORY, "host allocation failed");
  } catch (const std::exception& e) {
    set_error("%s: %s", path, e.what());
    return GD_ERR_IO;
  }
}

int64_t gd_weight_store_count(const gd_weight_store* store) {
  return store ? (int64_t)store->impl.tensors.size() : 0;
}

int gd_weight_store_get(const gd_weight_store* store, const char* key, int32_t* dtype, int64_t* shape,
                        int32_t* ndim, const void** host_data, int64_t* nbytes) {
  clear_error();
  GD_CHECK_ARG(store && key && dtype && shape && ndim && host_data && nbytes, "null argument");
  const gd::HostTensor* t = store->impl.find(key);
  if (!t) {
    set_error("Missing model weight: %s", key);
    return GD_ERR_MISSING_WEIGHT;
  }
  *dtype = t->dtype;
  *ndim = (int32_t)t->shape.size();
  for (size_t i = 0; i < t->shape.size() && i < 8; ++i) shape[i] = t->shape[i];
  *host_data = t->data.data();
  *nbytes = (int64_t)t->data.size();
  return GD_OK;
}

int gd_classifier_create(gd_classifier** out, const gd_weight_store* store, const gd_config* config, uint32_t flags,
                         void* stream) {
  clear_error();
  GD_CHECK_ARG(out && store, "null output or store");
  GD_CHECK_ARG((flags & ~(GD_USE_FUSED_KERNELS | GD_USE_COMPILED_GRAPH | GD_USE_GENERIC_ATTENTION | GD_FULL_ROWS |
                          GD_USE_CUSTOM_RELATIVE_KERNEL | GD_USE_FUSED_ATTENTION_KERNEL)) == 0,
               "unknown flags 0x%x", flags);
  gd_config cfg;
  if (config) {
    cfg = *config;
  } else {
    gd_config_default(&cfg);
  }
  *out = nullptr;
  gd_classifier* m = new (std::nothrow) gd_classifier();
  if (!m) return fail(GD_ERR_OUT_OF_MEMORY, "allocation failed");
  int st;
  try {
    st = m->impl.init(store->impl, cfg, flags, as_stream(stream));
  } catch (const std::bad_alloc&) {
    st = fail(GD_ERR_OUT_OF_MEMORY, "host allocation failed");
  }
  if (st != GD_OK) {
    std::string msg = last_error();
    delete m;
    set_error("%s", msg.c_str());
    return st;
  }
  *out = m;
  return GD_OK;
}

void gd_classifier_destroy(gd_classifier* model) { delete model; }

static int check_forward_args(const gd_classifier* model, const void* ids, const void* mask, int64_t batch,
                              int64_t seq_len) {
  GD_CHECK_ARG(model && ids && mask, "null model or input");
  GD_CHECK_SHAPE(batch >= 1 && batch <= 65536, "batch must be in [1, 65536] (got %lld)", (long long)batch);
  GD_CHECK_SHAPE(seq_len >= 16 && seq_len <= 512 && seq_len % 16 == 0,
                 "seq_len must be a multiple of 16 in [16, 512] (got %lld)", (long long)seq_len);
  GD_CHECK_ARG(aligned(mask, 8), "attention_mask must be 8-byte aligned");
  return GD_OK;
}

int gd_classifier_reserve(gd_classifier* model, int64_t max_batch, int64_t max_seq_len, int64_t max_heads,
                          int64_t max_options) {
  clear_error();
  GD_CHECK_ARG(model, "null model");
  GD_CHECK_SHAPE(max_batch > 0 && max_seq_len > 0 && max_heads > 0 && max_options > 0, "sizes must be positive");
  return model->impl.reserve(max_batch, max_seq_len, max_heads, max_options);
}

int gd_classifier_classify(gd_classifier* model, const int32_t* input_ids, const void* attention_mask,
                           const int32_t* marker_indices, const float* marker_mask, int64_t batch, int64_t seq_len,
                           int64_t max_heads, int64_t max_options, void* logits_out, void* stream) {
  clear_error();
  GD_RETURN_IF_ERROR(check_forward_args(model, input_ids, attention_mask, batch, seq_len));
  GD_CHECK_ARG(marker_indices && marker_mask && logits_out, "null marker or output pointer");
  GD_CHECK_SHAPE(max_heads >= 1 && max_options >= 1 && batch * max_heads * max_options <= (1 << 24),
                 "bad marker shape");
  return model->impl.classify(input_ids, attention_mask, marker_indices, marker_mask, batch, seq_len, max_heads,
                              max_options, logits_out, as_stream(stream));
}

int gd_classifier_classify_packed(gd_classifier* model, const int32_t* input_ids, const void* attention_mask,
                                  const int32_t* marker_indices, const float* marker_mask, int64_t batch,
                                  int64_t seq_len, int64_t max_heads, int64_t max_options, int64_t total_tokens,
                                  void* logits_out, void* stream) {
  clear_error();
  GD_RETURN_IF_ERROR(check_forward_args(model, input_ids, attention_mask, batch, seq_len));
  GD_CHECK_ARG(marker_indices && marker_mask && logits_out, "null marker or output pointer");
  GD_CHECK_SHAPE(max_heads >= 1 && max_options >= 1 && batch * max_heads * max_options <= (1 << 24),
                 "bad marker shape");
  GD_CHECK_SHAPE(total_tokens >= 0 && total_tokens <= batch * seq_len, "total_tokens %lld outside [0, %lld]",
                 (long long)total_tokens, (long long)(batch * seq_len));
  return model->impl.classify(input_ids, attention_mask, marker_indices, marker_mask, batch, seq_len, max_heads,
                              max_options, logits_out, as_stream(stream), total_tokens);
}

int gd_classifier_classify_static(gd_classifier* model, const int32_t* input_ids, const void* attention_mask,
                                  const int32_t* marker_indices, const float* marker_mask, int64_t batch,
                                  int64_t seq_len, int64_t max_heads, int64_t max_options, int64_t total_tokens,
                                  void* logits_out, void* stream) {
  clear_error();
  GD_RETURN_IF_ERROR(check_forward_args(model, input_ids, attention_mask, batch, seq_len));
  GD_CHECK_ARG(marker_indices && marker_mask && logits_out, "null marker or output pointer");
  GD_CHECK_SHAPE(max_heads >= 1 && max_options >= 1 && batch * max_heads * max_options <= (1 << 24),
                 "bad marker shape");
  GD_CHECK_SHAPE(total_tokens >= -1 && total_tokens <= batch * seq_len, "total_tokens %lld outside [-1, %lld]",
                 (long long)total_tokens, (long long)(batch * seq_len));
  return model->impl.classify_static(input_ids, attention_mask, marker_indices, marker_mask, batch, seq_len, max_heads,
                                     max_options, logits_out, as_stream(stream), total_tokens);
}

int gd_classifier_encode(gd_classifier* model, const int32_t* input_ids, const void* attention_mask, int64_t batch,
                         int64_t seq_len, int32_t num_layers, void* hidden_out, void* stream) {
  clear_error();
  GD_RETURN_IF_ERROR(check_forward_args(model, input_ids, attention_mask, batch, seq_len));
  GD_CHECK_ARG(hidden_out, "null output pointer");
  return model->impl.encode(input_ids, attention_mask, batch, seq_len, num_layers, hidden_out, as_stream(stream));
}

int gd_classifier_layer_forward(gd_classifier* model, int32_t layer_index, const void* hidden_in,
                                const void* attention_mask, int64_t batch, int64_t seq_len, void* hidden_out,
                                void* stream) {
  clear_error();
  GD_RETURN_IF_ERROR(check_forward_args(model, hidden_in, attention_mask, batch, seq_len));
  GD_CHECK_ARG(hidden_out, "null output pointer");
  GD_CHECK_ARG(aligned(hidden_in, 16) && aligned(hidden_out, 16), "hidden_in and hidden_out must be 16-byte aligned");
  return model->impl.layer(layer_index, hidden_in, attention_mask, batch, seq_len, hidden_out, as_stream(stream));
}

int gd_classifier_classify_profiled(gd_classifier* model, const int32_t* input_ids, const void* attention_mask,
                                    const int32_t* marker_indices, const float* marker_mask, int64_t batch,
                                    int64_t seq_len, int64_t max_heads, int64_t max_options, void* logits_out,
                                    gd_profile_event* events, int32_t capacity, int32_t* count, void* stream) {
  clear_error();
  GD_RETURN_IF_ERROR(check_forward_args(model, input_ids, attention_mask, batch, seq_len));
  GD_CHECK_ARG(marker_indices && marker_mask && logits_out && events && count, "null pointer");
  GD_CHECK_SHAPE(max_heads >= 1 && max_options >= 1 && batch * max_heads * max_options <= (1 << 24),
                 "bad marker shape");
  int n = 0;
  int st = model->impl.classify_profiled(input_ids, attention_mask, marker_indices, marker_mask, batch, seq_len,
                                         max_heads, max_options, logits_out, events, capacity, &n, as_stream(stream));
  *count = n;
  return st;
}

int gd_classifier_check_device_errors(gd_classifier* model, void* stream) {
  clear_error();
  GD_CHECK_ARG(model, "null model");
  return model->impl.check_device_errors(as_stream(stream));
}

int64_t gd_classifier_device_bytes(const gd_classifier* model) { return model ? model->impl.device_bytes() : 0; }

}  // extern "C"
