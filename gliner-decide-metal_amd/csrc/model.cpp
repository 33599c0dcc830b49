// GLiNERDecideClassifier on gfx950: weights resident in HBM, the per-layer
// relative projections precomputed at load, and the encoder forward as a
// fixed sequence of the library's kernels on one stream.
//
// Reference: GLiNERDecideClassifier (DeBERTa.swift:156-447).
//   init      :188-242  weight assembly (fused QKV and rel-QK weights), rel
//                        table LayerNorm, 24 relative projections
//   classify  :244-272  compiled (MLX compile) or eager forward, eval = sync
//   forward   :274-447  embedding -> 24 x layer -> classifier
//   profile   :466-496  per-stage eval + wall time
//
// HBM layout (all fp16 unless noted), one allocation per tensor family:
//   word_embeddings [V, C]; emb LN gamma/beta [C]
//   per layer: qkv_w [3C, C] (query;key;value rows, as FusedProjectionWeight
//   concatenates them), qkv_b [3C], out_w [C, C], out_b, ln1 g/b,
//   inter_w [F, C], inter_b [F], ffn_w [C, F], ffn_b [C], ln2 g/b,
//   pos_qk [512, 2C] = LN(rel) [Wq;Wk]^T + [bq;bk]: columns [0, C) are the
//   relative queries (head h at h*D), [C, 2C) the relative keys.
//   classifier: cls0_w [2048, C], cls0_b, cls2_w [1, 2048], cls2_b [1].
// Workspace for T = B*L tokens: hidden [T, C], qkv [T, 3C] (Q | K | V per
// token, so head h of Q is at column h*D with row stride 3C), ctx [T, C],
// tmp [T, C], ffn [T, F], plus the marker rows / classifier inner buffers.
#include "model.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>

#include "gd_common.hpp"
#include "gd_kernels.hpp"

namespace gd {

namespace {

// Workspace of classify_static, the classify that allocates nothing: one copy
// of this array per GPU (each device holds it from the library's first use
// there until the process ends), shared by every context on that GPU.  Host
// code names it only in hipGetSymbolAddress; kernels take its per-device
// address (static_ws_base_).
constexpr size_t kStaticWorkspaceBytes = size_t(48) << 20;
static __device__ __align__(256) unsigned char scratch[kStaticWorkspaceBytes];
std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {};  // device address of `scratch`, per device
// Orders the static-workspace calls on one GPU: each call's first launch
// waits for the event the previous call recorded after its last launch, on
// whatever stream that call used, and the mutex keeps a call's wait, launches
// and record together.  Calls from two streams or threads then run one after
// the other in the order they were made, instead of overwriting each other's
// activations.
std::mutex g_static_call_mu[64];
hipEvent_t g_static_event[64] = {};

struct HipDeviceGuard {
  int prev = -1;
  explicit HipDeviceGuard(int dev) {
    if (hipGetDevice(&prev) == hipSuccess && prev != dev) (void)hipSetDevice(dev);
  }
  ~HipDeviceGuard() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

}  // namespace

Classifier::~Classifier() {
  release_graphs();
  for (void* p : allocations_) (void)hipFree(p);
  for (void* p : workspace_allocs_) (void)hipFree(p);
  if (capture_stream_) (void)hipStreamDestroy(capture_stream_);
}

void Classifier::release_graphs() {
  for (auto& kv : graphs_) {
    if (kv.second.exec) (void)hipGraphExecDestroy(kv.second.exec);
    if (kv.second.graph) (void)hipGraphDestroy(kv.second.graph);
  }
  graphs_.clear();
}

int Classifier::device_alloc(size_t bytes, void** out, std::vector<void*>& owner) {
  void* p = nullptr;
  if (bytes == 0) bytes = 256;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) {
    set_error("hipMalloc(%zu) failed: %s", bytes, hipGetErrorName(e));
    (void)hipGetLastError();
    return GD_ERR_OUT_OF_MEMORY;
  }
  owner.push_back(p);
  device_bytes_ += (int64_t)bytes;
  *out = p;
  return GD_OK;
}

int Classifier::upload(const WeightStore& store, const std::string& key, const std::vector<int64_t>& shape,
                       void** out, hipStream_t stream) {
  const HostTensor* t = nullptr;
  GD_RETURN_IF_ERROR(store.require(key, shape, GD_F16, &t));
  GD_RETURN_IF_ERROR(device_alloc(t->data.size(), out, allocations_));
  GD_HIP_CHECK(hipMemcpyAsync(*out, t->data.data(), t->data.size(), hipMemcpyHostToDevice, stream));
  return GD_OK;
}

// Concatenates several [rows_i, cols] fp16 tensors along dim 0 into one
// device tensor (FusedProjectionWeight, DeBERTa.swift:78-87).
int Classifier::upload_concat(const WeightStore& store, const std::vector<std::string>& keys,
                              const std::vector<std::vector<int64_t>>& shapes, void** out, hipStream_t stream) {
  size_t total = 0;
  std::vector<const HostTensor*> parts;
  for (size_t i = 0; i < keys.size(); ++i) {
    const HostTensor* t = nullptr;
    GD_RETURN_IF_ERROR(store.require(keys[i], shapes[i], GD_F16, &t));
    parts.push_back(t);
    total += t->data.size();
  }
  GD_RETURN_IF_ERROR(device_alloc(total, out, allocations_));
  size_t off = 0;
  for (const HostTensor* t : parts) {
    GD_HIP_CHECK(hipMemcpyAsync(static_cast<uint8_t*>(*out) + off, t->data.data(), t->data.size(),
                                hipMemcpyHostToDevice, stream));
    off += t->data.size();
  }
  return GD_OK;
}

std::vector<std::pair<std::string, std::vector<int64_t>>> required_weights(const gd_config& cfg) {
  const int64_t C = cfg.hidden_size, F = cfg.intermediate_size, V = cfg.vocab_size, CH = cfg.classifier_hidden;
  std::vector<std::pair<std::string, std::vector<int64_t>>> r = {
      {"encoder.embeddings.word_embeddings.weight", {V, C}},
      {"encoder.embeddings.LayerNorm.weight", {C}},
      {"encoder.embeddings.LayerNorm.bias", {C}},
      {"encoder.encoder.rel_embeddings.weight", {Classifier::kPositions, C}},
      {"encoder.encoder.LayerNorm.weight", {C}},
      {"encoder.encoder.LayerNorm.bias", {C}},
  };
  for (int i = 0; i < cfg.num_hidden_layers; ++i) {
    const std::string p = "encoder.encoder.layer." + std::to_string(i);
    for (const char* n : {"query", "key", "value"}) {
      r.push_back({p + ".attention.self." + n + "_proj.weight", {C, C}});
      r.push_back({p + ".attention.self." + n + "_proj.bias", {C}});
    }
    r.push_back({p + ".attention.output.dense.weight", {C, C}});
    r.push_back({p + ".attention.output.dense.bias", {C}});
    r.push_back({p + ".attention.output.LayerNorm.weight", {C}});
    r.push_back({p + ".attention.output.LayerNorm.bias", {C}});
    r.push_back({p + ".intermediate.dense.weight", {F, C}});
    r.push_back({p + ".intermediate.dense.bias", {F}});
    r.push_back({p + ".output.dense.weight", {C, F}});
    r.push_back({p + ".output.dense.bias", {C}});
    r.push_back({p + ".output.LayerNorm.weight", {C}});
    r.push_back({p + ".output.LayerNorm.bias", {C}});
  }
  r.push_back({"classifier.0.weight", {CH, C}});
  r.push_back({"classifier.0.bias", {CH}});
  r.push_back({"classifier.2.weight", {1, CH}});
  r.push_back({"classifier.2.bias", {1}});
  return r;
}

int Classifier::init(const WeightStore& store, const gd_config& cfg, uint32_t flags, hipStream_t stream) {
  cfg_ = cfg;
  flags_ = flags;
  const int64_t C = cfg.hidden_size, F = cfg.intermediate_size, H = cfg.num_attention_heads;
  const int64_t V = cfg.vocab_size, CH = cfg.classifier_hidden;
  GD_CHECK_ARG(C > 0 && H > 0 && C % H == 0, "hidden_size %lld must be a positive multiple of heads %lld",
               (long long)C, (long long)H);
  GD_CHECK_ARG(C / H == 64, "head size must be 64 (got %lld)", (long long)(C / H));
  GD_CHECK_ARG(C % 128 == 0 && F % 128 == 0 && CH % 128 == 0 && C % 64 == 0 && F % 64 == 0,
               "hidden/intermediate/classifier widths must be multiples of 128");
  GD_CHECK_ARG(cfg.num_hidden_layers > 0, "num_hidden_layers must be positive");
  GD_CHECK_ARG(V > 0, "vocab_size must be positive");
  GD_CHECK_ARG(cfg.position_buckets == 256, "position_buckets must be 256 (the graph hard-codes 256/512)");
  GD_CHECK_ARG(cfg.layer_norm_eps > 0.f, "layer_norm_eps must be positive");

  // Host-side check of every key, shape and dtype before any device work, so
  // a bad checkpoint fails without allocating (WeightStore.array checks,
  // Weights.swift:83-106).
  for (const auto& req : required_weights(cfg)) {
    const HostTensor* t = nullptr;
    GD_RETURN_IF_ERROR(store.require(req.first, req.second, GD_F16, &t));
  }
  GD_HIP_CHECK(hipGetDevice(&device_));
  GD_RETURN_IF_ERROR(init_static_workspace());    // this device's address of the no-alloc workspace
  GD_RETURN_IF_ERROR(ensure_gelu_table(stream));  // before any graph capture of the FFN
  GD_RETURN_IF_ERROR(ensure_relative_index_table(stream));  // and of the attention

  // ---- weights (DeBERTa.swift:197-229) ----
  GD_RETURN_IF_ERROR(upload(store, "encoder.embeddings.word_embeddings.weight", {V, C}, &word_emb_, stream));
  GD_RETURN_IF_ERROR(upload(store, "encoder.embeddings.LayerNorm.weight", {C}, &emb_g_, stream));
  GD_RETURN_IF_ERROR(upload(store, "encoder.embeddings.LayerNorm.bias", {C}, &emb_b_, stream));
  void *rel = nullptr, *rel_g = nullptr, *rel_b = nullptr;
  GD_RETURN_IF_ERROR(upload(store, "encoder.encoder.rel_embeddings.weight", {kPositions, C}, &rel, stream));
  GD_RETURN_IF_ERROR(upload(store, "encoder.encoder.LayerNorm.weight", {C}, &rel_g, stream));
  GD_RETURN_IF_ERROR(upload(store, "encoder.encoder.LayerNorm.bias", {C}, &rel_b, stream));
  layers_.resize(cfg.num_hidden_layers);
  for (int i = 0; i < cfg.num_hidden_layers; ++i) {
    const std::string p = "encoder.encoder.layer." + std::to_string(i);
    Layer& L = layers_[i];
    GD_RETURN_IF_ERROR(upload_concat(store,
                                     {p + ".attention.self.query_proj.weight", p + ".attention.self.key_proj.weight",
                                      p + ".attention.self.value_proj.weight"},
                                     {{C, C}, {C, C}, {C, C}}, &L.qkv_w, stream));
    GD_RETURN_IF_ERROR(upload_concat(store,
                                     {p + ".attention.self.query_proj.bias", p + ".attention.self.key_proj.bias",
                                      p + ".attention.self.value_proj.bias"},
                                     {{C}, {C}, {C}}, &L.qkv_b, stream));
    GD_RETURN_IF_ERROR(upload(store, p + ".attention.output.dense.weight", {C, C}, &L.out_w, stream));
    GD_RETURN_IF_ERROR(upload(store, p + ".attention.output.dense.bias", {C}, &L.out_b, stream));
    GD_RETURN_IF_ERROR(upload(store, p + ".attention.output.LayerNorm.weight", {C}, &L.ln1_g, stream));
    GD_RETURN_IF_ERROR(upload(store, p + ".attention.output.LayerNorm.bias", {C}, &L.ln1_b, stream));
    GD_RETURN_IF_ERROR(upload(store, p + ".intermediate.dense.weight", {F, C}, &L.inter_w, stream));
    GD_RETURN_IF_ERROR(upload(store, p + ".intermediate.dense.bias", {F}, &L.inter_b, stream));
    GD_RETURN_IF_ERROR(upload(store, p + ".output.dense.weight", {C, F}, &L.ffn_w, stream));
    GD_RETURN_IF_ERROR(upload(store, p + ".output.dense.bias", {C}, &L.ffn_b, stream));
    GD_RETURN_IF_ERROR(upload(store, p + ".output.LayerNorm.weight", {C}, &L.ln2_g, stream));
    GD_RETURN_IF_ERROR(upload(store, p + ".output.LayerNorm.bias", {C}, &L.ln2_b, stream));
  }
  GD_RETURN_IF_ERROR(upload(store, "classifier.0.weight", {CH, C}, &cls0_w_, stream));
  GD_RETURN_IF_ERROR(upload(store, "classifier.0.bias", {CH}, &cls0_b_, stream));
  GD_RETURN_IF_ERROR(upload(store, "classifier.2.weight", {1, CH}, &cls2_w_, stream));
  GD_RETURN_IF_ERROR(upload(store, "classifier.2.bias", {1}, &cls2_b_, stream));
  GD_RETURN_IF_ERROR(device_alloc(sizeof(int32_t), reinterpret_cast<void**>(&err_flag_), allocations_));
  GD_HIP_CHECK(hipMemsetAsync(err_flag_, 0, sizeof(int32_t), stream));

  // ---- relative precompute (DeBERTa.swift:208-227) ----
  void* rel_n = nullptr;
  std::vector<void*> scratch;
  GD_RETURN_IF_ERROR(device_alloc((size_t)kPositions * C * 2, &rel_n, scratch));
  int st = launch_residual_layer_norm(rel, nullptr, rel_g, rel_b, rel_n, kPositions, C, cfg.layer_norm_eps, 0, stream);
  for (int i = 0; st == GD_OK && i < cfg.num_hidden_layers; ++i) {
    st = device_alloc((size_t)kPositions * 2 * C * 2, &layers_[i].pos_qk, allocations_);
    if (st != GD_OK) break;
    // [posQ | posK] = relN [Wq; Wk]^T + [bq; bk]: the first 2C rows of qkv_w.
    st = launch_linear(rel_n, layers_[i].qkv_w, layers_[i].qkv_b, layers_[i].pos_qk, kPositions, 2 * C, C, C, 2 * C,
                       nullptr, 0, GD_EPI_BIAS, stream);
  }
  // The upload buffers are host memory: wait before returning.
  hipError_t e = hipStreamSynchronize(stream);
  for (void* p : scratch) (void)hipFree(p);
  device_bytes_ -= (int64_t)kPositions * C * 2;
  if (st != GD_OK) return st;
  if (e != hipSuccess) {
    set_error("relative precompute failed: %s", hipGetErrorName(e));
    return GD_ERR_HIP;
  }
  return GD_OK;
}

int Classifier::reserve(int64_t B, int64_t L, int64_t Hh, int64_t O) {
  const int64_t T = B * L, M = B * Hh * O;
  if (T <= ws_.tokens && M <= ws_.markers_cap) return GD_OK;
  const int64_t C = cfg_.hidden_size, F = cfg_.intermediate_size, CH = cfg_.classifier_hidden;
  const int64_t nt = std::max(T, ws_.tokens), nm = std::max(M, ws_.markers_cap);
  release_graphs();  // captured graphs reference the old workspace
  HipDeviceGuard guard(device_);
  (void)hipDeviceSynchronize();
  for (void* p : workspace_allocs_) {
    (void)hipFree(p);
  }
  workspace_allocs_.clear();
  device_bytes_ -= ws_bytes_;
  const int64_t before = device_bytes_;
  ws_ = Workspace{};
  auto A = [&](size_t bytes, void** p) { return device_alloc(bytes, p, workspace_allocs_); };
  GD_RETURN_IF_ERROR(A((size_t)nt * C * 2, &ws_.hidden));
  GD_RETURN_IF_ERROR(A((size_t)nt * 3 * C * 2, &ws_.qkv));
  GD_RETURN_IF_ERROR(A((size_t)nt * C * 2, &ws_.ctx));
  GD_RETURN_IF_ERROR(A((size_t)nt * C * 2, &ws_.tmp));
  GD_RETURN_IF_ERROR(A((size_t)nt * F * 2, &ws_.ffn));
  GD_RETURN_IF_ERROR(A((size_t)nm * 4, &ws_.marker_rows));
  GD_RETURN_IF_ERROR(A((size_t)nm * CH * 2, &ws_.inner));
  // staging for graph replays (inputs copied in, logits copied out)
  GD_RETURN_IF_ERROR(A((size_t)nt * 4, &ws_.ids));
  GD_RETURN_IF_ERROR(A((size_t)nt * 2, &ws_.mask));
  GD_RETURN_IF_ERROR(A((size_t)nm * 4, &ws_.markers));
  GD_RETURN_IF_ERROR(A((size_t)nm * 4, &ws_.marker_mask));
  GD_RETURN_IF_ERROR(A((size_t)nm * 2, &ws_.logits));
  GD_RETURN_IF_ERROR(A((size_t)nt * 4, &ws_.row_len));  // B <= B * L
  GD_RETURN_IF_ERROR(A((size_t)(nt + 1) * 4, &ws_.row_off));
  GD_RETURN_IF_ERROR(A((size_t)nt * 4, &ws_.row_map));
  // schedule slots: at most B * H * ceil(L / 128) items (<= nt * H / 16) plus a round
  const int64_t sched_cap = nt * std::max<int64_t>(cfg_.num_attention_heads, 16) / 16 + 1024;
  GD_RETURN_IF_ERROR(A((size_t)sched_cap * 4, &ws_.sched));
  GD_RETURN_IF_ERROR(A((size_t)nt * 4, &ws_.q_len));  // B <= B * L
  ws_bytes_ = device_bytes_ - before;
  ws_.tokens = nt;
  ws_.markers_cap = nm;
  ws_.sched_cap = sched_cap;
  return GD_OK;
}

// Takes this device's address of the static workspace, once per device (the
// device is current: init runs on it).
int Classifier::init_static_workspace() {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (device_ < 0 || device_ >= 64) return fail(GD_ERR_UNSUPPORTED, "device index out of range");
  if (!g_scratch_ptr[device_]) {
    void* p = nullptr;
    GD_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    hipEvent_t ev = nullptr;
    GD_HIP_CHECK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    g_static_event[device_] = ev;
    g_scratch_ptr[device_] = p;
  }
  static_ws_base_ = g_scratch_ptr[device_];
  return GD_OK;
}

// The forward's buffers for T tokens, M marker slots and B batch rows, laid
// out from `base` (each 256-byte aligned); returns the bytes they span.  No
// graph staging (the static path runs eagerly).  With base = nullptr only
// the size is computed.
int64_t Classifier::carve_workspace(Workspace& w, uint8_t* base, int64_t T, int64_t M, int64_t B,
                                    int64_t sched_slots) const {
  const int64_t C = cfg_.hidden_size, F = cfg_.intermediate_size, CH = cfg_.classifier_hidden;
  int64_t off = 0;
  auto take = [&](int64_t bytes, void** p) {
    *p = base ? base + off : nullptr;
    off += (bytes + 255) / 256 * 256;
  };
  take(T * C * 2, &w.hidden);
  take(T * 3 * C * 2, &w.qkv);
  take(T * C * 2, &w.ctx);
  take(T * C * 2, &w.tmp);
  take(T * F * 2, &w.ffn);
  take(M * 4, &w.marker_rows);
  take(M * CH * 2, &w.inner);
  take(B * 4, &w.row_len);
  take((B + 1) * 4, &w.row_off);
  take(T * 4, &w.row_map);
  take(sched_slots * 4, &w.sched);
  take(B * 4, &w.q_len);
  w.tokens = T;
  w.markers_cap = M;
  w.sched_cap = sched_slots;
  return off;
}

int Classifier::classify_static(const int32_t* ids, const void* mask, const int32_t* markers, const float* marker_mask,
                                int64_t B, int64_t L, int64_t Hh, int64_t O, void* logits, hipStream_t stream,
                                int64_t packed_tokens) {
  if (!static_ws_base_) return fail(GD_ERR_UNSUPPORTED, "the static workspace has no device address");
  const int64_t T = packed_tokens >= 0 ? packed_tokens : B * L, M = B * Hh * O;
  const int64_t slots = attention_schedule_slots(B, cfg_.num_attention_heads, L);
  Workspace w;
  const int64_t need = carve_workspace(w, nullptr, T, M, B, slots);
  if (need > (int64_t)kStaticWorkspaceBytes) {
    set_error("classify_static: %lld tokens and %lld marker slots need %lld bytes of workspace; the static "
              "workspace holds %zu (2048 tokens and 1024 marker slots at hidden 1024, intermediate 4096)",
              (long long)T, (long long)M, (long long)need, kStaticWorkspaceBytes);
    return GD_ERR_SHAPE;
  }
  carve_workspace(w, static_cast<uint8_t*>(static_ws_base_), T, M, B, slots);
  // Eager calls are ordered through the device's event.  Under graph capture
  // the wait and record are left out (an event recorded outside the capture
  // cannot join it): replays are ordered by whoever launches them.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  const bool capturing = hipStreamIsCapturing(stream, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone;
  std::lock_guard<std::mutex> lock(g_static_call_mu[device_]);
  hipEvent_t ev = g_static_event[device_];
  if (!capturing) GD_HIP_CHECK(hipStreamWaitEvent(stream, ev, 0));
  const int st = forward(w, ids, mask, markers, marker_mask, B, L, Hh, O, logits, stream, nullptr, packed_tokens);
  // recorded after a failed call too: later calls wait for what it enqueued
  if (!capturing) GD_HIP_CHECK(hipEventRecord(ev, stream));
  return st;
}

// One encoder layer (DeBERTa.swift:296-428).
int Classifier::layer_forward(const Workspace& w, int li, const void* mask, int64_t B, int64_t L, hipStream_t stream, StageHook* hook,
                              const Rows& rows, const int32_t* q_len, int64_t marker_count, const void* hidden_in) {
  const Layer& Ly = layers_[li];
  const int64_t C = cfg_.hidden_size, F = cfg_.intermediate_size, H = cfg_.num_attention_heads, D = C / H;
  const int64_t T = rows.tokens >= 0 ? rows.tokens : B * L;
  const float eps = cfg_.layer_norm_eps;
  // The reference holds a FusedKernels instance -- and its residual LN keeps
  // x + residual in fp32 -- whenever any of the three kernel flags is set
  // (DeBERTa.swift:230-232, 449-462).
  const bool metal_ln =
      (flags_ & (GD_USE_FUSED_KERNELS | GD_USE_CUSTOM_RELATIVE_KERNEL | GD_USE_FUSED_ATTENTION_KERNEL)) != 0;
  const uint32_t ln_flags = metal_ln ? 0u : GD_LN_SUM_F16;
  char name[48];

  const void* in = hidden_in ? hidden_in : w.hidden;
  if (hook) hook->begin(stream);
  // QKV projection (:298-320)
  GD_RETURN_IF_ERROR(launch_linear(in, Ly.qkv_w, Ly.qkv_b, w.qkv, T, 3 * C, C, C, 3 * C, nullptr, 0,
                                   GD_EPI_BIAS, stream));
  if (hook) {
    std::snprintf(name, sizeof name, "layer_%d_attention_projection", li);
    hook->end(name, stream);
    hook->begin(stream);
  }
  // relative bias + masked softmax + P.V (:322-410)
  AttentionArgs a{};
  const half_t* qkv = static_cast<const half_t*>(w.qkv);
  a.q = qkv;
  a.k = qkv + C;
  a.v = qkv + 2 * C;
  a.qsb = a.ksb = a.vsb = L * 3 * C;
  a.qsh = a.ksh = a.vsh = D;
  a.qsl = a.ksl = a.vsl = 3 * C;
  const half_t* pos = static_cast<const half_t*>(Ly.pos_qk);
  a.pq = pos;
  a.pk = pos + C;
  a.pqsh = a.pksh = D;
  a.pqsp = a.pksp = 2 * C;
  a.mask = mask;
  a.mask_kind = GD_MASK_ATTENTION;
  a.B = B;
  a.H = H;
  a.L = L;
  a.P = kPositions;
  a.bucket_size = cfg_.position_buckets;
  a.scale_qk = 1.0f / std::sqrt((float)(3 * D));
  a.scale16 = (float)(_Float16)std::sqrt((float)(3 * D));
  a.output = GD_ATTN_OUT_CONTEXT;
  // Score chain per the constructor flags (DeBERTa.swift:337-409): the fused
  // kernel returns before anything else; the custom relative kernel replaces
  // the bias; useFastAttention = false takes the explicit-score path.
  const bool explicit_scores = (flags_ & GD_USE_GENERIC_ATTENTION) != 0;
  if (flags_ & GD_USE_FUSED_ATTENTION_KERNEL)
    a.score = kScoreFused;
  else if (flags_ & GD_USE_CUSTOM_RELATIVE_KERNEL)
    a.score = explicit_scores ? kScoreKernelBiasExplicit : kScoreKernelBias;
  else
    a.score = explicit_scores ? kScoreExplicit : kScoreDefault;
  a.scale_rel = a.scale_qk;  // 1 / sqrt(3 D), the Metal kernels' `scale` (:347, :366)
  a.out = w.ctx;
  a.ldo = C;
  a.row_len = rows.len;
  a.row_off = rows.off;
  a.q_len = q_len;
  a.sched = q_len ? nullptr : rows.sched;  // the schedule's costs assume every query
  a.n_sched = q_len ? 0 : rows.n_sched;
  GD_RETURN_IF_ERROR(launch_deberta_attention(a, stream));
  if (hook) {
    std::snprintf(name, sizeof name, "layer_%d_attention", li);
    hook->end(name, stream);
    hook->begin(stream);
  }
  // Rows leaving the layer: all T in w.hidden (the first residual LN reads
  // the input rows and writes there), or the marker rows compact in w.qkv
  // (free once the attention has read Q, K and V): their context rows
  // (gathered into w.ffn, free until the FFN) go through the output
  // projection, their hidden rows are gathered for the residual; every later
  // step is row-wise.
  const bool compact = marker_count >= 0;
  const int64_t R = compact ? marker_count : T;
  void* hid = compact ? w.qkv : w.hidden;
  void* ctx = compact ? w.ffn : w.ctx;
  const void* res = compact ? hid : in;
  if (compact) {
    const int32_t* rows_m = static_cast<const int32_t*>(w.marker_rows);
    GD_RETURN_IF_ERROR(launch_gather_rows(w.ctx, rows_m, R, T, C, ctx, stream));
    GD_RETURN_IF_ERROR(launch_gather_rows(in, rows_m, R, T, C, hid, stream));
  }
  // output projection + residual LayerNorm (:412-418)
  GD_RETURN_IF_ERROR(
      launch_linear(ctx, Ly.out_w, Ly.out_b, w.tmp, R, C, C, C, C, nullptr, 0, GD_EPI_BIAS, stream));
  GD_RETURN_IF_ERROR(
      launch_residual_layer_norm(w.tmp, res, Ly.ln1_g, Ly.ln1_b, hid, R, C, eps, ln_flags, stream));
  if (hook) {
    std::snprintf(name, sizeof name, "layer_%d_attention_output", li);
    hook->end(name, stream);
    hook->begin(stream);
  }
  // feed-forward + residual LayerNorm (:420-427)
  GD_RETURN_IF_ERROR(
      launch_linear(hid, Ly.inter_w, Ly.inter_b, w.ffn, R, F, C, C, F, nullptr, 0, GD_EPI_BIAS_GELU, stream));
  GD_RETURN_IF_ERROR(
      launch_linear(w.ffn, Ly.ffn_w, Ly.ffn_b, w.tmp, R, C, F, F, C, nullptr, 0, GD_EPI_BIAS, stream));
  GD_RETURN_IF_ERROR(
      launch_residual_layer_norm(w.tmp, hid, Ly.ln2_g, Ly.ln2_b, hid, R, C, eps, ln_flags, stream));
  if (hook) {
    std::snprintf(name, sizeof name, "layer_%d_feed_forward", li);
    hook->end(name, stream);
  }
  return GD_OK;
}

int Classifier::encode_into_workspace(const Workspace& w, const int32_t* ids, const void* mask, int64_t B, int64_t L, int num_layers,
                                      hipStream_t stream, StageHook* hook, const Rows& rows) {
  const int64_t T = rows.tokens >= 0 ? rows.tokens : B * L;
  if (hook) hook->begin(stream);
  GD_RETURN_IF_ERROR(launch_embedding_layer_norm(ids, mask, word_emb_, emb_g_, emb_b_, w.hidden, T,
                                                 cfg_.hidden_size, cfg_.vocab_size, cfg_.layer_norm_eps, err_flag_,
                                                 stream, rows.map, B * L));
  if (hook) hook->end("embedding", stream);
  for (int i = 0; i < num_layers; ++i) GD_RETURN_IF_ERROR(layer_forward(w, i, mask, B, L, stream, hook, rows));
  return GD_OK;
}

int Classifier::forward(const Workspace& w, const int32_t* ids, const void* mask, const int32_t* markers, const float* marker_mask,
                        int64_t B, int64_t L, int64_t Hh, int64_t O, void* logits, hipStream_t stream,
                        StageHook* hook, int64_t packed_tokens, bool packed_exact) {
  const int64_t C = cfg_.hidden_size, CH = cfg_.classifier_hidden;
  const int64_t M = B * Hh * O;
  // Each row's attention stops at its extent (unless GD_FULL_ROWS): every
  // position the classifier reads lies before it, and positions past it are
  // masked keys that feed nothing before it.  Packed, every kernel runs on
  // the extents' tokens only, batch row after batch row.
  const bool packed = packed_tokens >= 0;
  Rows rows;
  if (packed || !(flags_ & GD_FULL_ROWS)) {
    rows.len = static_cast<const int32_t*>(w.row_len);
    GD_RETURN_IF_ERROR(launch_row_extent(mask, markers, marker_mask, B, L, Hh * O, static_cast<int32_t*>(w.row_len),
                                         stream));
  }
  if (packed) {
    rows.off = static_cast<const int32_t*>(w.row_off);
    rows.map = static_cast<const int32_t*>(w.row_map);
    rows.tokens = packed_tokens;
    GD_RETURN_IF_ERROR(launch_pack_rows(rows.len, B, L, packed_tokens, packed_exact,
                                        static_cast<int32_t*>(w.row_off), static_cast<int32_t*>(w.row_map),
                                        err_flag_, stream));
  }
  if (rows.len) {  // one item schedule for every layer's attention
    const int n = attention_schedule_slots(B, cfg_.num_attention_heads, L);
    if (n > 0 && n <= w.sched_cap) {
      GD_RETURN_IF_ERROR(launch_attention_schedule(rows.len, B, cfg_.num_attention_heads, L,
                                                   static_cast<int32_t*>(w.sched), stream));
      rows.sched = static_cast<const int32_t*>(w.sched);
      rows.n_sched = n;
    }
  }
  const int64_t T = packed ? packed_tokens : B * L;
  // The classifier reads the last layer's marker rows only: that layer runs
  // its queries up to each row's last marker and everything after the
  // attention on the M marker rows (unless GD_FULL_ROWS, or M > the
  // workspace's rows).  The logits are those of the full computation.
  const int N = cfg_.num_hidden_layers;
  const bool prune = rows.len != nullptr && !(flags_ & GD_FULL_ROWS) && N > 0 && M > 0 && M <= w.tokens;
  GD_RETURN_IF_ERROR(launch_marker_rows(markers, static_cast<int32_t*>(w.marker_rows), B, L, Hh * O, err_flag_,
                                        stream, rows.off));
  if (prune)
    GD_RETURN_IF_ERROR(
        launch_query_extent(markers, marker_mask, B, L, Hh * O, static_cast<int32_t*>(w.q_len), stream));
  GD_RETURN_IF_ERROR(encode_into_workspace(w, ids, mask, B, L, prune ? N - 1 : N, stream, hook, rows));
  if (prune)
    GD_RETURN_IF_ERROR(
        layer_forward(w, N - 1, mask, B, L, stream, hook, rows, static_cast<const int32_t*>(w.q_len), M));
  // classifier (:430-444)
  if (hook) hook->begin(stream);
  if (prune)
    GD_RETURN_IF_ERROR(launch_linear(w.qkv, cls0_w_, cls0_b_, w.inner, M, CH, C, C, CH, nullptr, 0,
                                     GD_EPI_BIAS_RELU, stream));
  else
    GD_RETURN_IF_ERROR(launch_linear(w.hidden, cls0_w_, cls0_b_, w.inner, M, CH, C, C, CH,
                                     static_cast<const int32_t*>(w.marker_rows), T > 0 ? T : 1, GD_EPI_BIAS_RELU,
                                     stream));
  GD_RETURN_IF_ERROR(launch_head_output(w.inner, cls2_w_, cls2_b_, marker_mask, logits, M, CH, stream));
  if (hook) hook->end("classifier", stream);
  return GD_OK;
}

int Classifier::classify(const int32_t* ids, const void* mask, const int32_t* markers, const float* marker_mask,
                         int64_t B, int64_t L, int64_t Hh, int64_t O, void* logits, hipStream_t stream,
                         int64_t packed_tokens) {
  GD_RETURN_IF_ERROR(reserve(B, L, Hh, O));
  if (!(flags_ & GD_USE_COMPILED_GRAPH))
    return forward(ws_, ids, mask, markers, marker_mask, B, L, Hh, O, logits, stream, nullptr, packed_tokens);

  // Compiled path (MLX compile, DeBERTa.swift:175-186, 249-261): the forward
  // for one shape is captured once into a hipGraph over the context's staging
  // buffers; each call copies the inputs in, replays it and copies the
  // logits out.
  const int64_t T = B * L, M = B * Hh * O;
  GD_HIP_CHECK(hipMemcpyAsync(ws_.ids, ids, (size_t)T * 4, hipMemcpyDeviceToDevice, stream));
  GD_HIP_CHECK(hipMemcpyAsync(ws_.mask, mask, (size_t)T * 2, hipMemcpyDeviceToDevice, stream));
  GD_HIP_CHECK(hipMemcpyAsync(ws_.markers, markers, (size_t)M * 4, hipMemcpyDeviceToDevice, stream));
  GD_HIP_CHECK(hipMemcpyAsync(ws_.marker_mask, marker_mask, (size_t)M * 4, hipMemcpyDeviceToDevice, stream));
  // Packed: one graph per token capacity (the total rounded up to 256, at
  // most B * L), not per total; the forward checks the sum against it.
  if (packed_tokens >= 0) {
    const int64_t cap = (packed_tokens + 255) / 256 * 256;
    packed_tokens = cap < T ? cap : T;
  }
  const ShapeKey key{B, L, Hh, O, packed_tokens};
  auto it = graphs_.find(key);
  if (it == graphs_.end()) {
    GraphEntry ge;
    // Capture on the context's own stream: the caller's stream may be the
    // legacy null stream, which cannot be captured.  Capturing enqueues no
    // work; the instantiated graph is launched on the caller's stream below.
    if (!capture_stream_) GD_HIP_CHECK(hipStreamCreateWithFlags(&capture_stream_, hipStreamNonBlocking));
    GD_HIP_CHECK(hipStreamBeginCapture(capture_stream_, hipStreamCaptureModeThreadLocal));
    int st = forward(ws_, static_cast<const int32_t*>(ws_.ids), ws_.mask, static_cast<const int32_t*>(ws_.markers),
                     static_cast<const float*>(ws_.marker_mask), B, L, Hh, O, ws_.logits, capture_stream_, nullptr,
                     packed_tokens, false);
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(capture_stream_, &graph);
    (void)hipGetLastError();
    if (st != GD_OK) {
      if (graph) (void)hipGraphDestroy(graph);
      return st;
    }
    if (e != hipSuccess) {
      set_error("graph capture failed: %s", hipGetErrorName(e));
      return GD_ERR_HIP;
    }
    ge.graph = graph;
    e = hipGraphInstantiate(&ge.exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
      (void)hipGraphDestroy(graph);
      set_error("graph instantiate failed: %s", hipGetErrorName(e));
      return GD_ERR_HIP;
    }
    it = graphs_.emplace(key, ge).first;
  }
  GD_HIP_CHECK(hipGraphLaunch(it->second.exec, stream));
  GD_HIP_CHECK(hipMemcpyAsync(logits, ws_.logits, (size_t)M * 2, hipMemcpyDeviceToDevice, stream));
  return GD_OK;
}

int Classifier::encode(const int32_t* ids, const void* mask, int64_t B, int64_t L, int num_layers, void* hidden_out,
                       hipStream_t stream) {
  GD_RETURN_IF_ERROR(reserve(B, L, 1, 1));
  const int n = num_layers < 0 ? cfg_.num_hidden_layers : std::min(num_layers, cfg_.num_hidden_layers);
  GD_RETURN_IF_ERROR(encode_into_workspace(ws_, ids, mask, B, L, n, stream, nullptr, Rows{}));
  GD_HIP_CHECK(hipMemcpyAsync(hidden_out, ws_.hidden, (size_t)B * L * cfg_.hidden_size * 2, hipMemcpyDeviceToDevice,
                              stream));
  return GD_OK;
}

int Classifier::layer(int li, const void* hidden_in, const void* mask, int64_t B, int64_t L, void* hidden_out,
                      hipStream_t stream) {
  GD_CHECK_ARG(li >= 0 && li < cfg_.num_hidden_layers, "layer index %d out of range", li);
  GD_RETURN_IF_ERROR(reserve(B, L, 1, 1));
  // The layer reads hidden_in and its first residual LN writes hidden_out,
  // which then serves as the layer's hidden rows: no staging copies.
  Workspace w = ws_;
  w.hidden = hidden_out;
  return layer_forward(w, li, mask, B, L, stream, nullptr, Rows{}, nullptr, -1, hidden_in);
}

namespace {

struct EventHook : StageHook {
  struct Rec {
    std::string name;
    hipEvent_t a, b;
  };
  std::vector<Rec> recs;
  hipEvent_t pending = nullptr;
  int status = GD_OK;
  void begin(hipStream_t s) override {
    if (hipEventCreate(&pending) != hipSuccess || hipEventRecord(pending, s) != hipSuccess) status = GD_ERR_HIP;
  }
  void end(const char* name, hipStream_t s) override {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess || hipEventRecord(e, s) != hipSuccess) {
      status = GD_ERR_HIP;
      return;
    }
    recs.push_back({name, pending, e});
    pending = nullptr;
  }
  ~EventHook() override {
    for (auto& r : recs) {
      (void)hipEventDestroy(r.a);
      (void)hipEventDestroy(r.b);
    }
    if (pending) (void)hipEventDestroy(pending);
  }
};

}  // namespace

int Classifier::classify_profiled(const int32_t* ids, const void* mask, const int32_t* markers,
                                  const float* marker_mask, int64_t B, int64_t L, int64_t Hh, int64_t O, void* logits,
                                  gd_profile_event* events, int capacity, int* count, hipStream_t stream) {
  GD_RETURN_IF_ERROR(reserve(B, L, Hh, O));
  EventHook hook;
  GD_RETURN_IF_ERROR(forward(ws_, ids, mask, markers, marker_mask, B, L, Hh, O, logits, stream, &hook));
  if (hook.status != GD_OK) return fail(GD_ERR_HIP, "event record failed");
  GD_HIP_CHECK(hipStreamSynchronize(stream));
  int n = 0;
  for (auto& r : hook.recs) {
    if (n >= capacity) break;
    float ms = 0.f;
    GD_HIP_CHECK(hipEventElapsedTime(&ms, r.a, r.b));
    std::snprintf(events[n].name, sizeof events[n].name, "%s", r.name.c_str());
    events[n].milliseconds = ms;
    ++n;
  }
  *count = n;
  return GD_OK;
}

int Classifier::check_device_errors(hipStream_t stream) {
  int32_t host = 0;
  GD_HIP_CHECK(hipMemcpyAsync(&host, err_flag_, sizeof host, hipMemcpyDeviceToHost, stream));
  GD_HIP_CHECK(hipStreamSynchronize(stream));
  if (host) {
    GD_HIP_CHECK(hipMemsetAsync(err_flag_, 0, sizeof(int32_t), stream));
    GD_HIP_CHECK(hipStreamSynchronize(stream));
    return fail(GD_ERR_DEVICE_INDEX, "an input id or marker index was out of range (row 0 / position 0 was used)");
  }
  return GD_OK;
}

}  // namespace gd
