// GLiNERDecideClassifier context (DeBERTa.swift:156-447).
#pragma once

#include <hip/hip_runtime.h>

#include <map>
#include <string>
#include <tuple>
#include <utility>
#include <vector>

#include "gliner_decide.h"
#include "weights.hpp"

namespace gd {

// Every (key, shape) the classifier needs, in checkpoint names.
std::vector<std::pair<std::string, std::vector<int64_t>>> required_weights(const gd_config& cfg);

// Per-stage timing hook (the reference `stage` / `stage3` wrappers).
struct StageHook {
  virtual ~StageHook() = default;
  virtual void begin(hipStream_t s) = 0;
  virtual void end(const char* name, hipStream_t s) = 0;
};

class Classifier {
 public:
  static constexpr int64_t kPositions = 512;  // DeBERTa.swift:205-206, :505

  ~Classifier();
  int init(const WeightStore& store, const gd_config& cfg, uint32_t flags, hipStream_t stream);
  int reserve(int64_t B, int64_t L, int64_t Hh, int64_t O);
  // packed_tokens >= 0: the forward runs on packed rows (the sum of the row
  // extents, which it must equal); -1: every row is B x L tokens.
  int classify(const int32_t* ids, const void* mask, const int32_t* markers, const float* marker_mask, int64_t B,
               int64_t L, int64_t Hh, int64_t O, void* logits, hipStream_t stream, int64_t packed_tokens = -1);
  // classify with the workspace in the library's static device array (no
  // allocation, no graph); GD_ERR_SHAPE when the call's buffers exceed it.
  int classify_static(const int32_t* ids, const void* mask, const int32_t* markers, const float* marker_mask,
                      int64_t B, int64_t L, int64_t Hh, int64_t O, void* logits, hipStream_t stream,
                      int64_t packed_tokens);
  int classify_profiled(const int32_t* ids, const void* mask, const int32_t* markers, const float* marker_mask,
                        int64_t B, int64_t L, int64_t Hh, int64_t O, void* logits, gd_profile_event* events,
                        int capacity, int* count, hipStream_t stream);
  int encode(const int32_t* ids, const void* mask, int64_t B, int64_t L, int num_layers, void* hidden_out,
             hipStream_t stream);
  int layer(int li, const void* hidden_in, const void* mask, int64_t B, int64_t L, void* hidden_out,
            hipStream_t stream);
  int check_device_errors(hipStream_t stream);
  int64_t device_bytes() const { return device_bytes_; }
  const gd_config& config() const { return cfg_; }

 private:
  struct Layer {
    void *qkv_w = nullptr, *qkv_b = nullptr, *out_w = nullptr, *out_b = nullptr, *ln1_g = nullptr, *ln1_b = nullptr;
    void *inter_w = nullptr, *inter_b = nullptr, *ffn_w = nullptr, *ffn_b = nullptr, *ln2_g = nullptr,
         *ln2_b = nullptr;
    void* pos_qk = nullptr;
  };
  struct Workspace {
    void *hidden = nullptr, *qkv = nullptr, *ctx = nullptr, *tmp = nullptr, *ffn = nullptr;
    void *marker_rows = nullptr, *inner = nullptr;
    void* row_len = nullptr;  // int32 [B]: per-row attention extents of classify
    void* row_off = nullptr;  // int32 [B + 1]: packed rows: first token row of each batch row
    void* row_map = nullptr;  // int32 [T]: packed rows: token index b * L + l of each packed row
    void* sched = nullptr;    // int32 [sched_cap]: attention item schedule under row extents
    void* q_len = nullptr;    // int32 [B]: last marker position + 1 per batch row (classify's last layer)
    void *ids = nullptr, *mask = nullptr, *markers = nullptr, *marker_mask = nullptr, *logits = nullptr;
    int64_t tokens = 0, markers_cap = 0, sched_cap = 0;  // capacities: T, B*Hh*O, schedule slots
  };
  using ShapeKey = std::tuple<int64_t, int64_t, int64_t, int64_t, int64_t>;  // B, L, Hh, O, packed tokens
  struct GraphEntry {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
  };

  int device_alloc(size_t bytes, void** out, std::vector<void*>& owner);
  int upload(const WeightStore& store, const std::string& key, const std::vector<int64_t>& shape, void** out,
             hipStream_t stream);
  int upload_concat(const WeightStore& store, const std::vector<std::string>& keys,
                    const std::vector<std::vector<int64_t>>& shapes, void** out, hipStream_t stream);
  // Rows: every (b, l) without `rows`; with it, the row extents and (packed)
  // the offsets, the row map and the token count.
  struct Rows {
    const int32_t* len = nullptr;
    const int32_t* off = nullptr;
    const int32_t* map = nullptr;
    int64_t tokens = -1;
    const int32_t* sched = nullptr;
    int n_sched = 0;
  };
  // marker_count >= 0: only the marker rows ws_.marker_rows[0, marker_count)
  // leave the layer, compact (row i = marker slot i) in ws_.qkv; attention
  // queries stop at q_len[b] (the classifier reads nothing else of the last
  // layer).
  // hidden_in (optional): the layer's input rows when they are not w.hidden;
  // the output is written to w.hidden either way.
  int layer_forward(const Workspace& w, int li, const void* mask, int64_t B, int64_t L, hipStream_t stream, StageHook* hook,
                    const Rows& rows, const int32_t* q_len = nullptr, int64_t marker_count = -1,
                    const void* hidden_in = nullptr);
  int encode_into_workspace(const Workspace& w, const int32_t* ids, const void* mask, int64_t B, int64_t L, int num_layers,
                            hipStream_t stream, StageHook* hook, const Rows& rows);
  // packed_exact = false: packed_tokens is a capacity >= the extents' sum.
  int forward(const Workspace& w, const int32_t* ids, const void* mask, const int32_t* markers, const float* marker_mask, int64_t B,
              int64_t L, int64_t Hh, int64_t O, void* logits, hipStream_t stream, StageHook* hook,
              int64_t packed_tokens = -1, bool packed_exact = true);
  void release_graphs();
  int init_static_workspace();
  int64_t carve_workspace(Workspace& w, uint8_t* base, int64_t T, int64_t M, int64_t B, int64_t sched_slots) const;

  gd_config cfg_{};
  uint32_t flags_ = 0;
  int device_ = 0;
  std::vector<void*> allocations_;
  std::vector<void*> workspace_allocs_;
  int64_t device_bytes_ = 0;
  int64_t ws_bytes_ = 0;
  void *word_emb_ = nullptr, *emb_g_ = nullptr, *emb_b_ = nullptr;
  std::vector<Layer> layers_;
  void *cls0_w_ = nullptr, *cls0_b_ = nullptr, *cls2_w_ = nullptr, *cls2_b_ = nullptr;
  int32_t* err_flag_ = nullptr;
  Workspace ws_;
  void* static_ws_base_ = nullptr;  // this device's address of the static workspace
  std::map<ShapeKey, GraphEntry> graphs_;
  hipStream_t capture_stream_ = nullptr;  // default priority, non-blocking
};

}  // namespace gd
