// The tokenizer.json pipeline the decision front end runs on each schema
// entry and word: normaliser -> Metaspace pre-tokenizer -> Unigram Viterbi ->
// ids, with `add_special_tokens = false` and no added-token matching (the
// front end cuts added tokens out of the text before calling it).
//
// The reference runs this pipeline through swift-transformers 1.3.4
// (Package.resolved:76-82; NativeTokenizer.swift:63, 183-190) and states that
// the tokenizer JSON of the upstream DebertaV2Tokenizer stays exact
// (NativeTokenizer.swift:256-259).  The upstream semantics restated here are
// those of HF `tokenizers` (the library the checkpoint's tokenizer.json was
// written by), component by component:
//   Strip          trims White_Space code points at either end;
//   Precompiled    sentencepiece's precompiled charsmap (a darts-clone double
//                  array over UTF-8 keys plus a blob of NUL-terminated
//                  replacements), applied per extended grapheme cluster: a
//                  cluster shorter than 6 bytes whose bytes start with a key
//                  is replaced by the replacement of the shortest such key;
//                  otherwise each code point is looked up on its own;
//   Replace        literal pattern, or a run `c{n,}` / `c+` of one character;
//   Lowercase      the full lower-case mapping of each code point;
//   NFC/NFD/NFKC/NFKD  Unicode normal forms;
//   Metaspace      ' ' -> replacement, the replacement prepended (scheme
//                  always; or never) and, with split, a new piece at every
//                  replacement character;
//   WhitespaceSplit  pieces split at White_Space code points, which are dropped;
//   WordLevel      one vocabulary entry per piece, else unk_token;
//   Unigram        Viterbi over byte positions: every vocabulary piece that
//                  starts at a code point boundary is an edge scored by its
//                  log-probability; a code point no single piece covers gets
//                  an unknown edge scored min(score) - 10; ties keep the
//                  first candidate (shorter pieces, earlier starts); runs of
//                  unknown pieces are fused into one unknown token.
#pragma once

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "json.hpp"

namespace gdf {

// An error with a gd_status code.
struct FrontendError : std::runtime_error {
  int code;
  FrontendError(int c, const std::string& msg) : std::runtime_error(msg), code(c) {}
};

// UTF-8 helpers (the input is validated once at the C-ABI boundary).
bool valid_utf8(const char* s, size_t n);
// Length in bytes of the code point starting with lead byte `c`.
inline int utf8_len(unsigned char c) { return c < 0x80 ? 1 : (c < 0xE0 ? 2 : (c < 0xF0 ? 3 : 4)); }
uint32_t utf8_decode(const char* s, int len);
void utf8_append(std::string& out, uint32_t cp);

class Tokenizer {
 public:
  // Reads the "normalizer", "pre_tokenizer", "model" and "added_tokens"
  // members of a parsed tokenizer.json.  Unsupported components throw
  // FrontendError(GD_ERR_UNSUPPORTED).
  explicit Tokenizer(const Json& root);
  ~Tokenizer();
  Tokenizer(const Tokenizer&) = delete;
  Tokenizer& operator=(const Tokenizer&) = delete;

  // Appends the ids of `text` (valid UTF-8).
  void encode(const std::string& text, std::vector<int32_t>& ids) const;
  // The normalised text and its pre-tokenized pieces (for tests).
  std::string normalize(const std::string& text) const;
  std::vector<std::string> pre_tokenize(const std::string& normalized) const;
  // Unigram pieces of one pre-tokenized piece (Unigram model only).
  std::vector<std::string> unigram_pieces(const std::string& piece) const;

  // Model vocabulary lookup (Unigram pieces or WordLevel entries), -1 when
  // absent.
  int32_t vocab_id(const std::string& token) const;
  int32_t unk_id() const { return unk_id_; }
  // `added_tokens` as (content, id) in file order.
  const std::vector<std::pair<std::string, int32_t>>& added_tokens() const { return added_; }

  // One normaliser component (defined in tokenizer.cpp).
  struct Step;

 private:
  std::vector<Step> steps_;
  // Pre-tokenizer steps in order: Metaspace or WhitespaceSplit.
  struct PreStep {
    bool metaspace = false;
    std::string replacement;
    int prepend = 0;  // 0 never, 1 always
    bool split = true;
  };
  std::vector<PreStep> pre_;
  // Model: Unigram, or WordLevel (every pre-tokenized piece one vocabulary
  // entry, else unk_token).
  bool word_level_ = false;
  std::unordered_map<std::string, int32_t> words_;
  std::string unk_token_;
  // Unigram
  void load_unigram(const Json& model);
  std::vector<std::string> pieces_;
  std::vector<double> scores_;
  std::unordered_map<std::string, int32_t> piece_id_;
  std::unordered_map<uint64_t, int32_t> edges_;  // (node << 8 | byte) -> child node
  std::vector<int32_t> node_piece_;              // piece id ending at a node, or -1
  double min_score_ = 0.0;
  int32_t unk_id_ = -1;
  std::vector<std::pair<std::string, int32_t>> added_;
};

}  // namespace gdf
