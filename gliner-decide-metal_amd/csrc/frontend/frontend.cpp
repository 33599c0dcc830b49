// `NativeDecisionTokenizer` (NativeTokenizer.swift:56-227) and its C-ABI
// (include/gliner_decide_frontend.h): the classification-schema formatter,
// word split, special-token cut and bucket choice over the tokenizer.json
// pipeline of tokenizer.cpp.
#include <unicode/brkiter.h>
#include <unicode/regex.h>
#include <unicode/unistr.h>
#include <unicode/ustring.h>
#include <unicode/utf16.h>

#include <algorithm>
#include <cstring>
#include <fstream>
#include <mutex>
#include <sstream>
#include <string>
#include <unordered_map>
#include <vector>

#include "gliner_decide.h"
#include "gliner_decide_frontend.h"
#include "json.hpp"
#include "tokenizer.hpp"

namespace gdf {
namespace {

thread_local std::string g_error;

int fail(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

// NativeTokenizer.swift:69-72, compiled case-insensitive by ICU as
// NSRegularExpression compiles it.
const char* const kWordPattern =
    "(?:https?://[^\\s]+|www\\.[^\\s]+)|[a-z0-9._%+-]+@[a-z0-9.-]+\\.[a-z]{2,}|@[a-z0-9_]+|\\w+(?:[-_]\\w+)*|\\S";

struct Task {
  std::string name;
  std::vector<std::string> labels;
  bool has_prompt = false;
  std::string prompt;
  std::vector<std::pair<std::string, std::string>> descriptions;  // labelDescriptions (last duplicate wins)

  const std::string* description(const std::string& label) const {
    const std::string* d = nullptr;
    for (const auto& kv : descriptions)
      if (kv.first == label) d = &kv.second;
    return d;
  }
};

std::string bucket_list(const std::vector<int64_t>& b) {
  std::string s = "[";
  for (size_t i = 0; i < b.size(); ++i) s += (i ? ", " : "") + std::to_string(b[i]);
  return s + "]";
}

}  // namespace

class DecisionFrontend {
 public:
  explicit DecisionFrontend(const Json& tokenizer_json) : tok_(tokenizer_json) {
    for (const auto& kv : tok_.added_tokens()) special_[kv.first] = kv.second;  // last duplicate wins
    for (const auto& kv : special_)
      if (!kv.first.empty()) cut_.push_back(kv.first);
    auto pad = special_.find("[PAD]");
    if (pad != special_.end()) {
      pad_id_ = pad->second;
    } else {
      const int32_t v = tok_.vocab_id("[PAD]");
      pad_id_ = v >= 0 ? v : 0;
    }
    UErrorCode st = U_ZERO_ERROR;
    UParseError pe;
    pattern_.reset(icu::RegexPattern::compile(icu::UnicodeString::fromUTF8(kWordPattern), UREGEX_CASE_INSENSITIVE,
                                              pe, st));
    if (U_FAILURE(st) || !pattern_) throw FrontendError(GD_ERR_UNSUPPORTED, "ICU regex unavailable");
  }

  const Tokenizer& tokenizer() const { return tok_; }
  int32_t pad_id() const { return pad_id_; }

  // NativeTokenizer.swift:193-208: a final '.' unless the last character
  // (grapheme cluster) is '.', '!' or '?'; the word pattern's matches, each
  // lower-cased code point by code point.
  std::vector<std::string> split_words(const std::string& text) const {
    icu::UnicodeString u = icu::UnicodeString::fromUTF8(text);
    bool ends_ok = false;
    if (u.length() > 0) {
      thread_local std::unique_ptr<icu::BreakIterator> bi;  // ICU iterators are per thread
      if (!bi) {
        UErrorCode st = U_ZERO_ERROR;
        bi.reset(icu::BreakIterator::createCharacterInstance(icu::Locale::getRoot(), st));
        if (U_FAILURE(st) || !bi) throw FrontendError(GD_ERR_UNSUPPORTED, "ICU character break iterator unavailable");
      }
      bi->setText(u);
      const int32_t last = bi->last();
      const int32_t prev = bi->previous();
      if (last - prev == 1) {
        const UChar c = u.charAt(prev);
        ends_ok = c == u'.' || c == u'!' || c == u'?';
      }
    }
    if (u.length() == 0)
      u = icu::UnicodeString(u".");
    else if (!ends_ok)
      u.append((UChar)u'.');
    UErrorCode st = U_ZERO_ERROR;
    std::unique_ptr<icu::RegexMatcher> m(pattern_->matcher(u, st));
    if (U_FAILURE(st)) throw FrontendError(GD_ERR_UNSUPPORTED, "ICU regex matcher unavailable");
    std::vector<std::string> words;
    while (m->find(st) && U_SUCCESS(st)) {
      const int32_t a = m->start(st), b = m->end(st);
      std::string w;
      for (int32_t i = a; i < b;) {
        UChar32 c;
        U16_NEXT(u.getBuffer(), i, b, c);
        lower_append(w, (uint32_t)c);
      }
      words.push_back(std::move(w));
    }
    if (U_FAILURE(st)) throw FrontendError(GD_ERR_UNSUPPORTED, "ICU regex search failed");
    return words;
  }

  // NativeTokenizer.swift:159-191: added tokens cut out first (leftmost
  // occurrence, the longer token on a tie), the text between through the
  // tokenizer.  Each entry's ids are a pure function of its text, kept in a
  // bounded cache.
  void append_tokenized(const std::string& text, std::vector<int32_t>& ids) {
    auto hit = cache_.find(text);
    if (hit == cache_.end()) {
      std::vector<int32_t> out;
      size_t cursor = 0;
      while (cursor < text.size()) {
        size_t best = std::string::npos;
        const std::string* tok = nullptr;
        for (const std::string& t : cut_) {
          const size_t f = text.find(t, cursor);
          if (f == std::string::npos) continue;
          if (best == std::string::npos || f < best || (f == best && t.size() > tok->size())) {
            best = f;
            tok = &t;
          }
        }
        if (tok == nullptr) {
          tok_.encode(text.substr(cursor), out);
          break;
        }
        if (best > cursor) tok_.encode(text.substr(cursor, best - cursor), out);
        out.push_back(special_.at(*tok));
        cursor = best + tok->size();
      }
      if (cache_.size() >= kCacheSize) cache_.clear();
      hit = cache_.emplace(text, std::move(out)).first;
    }
    ids.insert(ids.end(), hit->second.begin(), hit->second.end());
  }

  // makeInput (NativeTokenizer.swift:76-157) up to the padding: the unpadded
  // ids and the label-marker positions of each task.
  void encode_schema(const std::string& text, const std::vector<Task>& tasks, std::vector<int32_t>& ids,
                     std::vector<std::vector<int64_t>>& markers) {
    struct Entry {
      std::string text;
      int label_task;
    };
    std::vector<Entry> combined;
    for (size_t ti = 0; ti < tasks.size(); ++ti) {
      const Task& t = tasks[ti];
      std::string prompt = t.has_prompt ? t.name + ": " + t.prompt : t.name;
      for (const std::string& label : t.labels)
        if (const std::string* d = t.description(label)) prompt += " [DESCRIPTION] " + label + ": " + *d;
      combined.push_back({"(", -1});
      combined.push_back({"[P]", -1});
      combined.push_back({prompt, -1});
      combined.push_back({"(", -1});
      for (const std::string& label : t.labels) {
        combined.push_back({"[L]", (int)ti});
        combined.push_back({label, -1});
      }
      combined.push_back({")", -1});
      combined.push_back({")", -1});
      if (ti + 1 < tasks.size()) combined.push_back({"[SEP_STRUCT]", -1});
    }
    combined.push_back({"[SEP_TEXT]", -1});
    for (std::string& w : split_words(text)) combined.push_back({std::move(w), -1});
    markers.assign(tasks.size(), {});
    for (const Entry& e : combined) {
      const int64_t start = (int64_t)ids.size();
      append_tokenized(e.text, ids);
      if (e.label_task >= 0) markers[(size_t)e.label_task].push_back(start);
    }
  }

  void clear_cache() { cache_.clear(); }

  static constexpr size_t kCacheSize = 1u << 16;

 private:
  static void lower_append(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
      out.push_back((char)(cp >= 'A' && cp <= 'Z' ? cp + 32 : cp));
      return;
    }
    UChar src[2];
    int32_t n = 0;
    U16_APPEND_UNSAFE(src, n, cp);
    UChar dst[16];
    UErrorCode st = U_ZERO_ERROR;
    const int32_t m = u_strToLower(dst, 16, src, n, "", &st);
    if (U_FAILURE(st)) {
      utf8_append(out, cp);
      return;
    }
    for (int32_t i = 0; i < m;) {
      UChar32 c;
      U16_NEXT(dst, i, m, c);
      utf8_append(out, (uint32_t)c);
    }
  }

  Tokenizer tok_;
  std::unordered_map<std::string, int32_t> special_;
  std::vector<std::string> cut_;
  int32_t pad_id_ = 0;
  std::unique_ptr<icu::RegexPattern> pattern_;
  std::unordered_map<std::string, std::vector<int32_t>> cache_;
};

namespace {

bool read_file(const std::string& path, std::string& out) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return false;
  std::ostringstream ss;
  ss << f.rdbuf();
  out = ss.str();
  return true;
}

std::vector<Task> parse_tasks(const char* json, size_t len) {
  Json root;
  try {
    root = parse_json(json, len);
  } catch (const std::exception& e) {
    throw FrontendError(GD_ERR_INVALID_ARGUMENT, std::string("tasks: ") + e.what());
  }
  if (!root.is_array()) throw FrontendError(GD_ERR_INVALID_ARGUMENT, "tasks must be a JSON array");
  std::vector<Task> tasks;
  for (const Json& t : root.arr) {
    if (!t.is_object()) throw FrontendError(GD_ERR_INVALID_ARGUMENT, "each task must be an object");
    Task task;
    const Json* name = t.get("name");
    const Json* labels = t.get("labels");
    if (!name || !name->is_string()) throw FrontendError(GD_ERR_INVALID_ARGUMENT, "task needs a string \"name\"");
    if (!labels || !labels->is_array()) throw FrontendError(GD_ERR_INVALID_ARGUMENT, "task needs \"labels\"");
    task.name = name->str;
    for (const Json& l : labels->arr) {
      if (!l.is_string()) throw FrontendError(GD_ERR_INVALID_ARGUMENT, "labels must be strings");
      task.labels.push_back(l.str);
    }
    if (const Json* p = t.get("prompt"); p && !p->is_null()) {
      if (!p->is_string()) throw FrontendError(GD_ERR_INVALID_ARGUMENT, "\"prompt\" must be a string");
      task.has_prompt = true;
      task.prompt = p->str;
    }
    if (const Json* d = t.get("labelDescriptions"); d && !d->is_null()) {
      if (!d->is_object()) throw FrontendError(GD_ERR_INVALID_ARGUMENT, "\"labelDescriptions\" must be an object");
      for (const auto& kv : d->obj) {
        if (!kv.second.is_string())
          throw FrontendError(GD_ERR_INVALID_ARGUMENT, "label descriptions must be strings");
        task.descriptions.emplace_back(kv.first, kv.second.str);
      }
    }
    if (const Json* m = t.get("multiLabel"); m && !m->is_null() && !m->is_bool())
      throw FrontendError(GD_ERR_INVALID_ARGUMENT, "\"multiLabel\" must be a boolean");
    tasks.push_back(std::move(task));
  }
  return tasks;
}

template <typename F>
int guarded(F&& f) {
  try {
    return f();
  } catch (const FrontendError& e) {
    return fail(e.code, e.what());
  } catch (const std::bad_alloc&) {
    return fail(GD_ERR_OUT_OF_MEMORY, "out of host memory");
  } catch (const std::exception& e) {
    return fail(GD_ERR_IO, e.what());
  }
}

int check_text(const char* s, size_t n, const char* what) {
  if (s == nullptr && n != 0) return fail(GD_ERR_INVALID_ARGUMENT, std::string(what) + " is null");
  if (n != 0 && !valid_utf8(s, n)) return fail(GD_ERR_INVALID_ARGUMENT, std::string(what) + " is not valid UTF-8");
  return GD_OK;
}

}  // namespace
}  // namespace gdf

using gdf::DecisionFrontend;

// Copies `v` to out[0, capacity); *count = v.size() (also when it does not fit).
template <typename T, typename U>
static int copy_out(const std::vector<T>& v, U* out, int64_t capacity, int64_t* count, const char* what) {
  if (count) *count = (int64_t)v.size();
  if ((int64_t)v.size() > capacity)
    return gdf::fail(GD_ERR_SHAPE, std::string(what) + ": capacity " + std::to_string(capacity) + " < " +
                                       std::to_string(v.size()));
  if (!v.empty() && out == nullptr) return gdf::fail(GD_ERR_INVALID_ARGUMENT, std::string(what) + " is null");
  for (size_t i = 0; i < v.size(); ++i) out[i] = (U)v[i];
  return GD_OK;
}

struct gd_frontend {
  std::unique_ptr<DecisionFrontend> impl;
  std::mutex mu;  // one call at a time per handle (the entry cache is shared)
};

extern "C" {

const char* gd_frontend_last_error(void) { return gdf::g_error.c_str(); }

int gd_frontend_open(gd_frontend** out, const char* directory) {
  return gdf::guarded([&]() -> int {
    if (out == nullptr || directory == nullptr) return gdf::fail(GD_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    const std::string dir(directory);
    std::string tj, cfg;
    if (!gdf::read_file(dir + "/tokenizer.json", tj) || !gdf::read_file(dir + "/tokenizer_config.json", cfg))
      return gdf::fail(GD_ERR_TOKENIZER_FILES,
                       "Tokenizer directory is missing tokenizer.json/tokenizer_config.json: " + dir);
    try {
      if (!gdf::parse_json(cfg.data(), cfg.size()).is_object()) throw std::runtime_error("not an object");
    } catch (const std::exception&) {
      return gdf::fail(GD_ERR_TOKENIZER_CONFIG, "Could not decode tokenizer_config.json");
    }
    gdf::Json root;
    try {
      root = gdf::parse_json(tj.data(), tj.size());
    } catch (const std::exception& e) {
      return gdf::fail(GD_ERR_IO, std::string("tokenizer.json: ") + e.what());
    }
    auto h = std::make_unique<gd_frontend>();
    h->impl = std::make_unique<DecisionFrontend>(root);
    *out = h.release();
    return GD_OK;
  });
}

int gd_frontend_create(gd_frontend** out, const char* tokenizer_json, size_t length) {
  return gdf::guarded([&]() -> int {
    if (out == nullptr || tokenizer_json == nullptr) return gdf::fail(GD_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    gdf::Json root;
    try {
      root = gdf::parse_json(tokenizer_json, length);
    } catch (const std::exception& e) {
      return gdf::fail(GD_ERR_IO, std::string("tokenizer.json: ") + e.what());
    }
    auto h = std::make_unique<gd_frontend>();
    h->impl = std::make_unique<DecisionFrontend>(root);
    *out = h.release();
    return GD_OK;
  });
}

void gd_frontend_destroy(gd_frontend* h) { delete h; }

int gd_frontend_clear_cache(gd_frontend* h) {
  if (h == nullptr) return gdf::fail(GD_ERR_INVALID_ARGUMENT, "null argument");
  std::lock_guard<std::mutex> lock(h->mu);
  h->impl->clear_cache();
  return GD_OK;
}

int gd_frontend_pad_id(gd_frontend* h, int32_t* out) {
  if (h == nullptr || out == nullptr) return gdf::fail(GD_ERR_INVALID_ARGUMENT, "null argument");
  *out = h->impl->pad_id();
  return GD_OK;
}

int gd_frontend_encode(gd_frontend* h, const char* text, size_t length, int32_t* ids,
                                       int64_t capacity, int64_t* count) {
  return gdf::guarded([&]() -> int {
    if (h == nullptr || count == nullptr) return gdf::fail(GD_ERR_INVALID_ARGUMENT, "null argument");
    if (int s = gdf::check_text(text, length, "text")) return s;
    std::vector<int32_t> out;
    h->impl->tokenizer().encode(std::string(text ? text : "", length), out);
    return copy_out(out, ids, capacity, count, "ids");
  });
}

int gd_frontend_append_tokenized(gd_frontend* h, const char* text, size_t length, int32_t* ids,
                                                 int64_t capacity, int64_t* count) {
  return gdf::guarded([&]() -> int {
    if (h == nullptr || count == nullptr) return gdf::fail(GD_ERR_INVALID_ARGUMENT, "null argument");
    if (int s = gdf::check_text(text, length, "text")) return s;
    std::vector<int32_t> out;
    std::lock_guard<std::mutex> lock(h->mu);
    h->impl->append_tokenized(std::string(text ? text : "", length), out);
    return copy_out(out, ids, capacity, count, "ids");
  });
}

int gd_frontend_split_words(gd_frontend* h, const char* text, size_t length, char* buffer,
                                            int64_t capacity, int64_t* bytes, int64_t* count) {
  return gdf::guarded([&]() -> int {
    if (h == nullptr || bytes == nullptr || count == nullptr)
      return gdf::fail(GD_ERR_INVALID_ARGUMENT, "null argument");
    if (int s = gdf::check_text(text, length, "text")) return s;
    const std::vector<std::string> words = h->impl->split_words(std::string(text ? text : "", length));
    std::vector<char> flat;
    for (const std::string& w : words) {
      flat.insert(flat.end(), w.begin(), w.end());
      flat.push_back('\0');
    }
    *count = (int64_t)words.size();
    return copy_out(flat, buffer, capacity, bytes, "buffer");
  });
}

int gd_frontend_make_input(gd_frontend* h, const char* text, size_t text_length,
                                           const char* tasks_json, size_t tasks_length, const int64_t* buckets,
                                           int64_t bucket_count, int32_t* input_ids, uint16_t* attention_mask,
                                           int64_t capacity, int32_t* marker_indices, float* marker_mask,
                                           int64_t marker_capacity, int64_t* bucket, int64_t* length,
                                           int64_t* heads, int64_t* options) {
  return gdf::guarded([&]() -> int {
    if (h == nullptr || bucket == nullptr || length == nullptr || heads == nullptr || options == nullptr ||
        tasks_json == nullptr || (buckets == nullptr && bucket_count != 0) || bucket_count < 0)
      return gdf::fail(GD_ERR_INVALID_ARGUMENT, "null argument");
    if (int s = gdf::check_text(text, text_length, "text")) return s;
    if (int s = gdf::check_text(tasks_json, tasks_length, "tasks")) return s;
    const std::vector<gdf::Task> tasks = gdf::parse_tasks(tasks_json, tasks_length);
    if (tasks.empty() || std::any_of(tasks.begin(), tasks.end(), [](const gdf::Task& t) { return t.labels.empty(); }))
      return gdf::fail(GD_ERR_NO_TASK_LABELS, "Every decision task must contain at least one label");
    std::vector<int64_t> given(buckets, buckets + bucket_count);
    std::vector<int64_t> ordered = given;
    std::sort(ordered.begin(), ordered.end());
    ordered.erase(std::unique(ordered.begin(), ordered.end()), ordered.end());
    if (ordered.empty())
      return gdf::fail(GD_ERR_INPUT_DOES_NOT_FIT,
                       "Encoded schema/text does not fit any requested bucket: " + gdf::bucket_list(given));
    std::vector<int32_t> ids;
    std::vector<std::vector<int64_t>> markers;
    {
      std::lock_guard<std::mutex> lock(h->mu);
      h->impl->encode_schema(std::string(text ? text : "", text_length), tasks, ids, markers);
    }
    const int64_t n = (int64_t)ids.size();
    int64_t O = 1;
    for (const gdf::Task& t : tasks) O = std::max<int64_t>(O, (int64_t)t.labels.size());
    const int64_t Hh = std::max<int64_t>((int64_t)tasks.size(), 1);
    *length = n;
    *heads = Hh;
    *options = O;
    *bucket = 0;
    auto it = std::find_if(ordered.begin(), ordered.end(), [&](int64_t b) { return b >= n; });
    if (it == ordered.end())
      return gdf::fail(GD_ERR_INPUT_DOES_NOT_FIT,
                       "Encoded schema/text does not fit any requested bucket: " + gdf::bucket_list(ordered));
    const int64_t L = *it;
    *bucket = L;
    if (capacity < L) return gdf::fail(GD_ERR_SHAPE, "input capacity " + std::to_string(capacity) + " < bucket " +
                                                         std::to_string(L));
    if (marker_capacity < Hh * O)
      return gdf::fail(GD_ERR_SHAPE, "marker capacity " + std::to_string(marker_capacity) + " < " +
                                         std::to_string(Hh * O));
    if (input_ids == nullptr || attention_mask == nullptr || marker_indices == nullptr || marker_mask == nullptr)
      return gdf::fail(GD_ERR_INVALID_ARGUMENT, "null output");
    const int32_t pad = h->impl->pad_id();
    for (int64_t i = 0; i < L; ++i) {
      input_ids[i] = i < n ? ids[(size_t)i] : pad;
      attention_mask[i] = i < n ? (uint16_t)0x3C00 : (uint16_t)0;  // fp16 1 / 0
    }
    for (int64_t i = 0; i < Hh * O; ++i) {
      marker_indices[i] = 0;
      marker_mask[i] = 0.f;
    }
    for (size_t hd = 0; hd < markers.size(); ++hd)
      for (size_t o = 0; o < markers[hd].size() && (int64_t)o < O; ++o) {
        marker_indices[(int64_t)hd * O + (int64_t)o] = (int32_t)markers[hd][o];
        marker_mask[(int64_t)hd * O + (int64_t)o] = 1.f;
      }
    return GD_OK;
  });
}

}  // extern "C"
