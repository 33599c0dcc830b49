#include "tokenizer.hpp"

#include <unicode/brkiter.h>
#include <unicode/bytestream.h>
#include <unicode/normalizer2.h>
#include <unicode/uchar.h>
#include <unicode/ustring.h>
#include <unicode/utext.h>
#include <unicode/utf16.h>

#include <cstring>

#include "gliner_decide.h"

namespace gdf {

bool valid_utf8(const char* s, size_t n) {
  size_t i = 0;
  while (i < n) {
    const unsigned char c = (unsigned char)s[i];
    if (c < 0x80) {
      ++i;
      continue;
    }
    int len;
    uint32_t cp, min;
    if (c >= 0xC2 && c <= 0xDF) {
      len = 2, cp = c & 0x1F, min = 0x80;
    } else if (c >= 0xE0 && c <= 0xEF) {
      len = 3, cp = c & 0x0F, min = 0x800;
    } else if (c >= 0xF0 && c <= 0xF4) {
      len = 4, cp = c & 0x07, min = 0x10000;
    } else {
      return false;
    }
    if (i + len > n) return false;
    for (int k = 1; k < len; ++k) {
      const unsigned char d = (unsigned char)s[i + k];
      if ((d & 0xC0) != 0x80) return false;
      cp = (cp << 6) | (d & 0x3F);
    }
    if (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
    i += len;
  }
  return true;
}

uint32_t utf8_decode(const char* s, int len) {
  const unsigned char c = (unsigned char)s[0];
  if (len == 1) return c;
  uint32_t cp = c & (len == 2 ? 0x1F : (len == 3 ? 0x0F : 0x07));
  for (int k = 1; k < len; ++k) cp = (cp << 6) | ((unsigned char)s[k] & 0x3F);
  return cp;
}

void utf8_append(std::string& out, uint32_t cp) {
  if (cp < 0x80) {
    out.push_back((char)cp);
  } else if (cp < 0x800) {
    out.push_back((char)(0xC0 | (cp >> 6)));
    out.push_back((char)(0x80 | (cp & 0x3F)));
  } else if (cp < 0x10000) {
    out.push_back((char)(0xE0 | (cp >> 12)));
    out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
    out.push_back((char)(0x80 | (cp & 0x3F)));
  } else {
    out.push_back((char)(0xF0 | (cp >> 18)));
    out.push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
    out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
    out.push_back((char)(0x80 | (cp & 0x3F)));
  }
}

namespace {

[[noreturn]] void unsupported(const std::string& what) {
  throw FrontendError(GD_ERR_UNSUPPORTED, "tokenizer.json: unsupported " + what);
}
[[noreturn]] void malformed(const std::string& what) {
  throw FrontendError(GD_ERR_IO, "tokenizer.json: " + what);
}

std::string base64_decode(const std::string& in) {
  auto val = [](char c) -> int {
    if (c >= 'A' && c <= 'Z') return c - 'A';
    if (c >= 'a' && c <= 'z') return c - 'a' + 26;
    if (c >= '0' && c <= '9') return c - '0' + 52;
    if (c == '+') return 62;
    if (c == '/') return 63;
    return -1;
  };
  std::string out;
  out.reserve(in.size() / 4 * 3);
  uint32_t acc = 0;
  int bits = 0;
  for (char c : in) {
    if (c == '=') break;
    const int v = val(c);
    if (v < 0) malformed("bad base64 in precompiled_charsmap");
    acc = (acc << 6) | (uint32_t)v;
    bits += 6;
    if (bits >= 8) {
      bits -= 8;
      out.push_back((char)((acc >> bits) & 0xFF));
    }
  }
  return out;
}

// The lower-case mapping of one code point with no context (full mapping,
// e.g. U+0130 -> "i" U+0307, capital sigma -> small sigma).
void append_lower(std::string& out, uint32_t cp) {
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

// One extended-grapheme-cluster iterator per thread (ICU iterators are not
// shareable between threads).
icu::BreakIterator* grapheme_iterator() {
  thread_local std::unique_ptr<icu::BreakIterator> it;
  if (!it) {
    UErrorCode st = U_ZERO_ERROR;
    it.reset(icu::BreakIterator::createCharacterInstance(icu::Locale::getRoot(), st));
    if (U_FAILURE(st) || !it) throw FrontendError(GD_ERR_UNSUPPORTED, "ICU character break iterator unavailable");
  }
  return it.get();
}

}  // namespace

struct Tokenizer::Step {
  enum Kind { Strip, Precompiled, ReplaceLiteral, ReplaceRun, Lowercase, NFC, NFD, NFKC, NFKD } kind;
  bool left = false, right = false;
  std::string pattern, content;
  uint32_t run_cp = 0;
  int run_min = 0;
  std::vector<uint32_t> units;  // darts-clone double array
  std::string replacements;     // NUL-terminated replacement strings

  // First (shortest) key that prefixes chunk[0, n): its replacement.
  bool lookup(const char* chunk, size_t n, std::string& out) const {
    const size_t na = units.size();
    if (na == 0) return false;
    auto offset = [](uint32_t u) -> size_t { return (size_t)((u >> 10) << ((u & (1u << 9)) >> 6)); };
    size_t node = offset(units[0]);
    for (size_t i = 0; i < n; ++i) {
      const uint8_t c = (uint8_t)chunk[i];
      if (c == 0) return false;
      node ^= c;
      if (node >= na) return false;
      const uint32_t unit = units[node];
      if ((unit & ((1u << 31) | 0xFFu)) != c) return false;
      node ^= offset(unit);
      if (node >= na) return false;
      if ((unit >> 8) & 1u) {
        const size_t at = units[node] & 0x7FFFFFFFu;
        if (at >= replacements.size()) return false;
        const char* s = replacements.data() + at;
        out.append(s, strnlen(s, replacements.size() - at));
        return true;
      }
    }
    return false;
  }

  void apply(std::string& s) const {
    switch (kind) {
      case Strip: {
        size_t b = 0, e = s.size();
        if (left) {
          while (b < e) {
            const int l = utf8_len((unsigned char)s[b]);
            if (!u_isUWhiteSpace((UChar32)utf8_decode(s.data() + b, l))) break;
            b += l;
          }
        }
        if (right) {
          while (e > b) {
            size_t k = e - 1;
            while (k > b && ((unsigned char)s[k] & 0xC0) == 0x80) --k;
            if (!u_isUWhiteSpace((UChar32)utf8_decode(s.data() + k, (int)(e - k)))) break;
            e = k;
          }
        }
        s = s.substr(b, e - b);
        return;
      }
      case Precompiled: {
        if (s.empty()) return;
        std::string out;
        out.reserve(s.size());
        UErrorCode st = U_ZERO_ERROR;
        UText* ut = utext_openUTF8(nullptr, s.data(), (int64_t)s.size(), &st);
        if (U_FAILURE(st)) throw FrontendError(GD_ERR_UNSUPPORTED, "ICU UText unavailable");
        icu::BreakIterator* bi = grapheme_iterator();
        bi->setText(ut, st);
        int32_t start = bi->first();
        for (int32_t end = bi->next(); end != icu::BreakIterator::DONE; start = end, end = bi->next()) {
          const char* g = s.data() + start;
          const size_t gl = (size_t)(end - start);
          if (gl < 6 && lookup(g, gl, out)) continue;
          for (size_t k = 0; k < gl;) {
            const int l = utf8_len((unsigned char)g[k]);
            if (!lookup(g + k, (size_t)l, out)) out.append(g + k, (size_t)l);
            k += (size_t)l;
          }
        }
        utext_close(ut);
        s.swap(out);
        return;
      }
      case ReplaceLiteral: {
        if (pattern.empty()) return;
        std::string out;
        size_t at = 0;
        for (size_t f; (f = s.find(pattern, at)) != std::string::npos; at = f + pattern.size()) {
          out.append(s, at, f - at);
          out += content;
        }
        out.append(s, at, std::string::npos);
        s.swap(out);
        return;
      }
      case ReplaceRun: {
        std::string unit;
        utf8_append(unit, run_cp);
        std::string out;
        size_t i = 0;
        while (i < s.size()) {
          size_t j = i;
          int count = 0;
          while (s.compare(j, unit.size(), unit) == 0) {
            j += unit.size();
            ++count;
          }
          if (count > 0 && count >= run_min) {
            out += content;
            i = j;
          } else if (count > 0) {
            out.append(s, i, j - i);
            i = j;
          } else {
            const int l = utf8_len((unsigned char)s[i]);
            out.append(s, i, (size_t)l);
            i += (size_t)l;
          }
        }
        s.swap(out);
        return;
      }
      case Lowercase: {
        std::string out;
        out.reserve(s.size());
        for (size_t i = 0; i < s.size();) {
          const int l = utf8_len((unsigned char)s[i]);
          const uint32_t cp = utf8_decode(s.data() + i, l);
          if (cp < 0x80)
            out.push_back((char)(cp >= 'A' && cp <= 'Z' ? cp + 32 : cp));
          else
            append_lower(out, cp);
          i += (size_t)l;
        }
        s.swap(out);
        return;
      }
      case NFC:
      case NFD:
      case NFKC:
      case NFKD: {
        UErrorCode st = U_ZERO_ERROR;
        const icu::Normalizer2* n = kind == NFC    ? icu::Normalizer2::getNFCInstance(st)
                                    : kind == NFD  ? icu::Normalizer2::getNFDInstance(st)
                                    : kind == NFKC ? icu::Normalizer2::getNFKCInstance(st)
                                                   : icu::Normalizer2::getNFKDInstance(st);
        if (U_FAILURE(st)) throw FrontendError(GD_ERR_UNSUPPORTED, "ICU normalizer unavailable");
        std::string out;
        icu::StringByteSink<std::string> sink(&out);
        n->normalizeUTF8(0, icu::StringPiece(s.data(), (int32_t)s.size()), sink, nullptr, st);
        if (U_FAILURE(st)) throw FrontendError(GD_ERR_UNSUPPORTED, "ICU normalization failed");
        s.swap(out);
        return;
      }
    }
  }
};

namespace {

const std::string& str_member(const Json& j, const char* key, const char* what) {
  const Json* v = j.get(key);
  if (!v || !v->is_string()) malformed(std::string(what) + " needs a string \"" + key + "\"");
  return v->str;
}

bool regex_meta(uint32_t cp) { return cp < 0x80 && std::strchr("\\^$.|?*+()[]{}", (int)cp) != nullptr; }

void add_normalizer(const Json& j, std::vector<Tokenizer::Step>& steps) {
  if (j.is_null()) return;
  if (!j.is_object()) malformed("normalizer must be an object");
  const std::string& type = str_member(j, "type", "normalizer");
  using S = Tokenizer::Step;
  S s{};
  if (type == "Sequence") {
    const Json* list = j.get("normalizers");
    if (!list || !list->is_array()) malformed("Sequence normalizer needs \"normalizers\"");
    for (const Json& n : list->arr) add_normalizer(n, steps);
    return;
  } else if (type == "Strip") {
    s.kind = S::Strip;
    const Json* l = j.get("strip_left");
    const Json* r = j.get("strip_right");
    s.left = l && l->is_bool() ? l->boolean : true;
    s.right = r && r->is_bool() ? r->boolean : true;
  } else if (type == "Precompiled") {
    s.kind = S::Precompiled;
    const Json* cm = j.get("precompiled_charsmap");
    if (!cm || cm->is_null()) return;  // no charsmap: the identity
    if (!cm->is_string()) malformed("precompiled_charsmap must be a base64 string");
    const std::string blob = base64_decode(cm->str);
    if (blob.empty()) return;
    if (blob.size() < 4) malformed("precompiled_charsmap too short");
    uint32_t trie_bytes;
    std::memcpy(&trie_bytes, blob.data(), 4);
    if ((size_t)trie_bytes > blob.size() - 4 || trie_bytes % 4 != 0) malformed("precompiled_charsmap trie size");
    s.units.resize(trie_bytes / 4);
    std::memcpy(s.units.data(), blob.data() + 4, trie_bytes);
    s.replacements = blob.substr(4 + (size_t)trie_bytes);
  } else if (type == "Replace") {
    const Json* pat = j.get("pattern");
    s.content = str_member(j, "content", "Replace normalizer");
    if (!pat || !pat->is_object()) malformed("Replace normalizer needs a pattern");
    if (const Json* lit = pat->get("String"); lit && lit->is_string()) {
      s.kind = S::ReplaceLiteral;
      s.pattern = lit->str;
    } else if (const Json* re = pat->get("Regex"); re && re->is_string()) {
      // One character repeated: `c{n,}` or `c+` (the checkpoint's " {2,}").
      const std::string& r = re->str;
      if (r.empty() || !valid_utf8(r.data(), r.size())) unsupported("Replace regex \"" + r + "\"");
      const int l = utf8_len((unsigned char)r[0]);
      const uint32_t cp = utf8_decode(r.data(), l);
      const std::string rest = r.substr((size_t)l);
      int min = -1;
      if (rest == "+") {
        min = 1;
      } else if (rest.size() >= 4 && rest.front() == '{' && rest.compare(rest.size() - 2, 2, ",}") == 0) {
        const std::string num = rest.substr(1, rest.size() - 3);
        if (!num.empty() && num.find_first_not_of("0123456789") == std::string::npos && num.size() < 6)
          min = std::stoi(num);
      }
      if (min < 1 || regex_meta(cp)) unsupported("Replace regex \"" + r + "\"");
      s.kind = S::ReplaceRun;
      s.run_cp = cp;
      s.run_min = min;
    } else {
      malformed("Replace pattern must be a String or a Regex");
    }
  } else if (type == "Lowercase") {
    s.kind = S::Lowercase;
  } else if (type == "NFC") {
    s.kind = S::NFC;
  } else if (type == "NFD") {
    s.kind = S::NFD;
  } else if (type == "NFKC") {
    s.kind = S::NFKC;
  } else if (type == "NFKD") {
    s.kind = S::NFKD;
  } else {
    unsupported("normalizer \"" + type + "\"");
  }
  steps.push_back(std::move(s));
}

}  // namespace

Tokenizer::~Tokenizer() = default;

Tokenizer::Tokenizer(const Json& root) {
  if (!root.is_object()) malformed("the root must be an object");
  if (const Json* n = root.get("normalizer")) add_normalizer(*n, steps_);

  if (const Json* pt = root.get("pre_tokenizer"); pt && !pt->is_null()) {
    std::vector<const Json*> list;
    if (!pt->is_object()) malformed("pre_tokenizer must be an object");
    const std::string& type = str_member(*pt, "type", "pre_tokenizer");
    if (type == "Sequence") {
      const Json* l = pt->get("pretokenizers");
      if (!l || !l->is_array()) malformed("Sequence pre_tokenizer needs \"pretokenizers\"");
      for (const Json& x : l->arr) list.push_back(&x);
    } else {
      list.push_back(pt);
    }
    for (const Json* x : list) {
      if (!x->is_object()) malformed("pre_tokenizer must be an object");
      const std::string& t = str_member(*x, "type", "pre_tokenizer");
      PreStep ps;
      if (t == "WhitespaceSplit") {
        pre_.push_back(ps);
        continue;
      }
      if (t != "Metaspace") unsupported("pre_tokenizer \"" + t + "\"");
      ps.metaspace = true;
      ps.replacement = str_member(*x, "replacement", "Metaspace");
      if (ps.replacement.empty() || !valid_utf8(ps.replacement.data(), ps.replacement.size()) ||
          (size_t)utf8_len((unsigned char)ps.replacement[0]) != ps.replacement.size())
        malformed("Metaspace replacement must be one character");
      if (const Json* sch = x->get("prepend_scheme"); sch && sch->is_string()) {
        // "first" prepends only where the normalised text still starts at
        // original offset 0, which depends on how each normaliser aligns its
        // replacements; only "always" and "never" are restated.
        if (sch->str == "always")
          ps.prepend = 1;
        else if (sch->str == "never")
          ps.prepend = 0;
        else
          unsupported("Metaspace prepend_scheme \"" + sch->str + "\"");
      } else {
        const Json* aps = x->get("add_prefix_space");
        ps.prepend = (!aps || !aps->is_bool() || aps->boolean) ? 1 : 0;
      }
      const Json* sp = x->get("split");
      ps.split = !sp || !sp->is_bool() || sp->boolean;
      pre_.push_back(ps);
    }
  }

  const Json* model = root.get("model");
  if (!model || !model->is_object()) malformed("missing model");
  const std::string& mt = str_member(*model, "type", "model");
  if (mt == "WordLevel") {
    word_level_ = true;
    const Json* wv = model->get("vocab");
    if (!wv || !wv->is_object()) malformed("WordLevel needs a vocab object");
    for (const auto& kv : wv->obj) {
      if (!kv.second.is_number()) malformed("WordLevel ids must be numbers");
      words_[kv.first] = (int32_t)kv.second.number;
    }
    if (const Json* u = model->get("unk_token"); u && u->is_string()) unk_token_ = u->str;
    if (auto it = words_.find(unk_token_); it != words_.end()) unk_id_ = it->second;
  } else if (mt != "Unigram") {
    unsupported("model \"" + mt + "\"");
  }
  if (!word_level_) load_unigram(*model);

  if (const Json* at = root.get("added_tokens"); at && at->is_array()) {
    for (const Json& t : at->arr) {
      const Json* c = t.get("content");
      const Json* i = t.get("id");
      if (c && c->is_string() && i && i->is_number()) added_.emplace_back(c->str, (int32_t)i->number);
    }
  }
}

void Tokenizer::load_unigram(const Json& m) {
  const Json* model = &m;
  if (const Json* bf = model->get("byte_fallback"); bf && bf->is_bool() && bf->boolean)
    unsupported("Unigram byte_fallback");
  const Json* vocab = model->get("vocab");
  if (!vocab || !vocab->is_array() || vocab->arr.empty()) malformed("Unigram needs a non-empty vocab");
  pieces_.reserve(vocab->arr.size());
  scores_.reserve(vocab->arr.size());
  min_score_ = 0.0;
  bool first = true;
  node_piece_.push_back(-1);  // root
  edges_.reserve(vocab->arr.size() * 4);
  for (const Json& e : vocab->arr) {
    if (!e.is_array() || e.arr.size() != 2 || !e.arr[0].is_string() || !e.arr[1].is_number())
      malformed("Unigram vocab entries must be [piece, score]");
    const int32_t id = (int32_t)pieces_.size();
    pieces_.push_back(e.arr[0].str);
    scores_.push_back(e.arr[1].number);
    piece_id_[e.arr[0].str] = id;  // a repeated piece resolves to its last id
    if (first || e.arr[1].number < min_score_) min_score_ = e.arr[1].number;
    first = false;
    int32_t node = 0;
    for (unsigned char c : e.arr[0].str) {
      const uint64_t key = ((uint64_t)node << 8) | c;
      auto it = edges_.find(key);
      if (it == edges_.end()) {
        const int32_t child = (int32_t)node_piece_.size();
        node_piece_.push_back(-1);
        edges_.emplace(key, child);
        node = child;
      } else {
        node = it->second;
      }
    }
    if (node != 0) node_piece_[node] = -2;  // terminal; resolved below
  }
  for (const auto& kv : piece_id_) {
    int32_t node = 0;
    for (unsigned char c : kv.first) node = edges_.at(((uint64_t)node << 8) | c);
    if (node != 0) node_piece_[node] = kv.second;
  }
  if (const Json* u = model->get("unk_id"); u && u->is_number()) {
    unk_id_ = (int32_t)u->number;
    if (unk_id_ < 0 || unk_id_ >= (int32_t)pieces_.size()) malformed("Unigram unk_id out of range");
  }
}

int32_t Tokenizer::vocab_id(const std::string& token) const {
  const auto& m = word_level_ ? words_ : piece_id_;
  auto it = m.find(token);
  return it == m.end() ? -1 : it->second;
}

std::string Tokenizer::normalize(const std::string& text) const {
  std::string s = text;
  for (const Step& st : steps_) st.apply(s);
  return s;
}

std::vector<std::string> Tokenizer::pre_tokenize(const std::string& normalized) const {
  std::vector<std::string> pieces;
  if (normalized.empty()) return pieces;
  pieces.push_back(normalized);
  for (const PreStep& ps : pre_) {
    std::vector<std::string> next;
    for (const std::string& p : pieces) {
      if (!ps.metaspace) {  // WhitespaceSplit
        size_t start = 0, i = 0;
        while (i < p.size()) {
          const int l = utf8_len((unsigned char)p[i]);
          if (u_isUWhiteSpace((UChar32)utf8_decode(p.data() + i, l))) {
            if (i > start) next.push_back(p.substr(start, i - start));
            start = i + (size_t)l;
          }
          i += (size_t)l;
        }
        if (start < p.size()) next.push_back(p.substr(start));
        continue;
      }
      std::string s;
      s.reserve(p.size() + 8);
      for (char c : p) {
        if (c == ' ')
          s += ps.replacement;
        else
          s.push_back(c);
      }
      if (ps.prepend != 0 && s.compare(0, ps.replacement.size(), ps.replacement) != 0) s.insert(0, ps.replacement);
      if (!ps.split) {
        next.push_back(s);
        continue;
      }
      size_t start = 0;
      for (size_t f = 0; (f = s.find(ps.replacement, f)) != std::string::npos; f += ps.replacement.size()) {
        if (f > start) next.push_back(s.substr(start, f - start));
        start = f;
      }
      if (start < s.size()) next.push_back(s.substr(start));
    }
    pieces.swap(next);
  }
  return pieces;
}

std::vector<std::string> Tokenizer::unigram_pieces(const std::string& s) const {
  std::vector<std::string> result;
  if (s.empty()) return result;
  const size_t n = s.size();
  struct Best {
    int32_t id = -1;
    double score = 0.0;
    int64_t start = -1;
  };
  std::vector<Best> best(n + 1);
  const double unk_score = min_score_ - 10.0;
  size_t pos = 0;
  while (pos < n) {
    const double base = best[pos].score;
    const int mblen = utf8_len((unsigned char)s[pos]);
    bool single = false;
    int32_t node = 0;
    for (size_t j = pos; j < n; ++j) {
      auto it = edges_.find(((uint64_t)node << 8) | (unsigned char)s[j]);
      if (it == edges_.end()) break;
      node = it->second;
      const int32_t pid = node_piece_[node];
      if (pid < 0) continue;
      Best& t = best[j + 1];
      const double cand = scores_[pid] + base;
      if (t.start < 0 || cand > t.score) {
        t.score = cand;
        t.start = (int64_t)pos;
        t.id = pid;
      }
      if ((int)(j + 1 - pos) == mblen) single = true;
    }
    if (!single) {
      if (unk_id_ < 0) throw FrontendError(GD_ERR_UNSUPPORTED, "Unigram: a character outside the vocabulary and no unk_id");
      Best& t = best[pos + mblen];
      const double cand = unk_score + base;
      if (t.start < 0 || cand > t.score) {
        t.score = cand;
        t.start = (int64_t)pos;
        t.id = unk_id_;
      }
    }
    pos += (size_t)mblen;
  }
  // Back to front; adjacent unknown pieces fuse into one.
  std::vector<std::string> rev;
  std::string fused;
  bool in_unk = false;
  for (size_t end = n; end > 0;) {
    const Best& b = best[end];
    const size_t start = (size_t)b.start;
    if (unk_id_ >= 0 && b.id == unk_id_) {
      fused.insert(0, s, start, end - start);
      in_unk = true;
    } else {
      if (in_unk) {
        rev.push_back(fused);
        fused.clear();
        in_unk = false;
      }
      rev.push_back(s.substr(start, end - start));
    }
    end = start;
  }
  if (in_unk) rev.push_back(fused);
  result.assign(rev.rbegin(), rev.rend());
  return result;
}

void Tokenizer::encode(const std::string& text, std::vector<int32_t>& ids) const {
  const std::string norm = normalize(text);
  for (const std::string& piece : pre_tokenize(norm)) {
    if (word_level_) {
      auto it = words_.find(piece);
      if (it != words_.end()) {
        ids.push_back(it->second);
      } else {
        if (unk_id_ < 0) throw FrontendError(GD_ERR_UNSUPPORTED, "WordLevel: a piece outside the vocabulary and no unk_token");
        ids.push_back(unk_id_);
      }
      continue;
    }
    for (const std::string& tok : unigram_pieces(piece)) {
      auto it = piece_id_.find(tok);
      if (it != piece_id_.end()) {
        ids.push_back(it->second);
      } else {
        if (unk_id_ < 0) throw FrontendError(GD_ERR_UNSUPPORTED, "Unigram: a piece outside the vocabulary and no unk_id");
        ids.push_back(unk_id_);
      }
    }
  }
}

}  // namespace gdf
