#include "json.hpp"

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <stdexcept>

namespace gdf {

const Json* Json::get(const std::string& key) const {
  if (type != Object) return nullptr;
  const Json* found = nullptr;
  for (const auto& kv : obj)
    if (kv.first == key) found = &kv.second;
  return found;
}

namespace {

struct Parser {
  const char* p;
  const char* end;
  int depth = 0;

  [[noreturn]] void fail(const char* what) const { throw std::runtime_error(std::string("JSON: ") + what); }
  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool lit(const char* s) {
    const size_t n = std::strlen(s);
    if ((size_t)(end - p) >= n && std::memcmp(p, s, n) == 0) {
      p += n;
      return true;
    }
    return false;
  }
  static void put_utf8(std::string& out, uint32_t cp) {
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
  uint32_t hex4() {
    if (end - p < 4) fail("truncated \\u escape");
    uint32_t v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p++;
      v <<= 4;
      if (c >= '0' && c <= '9')
        v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f')
        v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F')
        v |= (uint32_t)(c - 'A' + 10);
      else
        fail("bad \\u escape");
    }
    return v;
  }
  std::string string() {
    if (p >= end || *p != '"') fail("expected a string");
    ++p;
    std::string out;
    for (;;) {
      const char* run = p;
      while (p < end && *p != '"' && *p != '\\') {
        if ((unsigned char)*p < 0x20) fail("control character in a string");
        ++p;
      }
      out.append(run, p);
      if (p >= end) fail("unterminated string");
      if (*p == '"') {
        ++p;
        return out;
      }
      ++p;  // backslash
      if (p >= end) fail("unterminated escape");
      const char c = *p++;
      switch (c) {
        case '"': out.push_back('"'); break;
        case '\\': out.push_back('\\'); break;
        case '/': out.push_back('/'); break;
        case 'b': out.push_back('\b'); break;
        case 'f': out.push_back('\f'); break;
        case 'n': out.push_back('\n'); break;
        case 'r': out.push_back('\r'); break;
        case 't': out.push_back('\t'); break;
        case 'u': {
          uint32_t cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00) {  // a high surrogate takes the low one that follows
            if (end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
              p += 2;
              const uint32_t lo = hex4();
              if (lo < 0xDC00 || lo > 0xDFFF) fail("unpaired surrogate");
              cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
            } else {
              fail("unpaired surrogate");
            }
          } else if (cp >= 0xDC00 && cp < 0xE000) {
            fail("unpaired surrogate");
          }
          put_utf8(out, cp);
          break;
        }
        default: fail("bad escape");
      }
    }
  }
  Json value() {
    if (++depth > 512) fail("nesting too deep");
    ws();
    if (p >= end) fail("unexpected end");
    Json v;
    const char c = *p;
    if (c == '{') {
      ++p;
      v.type = Json::Object;
      ws();
      if (p < end && *p == '}') {
        ++p;
      } else {
        for (;;) {
          ws();
          std::string key = string();
          ws();
          if (p >= end || *p != ':') fail("expected ':'");
          ++p;
          v.obj.emplace_back(std::move(key), value());
          ws();
          if (p < end && *p == ',') {
            ++p;
            continue;
          }
          if (p < end && *p == '}') {
            ++p;
            break;
          }
          fail("expected ',' or '}'");
        }
      }
    } else if (c == '[') {
      ++p;
      v.type = Json::Array;
      ws();
      if (p < end && *p == ']') {
        ++p;
      } else {
        for (;;) {
          v.arr.push_back(value());
          ws();
          if (p < end && *p == ',') {
            ++p;
            continue;
          }
          if (p < end && *p == ']') {
            ++p;
            break;
          }
          fail("expected ',' or ']'");
        }
      }
    } else if (c == '"') {
      v.type = Json::String;
      v.str = string();
    } else if (lit("true")) {
      v.type = Json::Bool;
      v.boolean = true;
    } else if (lit("false")) {
      v.type = Json::Bool;
    } else if (lit("null")) {
      v.type = Json::Null;
    } else if (c == '-' || (c >= '0' && c <= '9')) {
      const char* s = p;
      if (*p == '-') ++p;
      while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' || *p == '-'))
        ++p;
      const std::string tok(s, p);
      char* stop = nullptr;
      v.type = Json::Number;
      v.number = std::strtod(tok.c_str(), &stop);
      if (stop != tok.c_str() + tok.size()) fail("bad number");
    } else {
      fail("unexpected character");
    }
    --depth;
    return v;
  }
};

}  // namespace

Json parse_json(const char* text, size_t size) {
  Parser ps{text, text + size};
  Json v = ps.value();
  ps.ws();
  if (ps.p != ps.end) ps.fail("trailing characters");
  return v;
}

}  // namespace gdf
