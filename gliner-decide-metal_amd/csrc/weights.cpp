// Weight store: key -> host tensor, filled from caller buffers or from a
// safetensors file.
//
// Reference: WeightStore (Weights.swift:23-58) over MLX `loadArrays`, and the
// fp16 safetensors written by Tools/prepare_model.py:82-113.  The safetensors
// layout is: u64 little-endian header length N, N bytes of JSON
// {"<key>": {"dtype": "F16", "shape": [...], "data_offsets": [begin, end]},
// "__metadata__": {...}}, then the raw tensor bytes (offsets relative to the
// end of the header).
#include "weights.hpp"

#include <cstring>
#include <fstream>
#include <sstream>

#include "gd_common.hpp"

namespace gd {

int64_t dtype_size(int dtype) {
  switch (dtype) {
    case GD_F16:
    case GD_BF16:
      return 2;
    case GD_F32:
    case GD_I32:
      return 4;
    case GD_I64:
      return 8;
    default:
      return -1;
  }
}

const char* dtype_name(int dtype) {
  switch (dtype) {
    case GD_F16:
      return "F16";
    case GD_BF16:
      return "BF16";
    case GD_F32:
      return "F32";
    case GD_I32:
      return "I32";
    case GD_I64:
      return "I64";
    default:
      return "?";
  }
}

int64_t HostTensor::numel() const {
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  return n;
}

// Bytes of a tensor of `shape` and element size `es`, or -1 when a
// dimension is negative or the product overflows int64.
static int64_t checked_bytes(const std::vector<int64_t>& shape, int64_t es) {
  int64_t n = es;
  for (int64_t d : shape) {
    if (d < 0 || __builtin_mul_overflow(n, d, &n)) return -1;
  }
  return n;
}

std::string HostTensor::shape_string() const {
  std::ostringstream os;
  os << "[";
  for (size_t i = 0; i < shape.size(); ++i) os << (i ? ", " : "") << shape[i];
  os << "]";
  return os.str();
}

namespace {

// Minimal JSON reader for safetensors headers: objects, arrays, strings,
// integers and the literals; values that are not needed are skipped.
class JsonCursor {
 public:
  explicit JsonCursor(const std::string& s) : s_(s) {}
  bool ok() const { return ok_; }
  void ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t')) ++i_;
  }
  bool eat(char c) {
    ws();
    if (i_ < s_.size() && s_[i_] == c) {
      ++i_;
      return true;
    }
    return false;
  }
  bool peek(char c) {
    ws();
    return i_ < s_.size() && s_[i_] == c;
  }
  bool string(std::string& out) {
    ws();
    if (i_ >= s_.size() || s_[i_] != '"') return bad();
    ++i_;
    out.clear();
    while (i_ < s_.size() && s_[i_] != '"') {
      char c = s_[i_++];
      if (c == '\\') {
        if (i_ >= s_.size()) return bad();
        char e = s_[i_++];
        switch (e) {
          case 'n':
            out += '\n';
            break;
          case 't':
            out += '\t';
            break;
          case 'u':  // keep \uXXXX escapes verbatim (metadata only)
            out += "\\u";
            break;
          default:
            out += e;
        }
      } else {
        out += c;
      }
    }
    if (i_ >= s_.size()) return bad();
    ++i_;
    return true;
  }
  // A decimal integer in int64 range (anything else marks the header bad).
  bool integer(int64_t& v) {
    ws();
    size_t j = i_;
    const bool neg = j < s_.size() && s_[j] == '-';
    if (neg) ++j;
    if (j >= s_.size() || s_[j] < '0' || s_[j] > '9') return bad();
    int64_t acc = 0;
    while (j < s_.size() && s_[j] >= '0' && s_[j] <= '9') {
      const int digit = s_[j] - '0';
      if (__builtin_mul_overflow(acc, (int64_t)10, &acc) || __builtin_add_overflow(acc, (int64_t)digit, &acc))
        return bad();
      ++j;
    }
    v = neg ? -acc : acc;
    i_ = j;
    return true;
  }
  bool skip_value() {
    ws();
    if (i_ >= s_.size()) return bad();
    const char c = s_[i_];
    if (c == '"') {
      std::string tmp;
      return string(tmp);
    }
    if (c == '{' || c == '[') {
      const char close = c == '{' ? '}' : ']';
      ++i_;
      if (eat(close)) return true;
      do {
        if (c == '{') {
          std::string k;
          if (!string(k) || !eat(':')) return bad();
        }
        if (!skip_value()) return false;
      } while (eat(','));
      return eat(close) ? true : bad();
    }
    // number / literal
    while (i_ < s_.size() && s_[i_] != ',' && s_[i_] != '}' && s_[i_] != ']') ++i_;
    return true;
  }
  bool at_end() {
    ws();
    return i_ == s_.size();
  }

 private:
  bool bad() {
    ok_ = false;
    return false;
  }
  const std::string& s_;
  size_t i_ = 0;
  bool ok_ = true;
};

int parse_dtype(const std::string& s) {
  if (s == "F16") return GD_F16;
  if (s == "F32") return GD_F32;
  if (s == "BF16") return GD_BF16;
  if (s == "I32") return GD_I32;
  if (s == "I64") return GD_I64;
  return -1;
}

}  // namespace

int WeightStore::add(const std::string& key, const void* data, int dtype, const int64_t* shape, int ndim) {
  const int64_t es = dtype_size(dtype);
  if (es < 0) {
    set_error("unknown dtype %d for %s", dtype, key.c_str());
    return GD_ERR_INVALID_ARGUMENT;
  }
  if (ndim < 0 || ndim > 8 || (ndim > 0 && !shape)) {
    set_error("bad rank %d for %s", ndim, key.c_str());
    return GD_ERR_INVALID_ARGUMENT;
  }
  HostTensor t;
  t.dtype = dtype;
  t.shape.assign(shape, shape + ndim);
  const int64_t bytes = checked_bytes(t.shape, es);
  if (bytes < 0) {
    set_error("negative or overflowing dimensions for %s", key.c_str());
    return GD_ERR_INVALID_ARGUMENT;
  }
  if (bytes > 0 && !data) {
    set_error("null data for %s", key.c_str());
    return GD_ERR_INVALID_ARGUMENT;
  }
  t.data.resize((size_t)bytes);
  if (bytes) std::memcpy(t.data.data(), data, (size_t)bytes);
  tensors[key] = std::move(t);
  return GD_OK;
}

int WeightStore::load_safetensors(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) {
    set_error("cannot open %s", path.c_str());
    return GD_ERR_IO;
  }
  uint64_t hlen = 0;
  f.read(reinterpret_cast<char*>(&hlen), 8);
  if (!f || hlen == 0 || hlen > (uint64_t)100 << 20) {
    set_error("%s: bad safetensors header length", path.c_str());
    return GD_ERR_IO;
  }
  std::string header((size_t)hlen, '\0');
  f.read(&header[0], (std::streamsize)hlen);
  if (!f) {
    set_error("%s: truncated header", path.c_str());
    return GD_ERR_IO;
  }
  f.seekg(0, std::ios::end);
  const int64_t file_size = (int64_t)f.tellg();
  const int64_t data_start = 8 + (int64_t)hlen;

  struct Entry {
    std::string key;
    int dtype;
    std::vector<int64_t> shape;
    int64_t begin, end;
  };
  std::vector<Entry> entries;
  JsonCursor j(header);
  if (!j.eat('{')) {
    set_error("%s: header is not a JSON object", path.c_str());
    return GD_ERR_IO;
  }
  if (!j.peek('}')) {
    do {
      std::string key;
      if (!j.string(key) || !j.eat(':')) break;
      if (key == "__metadata__") {
        if (!j.skip_value()) break;
        continue;
      }
      Entry e{key, -1, {}, -1, -1};
      if (!j.eat('{')) break;
      do {
        std::string field;
        if (!j.string(field) || !j.eat(':')) break;
        if (field == "dtype") {
          std::string dt;
          if (!j.string(dt)) break;
          e.dtype = parse_dtype(dt);
          if (e.dtype < 0) {
            set_error("%s: unsupported dtype %s for %s", path.c_str(), dt.c_str(), key.c_str());
            return GD_ERR_WEIGHT_DTYPE;
          }
        } else if (field == "shape") {
          if (!j.eat('[')) break;
          if (!j.eat(']')) {
            do {
              int64_t v;
              if (!j.integer(v)) break;
              e.shape.push_back(v);
            } while (j.eat(','));
            if (!j.eat(']')) break;
          }
        } else if (field == "data_offsets") {
          if (!j.eat('[') || !j.integer(e.begin) || !j.eat(',') || !j.integer(e.end) || !j.eat(']')) break;
        } else if (!j.skip_value()) {
          break;
        }
      } while (j.eat(','));
      if (!j.eat('}')) break;
      entries.push_back(std::move(e));
    } while (j.eat(','));
  }
  if (!j.ok() || !j.eat('}')) {
    set_error("%s: malformed safetensors header", path.c_str());
    return GD_ERR_IO;
  }
  for (const Entry& e : entries) {
    HostTensor t;
    t.dtype = e.dtype;
    t.shape = e.shape;
    // Every check runs before the resize: a negative dimension, an end
    // before the begin, a size that overflows or a range past the file's end
    // are header errors.
    const int64_t bytes = e.dtype < 0 || e.shape.size() > 8 ? -1 : checked_bytes(e.shape, dtype_size(e.dtype));
    if (bytes < 0 || e.begin < 0 || e.end < e.begin || e.end - e.begin != bytes ||
        e.end > file_size - data_start) {
      set_error("%s: bad data offsets for %s", path.c_str(), e.key.c_str());
      return GD_ERR_IO;
    }
    t.data.resize((size_t)bytes);
    f.seekg(data_start + e.begin);
    f.read(reinterpret_cast<char*>(t.data.data()), (std::streamsize)bytes);
    if (!f) {
      set_error("%s: short read for %s", path.c_str(), e.key.c_str());
      return GD_ERR_IO;
    }
    tensors[e.key] = std::move(t);
  }
  return GD_OK;
}

const HostTensor* WeightStore::find(const std::string& key) const {
  auto it = tensors.find(key);
  return it == tensors.end() ? nullptr : &it->second;
}

// WeightStore.array(_:shape:dtype:) (Weights.swift:83-106).
int WeightStore::require(const std::string& key, const std::vector<int64_t>& shape, int dtype,
                         const HostTensor** out) const {
  const HostTensor* t = find(key);
  if (!t) {
    set_error("Missing model weight: %s", key.c_str());
    return GD_ERR_MISSING_WEIGHT;
  }
  if (t->shape != shape) {
    HostTensor want;
    want.shape = shape;
    set_error("Weight %s has shape %s, expected %s", key.c_str(), t->shape_string().c_str(),
              want.shape_string().c_str());
    return GD_ERR_WEIGHT_SHAPE;
  }
  if (t->dtype != dtype) {
    set_error("Weight %s has dtype %s, expected %s", key.c_str(), dtype_name(t->dtype), dtype_name(dtype));
    return GD_ERR_WEIGHT_DTYPE;
  }
  *out = t;
  return GD_OK;
}

}  // namespace gd
