// GPT-2 artifact reader for libtinyinfer_llm: strict ASCII JSON manifest,
// SHA-256 of the weights binary and of every tensor, and the schema checks of
// reference llm/src/artifact.hpp:148-204 (alignment, extents, overlap, finite
// fp16, positive finite scales, no int8 -128).  The identity check accepts the
// reference's pinned official GPT-2 identity (artifact.hpp:156-158) or the
// synthetic random-init identity written by tinyinfer_amd/artifact.py.
#pragma once
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace tia::art {

struct Invalid : std::runtime_error {
  using std::runtime_error::runtime_error;
};
struct IOError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// ---------------------------------------------------------------- JSON
struct Value {
  enum Kind { Null, Bool, Number, String, Array, Object };
  Kind kind = Null;
  std::string text;  // string contents, or the number / literal spelling
  std::vector<Value> items;
  std::vector<std::pair<std::string, Value>> fields;

  const Value* find(const std::string& key) const {
    for (const auto& f : fields)
      if (f.first == key) return &f.second;
    return nullptr;
  }
  const Value& operator[](const std::string& key) const {
    const Value* v = kind == Object ? find(key) : nullptr;
    if (!v) throw Invalid("manifest field missing: " + key);
    return *v;
  }
  const std::string& str() const {
    if (kind != String) throw Invalid("manifest: expected a string");
    return text;
  }
  uint64_t u64() const {
    if (kind != Number || text.empty() || text.find_first_not_of("0123456789") != std::string::npos)
      throw Invalid("manifest: expected an unsigned integer");
    uint64_t v = 0;
    for (char c : text) {
      const uint64_t d = uint64_t(c - '0');
      if (v > (UINT64_MAX - d) / 10) throw Invalid("manifest: integer overflow");
      v = v * 10 + d;
    }
    return v;
  }
  double number() const {
    if (kind != Number) throw Invalid("manifest: expected a number");
    char* end = nullptr;
    const double v = std::strtod(text.c_str(), &end);
    if (end != text.c_str() + text.size() || !std::isfinite(v)) throw Invalid("manifest: bad number");
    return v;
  }
};

class JsonReader {
 public:
  explicit JsonReader(const std::string& s) : s_(s) {}
  Value parse() {
    Value v = value(0);
    skip();
    if (i_ != s_.size()) throw Invalid("JSON: trailing characters");
    return v;
  }

 private:
  const std::string& s_;
  size_t i_ = 0;

  void skip() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t')) ++i_;
  }
  char peek() {
    if (i_ >= s_.size()) throw Invalid("JSON: unexpected end");
    return s_[i_];
  }
  char next() {
    const char c = peek();
    ++i_;
    return c;
  }
  void expect(char c) {
    if (next() != c) throw Invalid(std::string("JSON: expected '") + c + "'");
  }
  std::string string_body() {
    expect('"');
    std::string out;
    for (;;) {
      const char c = next();
      if (c == '"') return out;
      const unsigned char u = static_cast<unsigned char>(c);
      if (u < 0x20 || u > 0x7e) throw Invalid("JSON: strings must be printable ASCII");
      if (c != '\\') {
        out.push_back(c);
        continue;
      }
      const char e = next();
      switch (e) {
        case '"': case '\\': case '/': out.push_back(e); break;
        case 'b': out.push_back('\b'); break;
        case 'f': out.push_back('\f'); break;
        case 'n': out.push_back('\n'); break;
        case 'r': out.push_back('\r'); break;
        case 't': out.push_back('\t'); break;
        default: throw Invalid("JSON: unsupported escape (no \\u escapes in manifests)");
      }
    }
  }
  static bool digit(char c) { return c >= '0' && c <= '9'; }
  std::string number_text() {
    const size_t start = i_;
    if (peek() == '-') ++i_;
    if (i_ >= s_.size() || !digit(s_[i_])) throw Invalid("JSON: bad number");
    if (s_[i_] == '0') ++i_;
    else
      while (i_ < s_.size() && digit(s_[i_])) ++i_;
    if (i_ < s_.size() && s_[i_] == '.') {
      ++i_;
      const size_t f = i_;
      while (i_ < s_.size() && digit(s_[i_])) ++i_;
      if (i_ == f) throw Invalid("JSON: bad fraction");
    }
    if (i_ < s_.size() && (s_[i_] == 'e' || s_[i_] == 'E')) {
      ++i_;
      if (i_ < s_.size() && (s_[i_] == '+' || s_[i_] == '-')) ++i_;
      const size_t e = i_;
      while (i_ < s_.size() && digit(s_[i_])) ++i_;
      if (i_ == e) throw Invalid("JSON: bad exponent");
    }
    return s_.substr(start, i_ - start);
  }
  Value value(int depth) {
    if (depth > 32) throw Invalid("JSON: nested too deeply");
    skip();
    Value v;
    const char c = peek();
    if (c == '{') {
      ++i_;
      v.kind = Value::Object;
      skip();
      if (peek() == '}') {
        ++i_;
        return v;
      }
      for (;;) {
        skip();
        std::string key = string_body();
        if (v.find(key)) throw Invalid("JSON: duplicate key " + key);
        skip();
        expect(':');
        v.fields.emplace_back(std::move(key), value(depth + 1));
        skip();
        const char d = next();
        if (d == '}') return v;
        if (d != ',') throw Invalid("JSON: expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++i_;
      v.kind = Value::Array;
      skip();
      if (peek() == ']') {
        ++i_;
        return v;
      }
      for (;;) {
        v.items.push_back(value(depth + 1));
        skip();
        const char d = next();
        if (d == ']') return v;
        if (d != ',') throw Invalid("JSON: expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = Value::String;
      v.text = string_body();
      return v;
    }
    for (const char* lit : {"true", "false", "null"}) {
      const size_t n = std::strlen(lit);
      if (s_.compare(i_, n, lit) == 0) {
        i_ += n;
        v.kind = lit[0] == 'n' ? Value::Null : Value::Bool;
        v.text = lit;
        return v;
      }
    }
    v.kind = Value::Number;
    v.text = number_text();
    return v;
  }
};

// ---------------------------------------------------------------- SHA-256 (FIPS 180-4)
class Sha256 {
 public:
  Sha256() { reset(); }
  void reset() {
    static const uint32_t iv[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                                   0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
    std::memcpy(h_, iv, sizeof h_);
    fill_ = 0;
    total_ = 0;
  }
  void update(const void* data, size_t n) {
    const uint8_t* p = static_cast<const uint8_t*>(data);
    total_ += n;
    if (fill_) {
      const size_t take = std::min(n, size_t(64) - fill_);
      std::memcpy(buf_ + fill_, p, take);
      fill_ += take;
      p += take;
      n -= take;
      if (fill_ == 64) {
        compress(buf_);
        fill_ = 0;
      }
    }
    for (; n >= 64; p += 64, n -= 64) compress(p);
    if (n) {
      std::memcpy(buf_, p, n);
      fill_ = n;
    }
  }
  std::string hex() {
    const uint64_t bits = total_ * 8;
    uint8_t pad[72] = {0x80};
    const size_t padlen = (fill_ < 56 ? 56 : 120) - fill_;
    update(pad, padlen);
    uint8_t len[8];
    for (int i = 0; i < 8; ++i) len[i] = uint8_t(bits >> (56 - 8 * i));
    update(len, 8);
    static const char* digits = "0123456789abcdef";
    std::string out;
    for (uint32_t w : h_)
      for (int s = 28; s >= 0; s -= 4) out.push_back(digits[(w >> s) & 15u]);
    return out;
  }
  static std::string of(const void* data, size_t n) {
    Sha256 s;
    s.update(data, n);
    return s.hex();
  }

 private:
  uint32_t h_[8];
  uint8_t buf_[64];
  size_t fill_;
  uint64_t total_;

  static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
  void compress(const uint8_t* blk) {
    static const uint32_t K[64] = {
        0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
        0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
        0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
        0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
        0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
        0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
        0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
        0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};
    uint32_t w[64];
    for (int t = 0; t < 16; ++t)
      w[t] = uint32_t(blk[4 * t]) << 24 | uint32_t(blk[4 * t + 1]) << 16 | uint32_t(blk[4 * t + 2]) << 8 |
             uint32_t(blk[4 * t + 3]);
    for (int t = 16; t < 64; ++t) {
      const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
      const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
      w[t] = w[t - 16] + s0 + w[t - 7] + s1;
    }
    uint32_t v[8];
    std::memcpy(v, h_, sizeof v);
    for (int t = 0; t < 64; ++t) {
      const uint32_t S1 = rotr(v[4], 6) ^ rotr(v[4], 11) ^ rotr(v[4], 25);
      const uint32_t ch = (v[4] & v[5]) ^ (~v[4] & v[6]);
      const uint32_t t1 = v[7] + S1 + ch + K[t] + w[t];
      const uint32_t S0 = rotr(v[0], 2) ^ rotr(v[0], 13) ^ rotr(v[0], 22);
      const uint32_t maj = (v[0] & v[1]) ^ (v[0] & v[2]) ^ (v[1] & v[2]);
      for (int i = 7; i > 0; --i) v[i] = v[i - 1];
      v[4] += t1;
      v[0] = t1 + S0 + maj;
    }
    for (int i = 0; i < 8; ++i) h_[i] += v[i];
  }
};

// ---------------------------------------------------------------- artifact
struct Tensor {
  std::string dtype;
  std::vector<int> shape;
  uint64_t offset = 0, nbytes = 0;
};

struct Arch {
  int layers = 0, heads = 0, hidden = 0, vocab = 0, capacity = 0;
};

struct Artifact {
  std::string precision;
  Arch arch;
  std::vector<uint8_t> binary;
  std::map<std::string, Tensor> tensors;

  const Tensor& require(const std::string& name, const std::vector<int>& shape, const std::string& dtype) const {
    auto it = tensors.find(name);
    if (it == tensors.end() || it->second.shape != shape || it->second.dtype != dtype)
      throw Invalid("tensor schema mismatch: " + name);
    return it->second;
  }
};

inline std::vector<uint8_t> read_file(const std::string& path, uint64_t limit) {
  std::unique_ptr<FILE, int (*)(FILE*)> f(std::fopen(path.c_str(), "rb"), &std::fclose);
  if (!f) throw IOError("cannot open " + path);
  if (std::fseek(f.get(), 0, SEEK_END) != 0) throw IOError("cannot seek " + path);
  const long size = std::ftell(f.get());
  if (size < 0 || uint64_t(size) > limit) throw Invalid("artifact file exceeds its size limit: " + path);
  std::rewind(f.get());
  std::vector<uint8_t> data(static_cast<size_t>(size));
  if (size && std::fread(data.data(), 1, data.size(), f.get()) != data.size()) throw IOError("short read " + path);
  return data;
}

inline Artifact load_artifact(const std::string& manifest_path) {
  const std::vector<uint8_t> raw = read_file(manifest_path, 1u << 20);
  const std::string text(raw.begin(), raw.end());
  const Value m = JsonReader(text).parse();
  if (m.kind != Value::Object) throw Invalid("manifest must be a JSON object");
  if (m["schema_version"].u64() != 1 || m["alignment"].u64() != 256 || m["binary"].str() != "weights.bin")
    throw Invalid("unsupported manifest schema");
  const std::string& id = m["model_id"].str();
  const bool official = id == "openai-community/gpt2" &&
                        m["revision"].str() == "607a30d783dfa663caf39e06633721c8d4cfcd7e" &&
                        m["source_sha256"].str() == "248dfc3911869ec493c76e65bf2fcf7f615828b0254c12b473182f0f81d3a707";
  const bool synthetic = id == "tinyinfer-amd/gpt2-synthetic" && m.find("synthetic") &&
                         m["synthetic"].kind == Value::Object && m["revision"].str().rfind("seed-", 0) == 0 &&
                         m["source_sha256"].str().size() == 64;
  if (!official && !synthetic) throw Invalid("unrecognized artifact identity");
  Artifact a;
  const Value& ar = m["architecture"];
  a.arch.layers = int(ar["layers"].u64());
  a.arch.heads = int(ar["heads"].u64());
  a.arch.hidden = int(ar["hidden"].u64());
  a.arch.vocab = int(ar["vocab"].u64());
  a.arch.capacity = int(ar["capacity"].u64());
  if (a.arch.layers < 1 || a.arch.layers > 256 || a.arch.heads < 1 || a.arch.hidden != a.arch.heads * 64 ||
      a.arch.vocab < 2 || a.arch.vocab > 1 << 20 || a.arch.capacity < 2 || a.arch.capacity > 1024 ||
      ar["gelu"].str() != "gelu_new" || ar["layer_norm_eps"].number() != 1e-5)
    throw Invalid("unsupported GPT-2 architecture");
  if (official && (a.arch.layers != 12 || a.arch.heads != 12 || a.arch.vocab != 50257 || a.arch.capacity != 1024))
    throw Invalid("official identity requires GPT-2 124M");
  a.precision = m["precision"].str();
  if (a.precision != "int8" && a.precision != "fp16") throw Invalid("unknown precision");

  std::string dir;
  const size_t slash = manifest_path.find_last_of('/');
  if (slash != std::string::npos) dir = manifest_path.substr(0, slash + 1);
  a.binary = read_file(dir + "weights.bin", uint64_t(8) << 30);
  if (a.binary.size() != m["binary_bytes"].u64() || Sha256::of(a.binary.data(), a.binary.size()) != m["binary_sha256"].str())
    throw Invalid("weights binary length or SHA-256 mismatch");
  const Value& list = m["tensors"];
  if (list.kind != Value::Array || list.items.size() > 4096) throw Invalid("invalid tensor list");
  std::vector<std::pair<uint64_t, uint64_t>> ranges;
  for (const Value& e : list.items) {
    Tensor t;
    t.dtype = e["dtype"].str();
    t.offset = e["offset"].u64();
    t.nbytes = e["nbytes"].u64();
    const Value& shape = e["shape"];
    if (shape.kind != Value::Array || shape.items.empty() || shape.items.size() > 2) throw Invalid("tensor rank");
    uint64_t count = 1;
    for (const Value& d : shape.items) {
      const uint64_t n = d.u64();
      if (n == 0 || n > (1u << 20)) throw Invalid("tensor dimension");
      count *= n;
      t.shape.push_back(int(n));
    }
    const uint64_t width = t.dtype == "float16" ? 2 : t.dtype == "float32" ? 4 : t.dtype == "int8" ? 1 : 0;
    if (!width || t.nbytes != count * width || t.offset % 256 || t.offset > a.binary.size() ||
        t.nbytes > a.binary.size() - t.offset)
      throw Invalid("tensor extent, dtype or alignment");
    const uint8_t* p = a.binary.data() + t.offset;
    if (Sha256::of(p, t.nbytes) != e["sha256"].str()) throw Invalid("tensor SHA-256 mismatch");
    if (t.dtype == "float16") {
      for (uint64_t i = 0; i < t.nbytes; i += 2)
        if (((uint16_t(p[i]) | uint16_t(p[i + 1]) << 8) & 0x7c00u) == 0x7c00u) throw Invalid("non-finite fp16 weight");
    } else if (t.dtype == "float32") {
      for (uint64_t i = 0; i < t.nbytes; i += 4) {
        float v;
        std::memcpy(&v, p + i, 4);
        if (!std::isfinite(v) || v <= 0.f) throw Invalid("non-positive or non-finite scale");
      }
    } else {
      for (uint64_t i = 0; i < t.nbytes; ++i)
        if (p[i] == 0x80) throw Invalid("int8 weight -128 is not allowed");
    }
    if (!a.tensors.emplace(e["name"].str(), t).second) throw Invalid("duplicate tensor name");
    ranges.emplace_back(t.offset, t.offset + t.nbytes);
  }
  std::sort(ranges.begin(), ranges.end());
  for (size_t i = 1; i < ranges.size(); ++i)
    if (ranges[i - 1].second > ranges[i].first) throw Invalid("overlapping tensors");
  return a;
}

}  // namespace tia::art
