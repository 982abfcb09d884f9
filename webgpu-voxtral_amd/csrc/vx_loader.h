// vx_loader.h -- local safetensors loading: header parsing and the
// reference's dtype conversions (src/weights.ts), on the host and as
// device kernels.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>
#include <map>
#include <string>
#include <vector>

namespace vx {

// ----------------------------------------------------------- conversions
// convertBF16toF16, src/weights.ts:94-138: sign kept; exponent rebiased;
// the 7 mantissa bits extended by 3 zero bits; exponent 0xFF -> inf, or NaN
// 0x7E00 | sign when the mantissa is non-zero; BF16 zero/subnormal -> signed
// zero; overflow -> inf; underflow -> the shift-based subnormal below (not
// correctly rounded) or signed zero.
__host__ __device__ inline uint16_t bf16_to_f16_ref(uint16_t bf16) {
  const uint32_t sign = (bf16 >> 15) & 1u, exp = (bf16 >> 7) & 0xFFu, mant = bf16 & 0x7Fu;
  if (exp == 0xFF) return (uint16_t)((sign << 15) | 0x7C00u | (mant ? 0x0200u : 0u));
  if (exp == 0) return (uint16_t)(sign << 15);
  const int unbiased = (int)exp - 127;
  if (unbiased > 15) return (uint16_t)((sign << 15) | 0x7C00u);
  if (unbiased < -14) {
    const int shift = -14 - unbiased;
    if (shift > 10) return (uint16_t)(sign << 15);
    const uint32_t f16m = ((0x80u | (mant << 1)) >> shift) >> 1;
    return (uint16_t)((sign << 15) | (f16m & 0x03FFu));
  }
  return (uint16_t)((sign << 15) | ((uint32_t)(unbiased + 15) << 10) | ((mant << 3) & 0x03FFu));
}

// float32ToFloat16, src/weights.ts:222-232: exponent rebiased, mantissa
// truncated to 10 bits, results below the normal range -> signed zero,
// above it (inf and NaN included) -> inf.
__host__ __device__ inline uint16_t f32_to_f16_ref(uint32_t bits) {
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const int exp = (int)((bits >> 23) & 0xFFu) - 127 + 15;
  const uint32_t frac = (bits >> 13) & 0x3FFu;
  if (exp <= 0) return (uint16_t)sign;
  if (exp >= 31) return (uint16_t)(sign | 0x7C00u);
  return (uint16_t)(sign | ((uint32_t)exp << 10) | frac);
}

__global__ void bf16_to_f16_kernel(const uint16_t *in, uint16_t *out, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    out[i] = bf16_to_f16_ref(in[i]);
}

__global__ void f32_to_f16_ref_kernel(const uint32_t *in, uint16_t *out, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    out[i] = f32_to_f16_ref(in[i]);
}

// ------------------------------------------------------- header parsing
// One tensor entry of a safetensors header: {"dtype", "shape", "data_offsets"}.
struct StEntry {
  std::string dtype;
  std::vector<int64_t> shape;
  uint64_t begin = 0, end = 0;
};

// Minimal JSON reader for the safetensors header: an object of tensor
// entries plus an optional "__metadata__" object of strings.  Returns false
// (with a message) on anything malformed.
class StHeaderParser {
 public:
  StHeaderParser(const char *p, size_t n) : p_(p), end_(p + n) {}

  bool parse(std::map<std::string, StEntry> &out, std::string &err) {
    ws();
    if (!eat('{')) return fail(err, "header is not a JSON object");
    ws();
    if (eat('}')) return true;
    for (;;) {
      std::string name;
      ws();
      if (!str(name)) return fail(err, "expected a tensor name");
      ws();
      if (!eat(':')) return fail(err, "expected ':'");
      ws();
      if (name == "__metadata__") {
        if (!skip_value()) return fail(err, "bad __metadata__");
      } else {
        StEntry e;
        if (!entry(e)) return fail(err, "bad entry for " + name);
        out[name] = e;
      }
      ws();
      if (eat(',')) continue;
      if (eat('}')) return true;
      return fail(err, "expected ',' or '}'");
    }
  }

 private:
  const char *p_, *end_;
  static bool fail(std::string &err, const std::string &m) {
    err = m;
    return false;
  }
  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) p_++;
  }
  bool eat(char c) {
    if (p_ < end_ && *p_ == c) {
      p_++;
      return true;
    }
    return false;
  }
  bool str(std::string &s) {
    if (!eat('"')) return false;
    while (p_ < end_ && *p_ != '"') {
      if (*p_ == '\\') {
        if (++p_ >= end_) return false;
        const char c = *p_++;
        if (c == 'u') {  // kept as the escape text: names here are ASCII
          if (end_ - p_ < 4) return false;
          s += "\\u";
          s.append(p_, 4);
          p_ += 4;
        } else {
          s += c == 'n' ? '\n' : c == 't' ? '\t' : c == 'r' ? '\r' : c == 'b' ? '\b' : c == 'f' ? '\f' : c;
        }
      } else {
        s += *p_++;
      }
    }
    return eat('"');
  }
  bool integer(int64_t &v) {
    const char *q = p_;
    bool neg = eat('-');
    if (p_ >= end_ || *p_ < '0' || *p_ > '9') {
      p_ = q;
      return false;
    }
    uint64_t x = 0;
    while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
      const uint64_t d = (uint64_t)(*p_++ - '0');
      if (x > ((uint64_t)INT64_MAX - d) / 10) return false;  // outside int64
      x = x * 10 + d;
    }
    v = neg ? -(int64_t)x : (int64_t)x;
    return true;
  }
  bool int_array(std::vector<int64_t> &a) {
    if (!eat('[')) return false;
    ws();
    if (eat(']')) return true;
    for (;;) {
      int64_t v;
      ws();
      if (!integer(v)) return false;
      a.push_back(v);
      ws();
      if (eat(',')) continue;
      return eat(']');
    }
  }
  bool entry(StEntry &e) {
    if (!eat('{')) return false;
    bool have_offsets = false;
    ws();
    if (eat('}')) return false;
    for (;;) {
      std::string key;
      ws();
      if (!str(key)) return false;
      ws();
      if (!eat(':')) return false;
      ws();
      if (key == "dtype") {
        if (!str(e.dtype)) return false;
      } else if (key == "shape") {
        if (!int_array(e.shape)) return false;
      } else if (key == "data_offsets") {
        std::vector<int64_t> o;
        if (!int_array(o) || o.size() != 2 || o[0] < 0 || o[1] < o[0]) return false;
        e.begin = (uint64_t)o[0];
        e.end = (uint64_t)o[1];
        have_offsets = true;
      } else if (!skip_value()) {
        return false;
      }
      ws();
      if (eat(',')) continue;
      if (eat('}')) return have_offsets && !e.dtype.empty();
      return false;
    }
  }
  // nesting deeper than kMaxDepth is rejected (a header of nested brackets
  // must not exhaust the stack)
  static constexpr int kMaxDepth = 64;
  bool skip_value(int depth = 0) {
    ws();
    if (p_ >= end_ || depth > kMaxDepth) return false;
    if (*p_ == '"') {
      std::string s;
      return str(s);
    }
    if (*p_ == '{' || *p_ == '[') {
      const char open = *p_, close = open == '{' ? '}' : ']';
      p_++;
      ws();
      if (eat(close)) return true;
      for (;;) {
        ws();
        if (open == '{') {
          std::string k;
          if (!str(k)) return false;
          ws();
          if (!eat(':')) return false;
        }
        if (!skip_value(depth + 1)) return false;
        ws();
        if (eat(',')) continue;
        return eat(close);
      }
    }
    // number or literal
    const char *q = p_;
    while (p_ < end_ && *p_ != ',' && *p_ != '}' && *p_ != ']' && *p_ != ' ' && *p_ != '\n') p_++;
    return p_ > q;
  }
};

// classifyComponent, src/weights.ts:478-483
inline const char *st_component(const std::string &name) {
  auto starts = [&](const char *p) { return name.rfind(p, 0) == 0; };
  if (starts("acoustic_transformer.")) return "fm";
  if (starts("audio_tokenizer.")) return "codec";
  if (starts("layers.") || starts("norm.") || starts("mm_audio_embeddings.")) return "backbone";
  return "other";
}

}  // namespace vx
