// libtinyinfer_host_codec.so: host INT8 weight codec (include/tinyinfer_host_codec.h).
// Arithmetic and validation contract of reference backend/host_codec.cpp:58-103:
// every check (extents, alignment, byte-range overflow, pairwise overlap, finite
// inputs, positive scales, round-to-nearest mode, no -128, no half overflow)
// runs before the first output byte is written.
#include <cfenv>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>

#include "../../include/tinyinfer_host_codec.h"

namespace {
static_assert(std::numeric_limits<float>::is_iec559, "IEEE binary32 required");

struct Range {
  uintptr_t lo = 0, hi = 0;
};
bool range(const void* p, size_t count, size_t width, Range& r) {
  if (!p || reinterpret_cast<uintptr_t>(p) % width != 0 || count > SIZE_MAX / width) return false;
  const uintptr_t base = reinterpret_cast<uintptr_t>(p);
  if (count * width > UINTPTR_MAX - base) return false;
  r.lo = base;
  r.hi = base + count * width;
  return true;
}
bool disjoint(const Range& a, const Range& b) { return a.hi <= b.lo || b.hi <= a.lo; }
bool matrix_ok(size_t elements, size_t columns) {
  return elements > 0 && columns > 0 && elements % columns == 0 &&
         elements <= size_t(std::numeric_limits<int64_t>::max()) / sizeof(float);
}

// binary16 -> binary32 (exact) for finite inputs.
float half_to_float(uint16_t h) {
  const uint32_t sign = uint32_t(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
  if (e == 0) {
    const float v = float(m) * 0x1p-24f;  // subnormal or zero: m units of 2^-24
    return sign ? -v : v;
  }
  const uint32_t bits = sign | ((e + 112u) << 23) | (m << 13);
  float out;
  std::memcpy(&out, &bits, 4);
  return out;
}

// binary32 -> binary16, round to nearest even, for finite inputs whose magnitude
// is below the 65520 overflow boundary (the callers check both).
uint16_t float_to_half(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint16_t sign = uint16_t((x >> 16) & 0x8000u);
  const uint32_t a = x & 0x7fffffffu;
  if (a < 0x38800000u) {
    // Below 2^-14 the result is a multiple of 2^-24: scale (exactly) and round the
    // integer under FE_TONEAREST; 1024 encodes the smallest normal.
    float mag;
    std::memcpy(&mag, &a, 4);
    return uint16_t(sign | uint32_t(std::nearbyint(mag * 0x1p24f)));
  }
  // Drop 13 mantissa bits with a round-half-even bias; a carry walks into the exponent.
  const uint32_t r = (a + 0x0fffu + ((a >> 13) & 1u)) >> 13;
  return uint16_t(sign | (r - (112u << 10)));
}

float column_scale(const uint16_t* in, size_t elements, size_t columns, size_t c) {
  float mx = 0.f;
  for (size_t i = c; i < elements; i += columns) mx = std::fmax(mx, std::fabs(half_to_float(in[i])));
  return mx != 0.f ? float(double(mx) / 127.0) : 1.0f;
}
}  // namespace

extern "C" int ti_host_codec_abi_version(void) { return 1; }

extern "C" int ti_host_quantize_f16(const uint16_t* in, size_t elements, size_t columns, int8_t* q,
                                    size_t q_elements, float* scales, size_t scale_elements) {
  Range ri, rq, rs;
  if (!matrix_ok(elements, columns) || q_elements != elements || scale_elements != columns ||
      std::fegetround() != FE_TONEAREST || !range(in, elements, 2, ri) || !range(q, q_elements, 1, rq) ||
      !range(scales, scale_elements, 4, rs) || !disjoint(ri, rq) || !disjoint(ri, rs) || !disjoint(rq, rs))
    return TI_HOST_INVALID;
  for (size_t i = 0; i < elements; ++i)
    if ((in[i] & 0x7c00u) == 0x7c00u) return TI_HOST_INVALID;
  for (size_t c = 0; c < columns; ++c) {
    const float s = column_scale(in, elements, columns, c);
    if (!std::isfinite(s) || s <= 0.f) return TI_HOST_INVALID;
  }
  for (size_t c = 0; c < columns; ++c) scales[c] = column_scale(in, elements, columns, c);
  for (size_t i = 0; i < elements; ++i) {
    // binary64 quotient of exact operands, then round half to even (FE_TONEAREST).
    const double v = std::nearbyint(double(half_to_float(in[i])) / double(scales[i % columns]));
    q[i] = int8_t(v < -127.0 ? -127 : (v > 127.0 ? 127 : int(v)));
  }
  return TI_HOST_OK;
}

extern "C" int ti_host_dequantize_i8(const int8_t* q, size_t elements, size_t columns, const float* scales,
                                     size_t scale_elements, uint16_t* out, size_t output_elements) {
  Range rq, rs, ro;
  if (!matrix_ok(elements, columns) || scale_elements != columns || output_elements != elements ||
      std::fegetround() != FE_TONEAREST || !range(q, elements, 1, rq) || !range(scales, scale_elements, 4, rs) ||
      !range(out, output_elements, 2, ro) || !disjoint(rq, rs) || !disjoint(rq, ro) || !disjoint(rs, ro))
    return TI_HOST_INVALID;
  for (size_t c = 0; c < columns; ++c)
    if (!std::isfinite(scales[c]) || scales[c] <= 0.f) return TI_HOST_INVALID;
  for (size_t i = 0; i < elements; ++i) {
    if (q[i] == std::numeric_limits<int8_t>::min()) return TI_HOST_INVALID;
    const float v = float(q[i]) * scales[i % columns];
    if (!std::isfinite(v) || std::fabs(v) >= 65520.0f) return TI_HOST_INVALID;
  }
  for (size_t i = 0; i < elements; ++i) out[i] = float_to_half(float(q[i]) * scales[i % columns]);
  return TI_HOST_OK;
}
