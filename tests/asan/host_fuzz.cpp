// Host-only robustness driver for the host INT8 codec (ti_host_quantize_f16 /
// ti_host_dequantize_i8, tinyinfer_amd/csrc/host_codec.cpp) and the legacy
// FP32 CPU entry points (ti_cpu_gemm / ti_cpu_softmax / ti_cpu_layernorm,
// tinyinfer_amd/csrc/cpu_ops.cpp), built with AddressSanitizer and UBSan by
// tests/test_host_asan.py.  Every buffer is a heap vector of exactly the size
// passed, so a read or write past it is a sanitizer report.
//
//   host_fuzz SEED ITERATIONS
//
// Per iteration, with seeded random shapes and bit patterns:
//  * quantize random fp16 bits (any pattern: NaN, inf, subnormal, normal):
//    the status is OK or INVALID; an OK result dequantizes OK and holds no -128;
//  * dequantize random int8 bytes with random fp32 scale bits: OK or INVALID;
//  * a q or output buffer one element short is refused (INVALID) before any
//    write;
//  * GEMM, softmax and LayerNorm over random finite inputs of ragged shapes.
// Aborts on any contract break; prints "ok <quantized> <rejected> <dequantized>".
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "tinyinfer_backend.h"
#include "tinyinfer_host_codec.h"

namespace {

[[noreturn]] void fail(const char* what, int iter) {
  std::fprintf(stderr, "contract broken at iteration %d: %s\n", iter, what);
  std::abort();
}

uint16_t random_half(std::mt19937& rng) {
  switch (rng() % 4) {
    case 0: return uint16_t(rng());                              // any pattern
    case 1: return uint16_t(rng() % 0x0400u | (rng() & 0x8000u));  // subnormal or zero
    default: {                                                     // normal, moderate exponent
      const uint32_t exp = 5 + rng() % 20;
      return uint16_t((rng() & 0x8000u) | (exp << 10) | (rng() & 0x3ffu));
    }
  }
}

float random_finite(std::mt19937& rng) {
  return std::uniform_real_distribution<float>(-4.f, 4.f)(rng);
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 3) return 2;
  std::mt19937 rng(uint32_t(std::strtoul(argv[1], nullptr, 10)));
  const int iterations = std::atoi(argv[2]);
  int quantized = 0, rejected = 0, dequantized = 0;
  for (int it = 0; it < iterations; ++it) {
    // ---- codec
    const size_t rows = 1 + rng() % 32, cols = 1 + rng() % 32, count = rows * cols;
    std::vector<uint16_t> half(count), out(count);
    std::vector<int8_t> q(count);
    std::vector<float> scales(cols);
    const bool all_normal = rng() % 2 == 0;
    for (auto& h : half) {
      h = random_half(rng);
      if (all_normal && (h & 0x7c00u) == 0x7c00u) h &= 0xbfffu;  // keep most inputs finite
    }
    const int st = ti_host_quantize_f16(half.data(), count, cols, q.data(), count, scales.data(), cols);
    if (st == TI_HOST_OK) {
      ++quantized;
      if (ti_host_dequantize_i8(q.data(), count, cols, scales.data(), cols, out.data(), count) != TI_HOST_OK)
        fail("a quantized matrix does not dequantize", it);
      for (int8_t v : q)
        if (v == -128) fail("quantized value -128", it);
    } else if (st == TI_HOST_INVALID) {
      ++rejected;
    } else {
      fail("quantize returned neither OK nor INVALID", it);
    }
    for (auto& v : q) v = int8_t(int(rng() % 256) - 128);
    for (auto& s : scales) {
      if (rng() % 4 == 0) {
        const uint32_t bits = uint32_t(rng());
        std::memcpy(&s, &bits, 4);
      } else {
        s = std::uniform_real_distribution<float>(1e-4f, 2.f)(rng);
      }
    }
    const int ds = ti_host_dequantize_i8(q.data(), count, cols, scales.data(), cols, out.data(), count);
    if (ds == TI_HOST_OK) ++dequantized;
    else if (ds != TI_HOST_INVALID) fail("dequantize returned neither OK nor INVALID", it);
    if (count > 1) {
      std::vector<int8_t> q_short(count - 1);
      std::vector<uint16_t> out_short(count - 1);
      if (ti_host_quantize_f16(half.data(), count, cols, q_short.data(), count - 1, scales.data(), cols) !=
          TI_HOST_INVALID)
        fail("a short q buffer was not refused", it);
      if (ti_host_dequantize_i8(q.data(), count, cols, scales.data(), cols, out_short.data(), count - 1) !=
          TI_HOST_INVALID)
        fail("a short output buffer was not refused", it);
    }
    // ---- CPU kernels over ragged shapes
    const int m = 1 + int(rng() % 65), n = 1 + int(rng() % 65), k = 1 + int(rng() % 65);
    std::vector<float> a(size_t(m) * k), b(size_t(k) * n), y(size_t(m) * n);
    for (auto& v : a) v = random_finite(rng);
    for (auto& v : b) v = random_finite(rng);
    ti_cpu_gemm(a.data(), b.data(), y.data(), m, k, n);
    for (float v : y)
      if (!std::isfinite(v)) fail("gemm of finite inputs is not finite", it);
    std::vector<float> x(size_t(m) * n), g(n), be(n), z(size_t(m) * n);
    for (auto& v : x) v = random_finite(rng);
    for (auto& v : g) v = random_finite(rng);
    for (auto& v : be) v = random_finite(rng);
    ti_cpu_softmax(x.data(), z.data(), m, n);
    for (int r = 0; r < m; ++r) {
      double s = 0;
      for (int c = 0; c < n; ++c) s += z[size_t(r) * n + c];
      if (std::fabs(s - 1.0) > 1e-4) fail("softmax row does not sum to 1", it);
    }
    ti_cpu_layernorm(x.data(), g.data(), be.data(), z.data(), m, n, 1e-5f);
    for (float v : z)
      if (!std::isfinite(v)) fail("layernorm of finite inputs is not finite", it);
  }
  std::printf("ok %d %d %d\n", quantized, rejected, dequantized);
  return 0;
}
