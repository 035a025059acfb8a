// A caller of the legacy FP32 CPU ABI shaped like tinyc's generated "hand" code
// (reference tinyc/codegen_cpp.py:102-132 with tinyc/runtime/tinyc_runtime.hpp:
// the GEMM goes through ti_cpu_gemm(a, b, tmp, m, k, n) -- the legacy (m, k, n)
// argument order -- into a temporary, then an epilogue adds the bias; LayerNorm
// and Softmax are the ti_cpu_* calls).  Built against include/tinyinfer_backend.h
// and linked to libtinyinfer_backend.so, as tinyc links TINYC_BACKEND_LIBRARY.
//
// Usage: hand_cpu M K N in.bin out.bin
//   in.bin : float32 x[M,K], w[K,N], bias[N], gamma[N], beta[N]
//   out.bin: float32 linear[M,N], layernorm[M,N], softmax[M,N]
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "tinyinfer_backend.h"

namespace {
template <class Epi>
void gemm_hand(float* tmp, const float* a, const float* b, int m, int k, int n, Epi epi) {
  ti_cpu_gemm(a, b, tmp, m, k, n);
  for (int i = 0; i < m; ++i)
    for (int j = 0; j < n; ++j) epi(i, j, tmp[size_t(i) * n + j]);
}
}  // namespace

int main(int argc, char** argv) {
  if (argc != 6) return 2;
  const int m = std::atoi(argv[1]), k = std::atoi(argv[2]), n = std::atoi(argv[3]);
  const size_t in_count = size_t(m) * k + size_t(k) * n + 3 * size_t(n);
  std::vector<float> in(in_count), out(3 * size_t(m) * n), tmp(size_t(m) * n);
  FILE* f = std::fopen(argv[4], "rb");
  if (!f || std::fread(in.data(), sizeof(float), in_count, f) != in_count) return 3;
  std::fclose(f);
  const float *x = in.data(), *w = x + size_t(m) * k, *bias = w + size_t(k) * n, *g = bias + n, *b = g + n;
  float *lin = out.data(), *ln = lin + size_t(m) * n, *sm = ln + size_t(m) * n;
  gemm_hand(tmp.data(), x, w, m, k, n, [&](int i, int j, float v) { v += bias[j]; lin[size_t(i) * n + j] = v; });
  ti_cpu_layernorm(lin, g, b, ln, m, n, 1e-5f);
  ti_cpu_softmax(ln, sm, m, n);
  f = std::fopen(argv[5], "wb");
  if (!f || std::fwrite(out.data(), sizeof(float), out.size(), f) != out.size()) return 4;
  std::fclose(f);
  return 0;
}
