// libtinyinfer_backend.so: legacy FP32 CPU entry points ti_cpu_* (declared in
// include/tinyinfer_backend.h), the host functions tinyc's "hand" dispatch emits
// for C++ targets (reference backend/runtime.cpp:6-8).  OpenMP over rows / output
// tiles, SIMD inner loops, synchronous, host pointers.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>

#include "../../include/tinyinfer_backend.h"

extern "C" void ti_cpu_gemm(const float* a, const float* b, float* y, int m, int k, int n) {
  // C[m,n] = A[m,k] B[k,n]; 32 x 512 output panels, K streamed in 128-row slabs so
  // a B slab (256 KiB) stays in L2 while a panel's rows reuse it.
  constexpr int PM = 32, PN = 512, PK = 128;
  std::memset(y, 0, sizeof(float) * size_t(m) * n);
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int i0 = 0; i0 < m; i0 += PM)
    for (int j0 = 0; j0 < n; j0 += PN) {
      const int i1 = std::min(m, i0 + PM), j1 = std::min(n, j0 + PN);
      for (int k0 = 0; k0 < k; k0 += PK) {
        const int k1 = std::min(k, k0 + PK);
        for (int i = i0; i < i1; ++i) {
          float* __restrict__ yr = y + size_t(i) * n;
          for (int kk = k0; kk < k1; ++kk) {
            const float av = a[size_t(i) * k + kk];
            const float* __restrict__ br = b + size_t(kk) * n;
#pragma omp simd
            for (int j = j0; j < j1; ++j) yr[j] += av * br[j];
          }
        }
      }
    }
}

extern "C" void ti_cpu_softmax(const float* x, float* y, int rows, int cols) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const float* __restrict__ xr = x + size_t(r) * cols;
    float* __restrict__ yr = y + size_t(r) * cols;
    float mx = -std::numeric_limits<float>::infinity();
#pragma omp simd reduction(max : mx)
    for (int c = 0; c < cols; ++c) mx = std::max(mx, xr[c]);
    float s = 0.f;
#pragma omp simd reduction(+ : s)
    for (int c = 0; c < cols; ++c) {
      const float e = std::exp(xr[c] - mx);
      yr[c] = e;
      s += e;
    }
    const float inv = 1.f / s;
#pragma omp simd
    for (int c = 0; c < cols; ++c) yr[c] *= inv;
  }
}

extern "C" void ti_cpu_layernorm(const float* x, const float* g, const float* b, float* y, int rows,
                                 int cols, float eps) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const float* __restrict__ xr = x + size_t(r) * cols;
    float* __restrict__ yr = y + size_t(r) * cols;
    float s = 0.f;
#pragma omp simd reduction(+ : s)
    for (int c = 0; c < cols; ++c) s += xr[c];
    const float mean = s / float(cols);
    float ss = 0.f;
#pragma omp simd reduction(+ : ss)
    for (int c = 0; c < cols; ++c) ss += (xr[c] - mean) * (xr[c] - mean);
    const float inv = 1.f / std::sqrt(ss / float(cols) + eps);
#pragma omp simd
    for (int c = 0; c < cols; ++c) yr[c] = (xr[c] - mean) * inv * g[c] + b[c];
  }
}
