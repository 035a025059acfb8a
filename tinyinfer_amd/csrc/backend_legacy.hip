// libtinyinfer_backend.so: legacy FP32 GPU entry points ti_cuda_* (declared in
// include/tinyinfer_backend.h).  Same contract as reference backend/runtime.cpp:10-12
// and kernels/src/cuda/common.cuh:6-14: device pointers, the legacy default
// stream, and abort() with a message when a launch fails.
#include <cstdio>
#include <cstdlib>

#include "../../include/tinyinfer_backend.h"
#include "kernels.hpp"

namespace {
void check(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    std::fprintf(stderr, "HIP error %s in %s\n", hipGetErrorString(e), what);
    std::abort();
  }
}
}  // namespace

extern "C" void ti_cuda_gemm(const float* a, const float* b, float* y, int m, int k, int n) {
  check(tia::legacy_gemm_f32(a, b, y, m, n, k, nullptr), "ti_cuda_gemm");
}
extern "C" void ti_cuda_softmax(const float* x, float* y, int rows, int cols) {
  check(tia::softmax_f32(x, y, rows, cols, nullptr), "ti_cuda_softmax");
}
extern "C" void ti_cuda_layernorm(const float* x, const float* g, const float* b, float* y, int rows,
                                  int cols, float eps) {
  check(tia::layernorm_f32(x, g, b, y, rows, cols, eps, nullptr), "ti_cuda_layernorm");
}
