// A caller of the legacy FP32 GPU ABI shaped like tinyc's generated CUDA "hand"
// code (reference tinyc/codegen_cuda.py:50-65 with
// tinyc/runtime/tinyc_cuda_runtime.cuh: ti_cuda_gemm(a, b, tmp, m, k, n) into a
// device temporary, an epilogue kernel adding the bias, then ti_cuda_layernorm
// and ti_cuda_softmax on device buffers and the default stream).  Built with
// hipcc against include/tinyinfer_backend.h, linked to libtinyinfer_backend.so.
//
// Usage: hand_gpu M K N in.bin out.bin   (file layout as hand_cpu.cpp)
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

#include "tinyinfer_backend.h"

#define CHECK(x)                                                                            \
  do {                                                                                      \
    hipError_t e_ = (x);                                                                    \
    if (e_ != hipSuccess) {                                                                 \
      std::fprintf(stderr, "HIP %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
      return 5;                                                                             \
    }                                                                                       \
  } while (0)

__global__ void bias_epilogue(const float* tmp, const float* bias, float* y, int m, int n) {
  const long i = long(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < long(m) * n) y[i] = tmp[i] + bias[i % n];
}

int main(int argc, char** argv) {
  if (argc != 6) return 2;
  const int m = std::atoi(argv[1]), k = std::atoi(argv[2]), n = std::atoi(argv[3]);
  const size_t in_count = size_t(m) * k + size_t(k) * n + 3 * size_t(n), mn = size_t(m) * n;
  std::vector<float> in(in_count), out(3 * mn);
  FILE* f = std::fopen(argv[4], "rb");
  if (!f || std::fread(in.data(), sizeof(float), in_count, f) != in_count) return 3;
  std::fclose(f);
  float *d_in = nullptr, *d_out = nullptr, *d_tmp = nullptr;
  CHECK(hipMalloc(&d_in, in_count * sizeof(float)));
  CHECK(hipMalloc(&d_out, 3 * mn * sizeof(float)));
  CHECK(hipMalloc(&d_tmp, mn * sizeof(float)));
  CHECK(hipMemcpy(d_in, in.data(), in_count * sizeof(float), hipMemcpyHostToDevice));
  const float *x = d_in, *w = x + size_t(m) * k, *bias = w + size_t(k) * n, *g = bias + n, *b = g + n;
  float *lin = d_out, *ln = lin + mn, *sm = ln + mn;
  ti_cuda_gemm(x, w, d_tmp, m, k, n);
  hipLaunchKernelGGL(bias_epilogue, dim3(unsigned((mn + 255) / 256)), dim3(256), 0, nullptr, d_tmp, bias, lin, m, n);
  CHECK(hipGetLastError());
  ti_cuda_layernorm(lin, g, b, ln, m, n, 1e-5f);
  ti_cuda_softmax(ln, sm, m, n);
  CHECK(hipDeviceSynchronize());
  CHECK(hipMemcpy(out.data(), d_out, 3 * mn * sizeof(float), hipMemcpyDeviceToHost));
  CHECK(hipFree(d_in));
  CHECK(hipFree(d_out));
  CHECK(hipFree(d_tmp));
  f = std::fopen(argv[5], "wb");
  if (!f || std::fwrite(out.data(), sizeof(float), out.size(), f) != out.size()) return 4;
  std::fclose(f);
  return 0;
}
