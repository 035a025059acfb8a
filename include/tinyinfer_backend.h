/* libtinyinfer_backend.so, legacy FP32 ABI — the symbols tinyc's "hand"
 * dispatch emits (reference tinyc/codegen_cpp.py:128-131, codegen_cuda.py:61-64).
 * Replaces reference backend/include/tinyinfer_backend.h:2-9 (definitions at
 * reference backend/runtime.cpp:6-12).  GEMM argument order is (m,k,n).
 * ti_cpu_* take host pointers and run on the host (OpenMP).  ti_cuda_* take
 * device pointers, run on the legacy default stream, are synchronous with
 * respect to the host only through later synchronizing calls, and abort() on a
 * HIP error, as the reference does (reference kernels/src/cuda/common.cuh:6-14). */
#ifndef TINYINFER_BACKEND_H
#define TINYINFER_BACKEND_H
#ifdef __cplusplus
extern "C" {
#endif
void ti_cpu_gemm(const float* a, const float* b, float* y, int m, int k, int n);
void ti_cpu_softmax(const float* x, float* y, int rows, int cols);
void ti_cpu_layernorm(const float* x, const float* gamma, const float* beta, float* y, int rows,
                      int cols, float eps);
void ti_cuda_gemm(const float* a, const float* b, float* y, int m, int k, int n);
void ti_cuda_softmax(const float* x, float* y, int rows, int cols);
void ti_cuda_layernorm(const float* x, const float* gamma, const float* beta, float* y, int rows,
                       int cols, float eps);
#ifdef __cplusplus
}
#endif
#endif
