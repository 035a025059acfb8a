/* libtinyinfer_backend.so, v2 kernel ABI — MI355X (gfx950) implementation.
 *
 * Every declaration below replaces the entry point of the same name declared at
 * reference backend/include/tinyinfer_backend_v2.h:7-38 (definitions at
 * reference backend/runtime_v2.cu:31-107).  Names, argument order, status codes
 * and validation rules are kept so that llm/native_ops.py (ctypes table at
 * reference llm/native_ops.py:40-50) binds this library unchanged.
 *
 * Conventions (same as the reference contract):
 *  - fp16 tensors are passed as uint16_t bit patterns; all tensor pointers are
 *    device pointers to contiguous row-major storage owned by the caller.
 *  - stream is a raw hipStream_t cast to uintptr_t (0 = legacy default stream);
 *    device must equal the caller's current HIP device (else status 2).
 *  - Success means "queued": device faults surface on a later call or sync.
 *  - Validation failures enqueue nothing and set a thread-local message
 *    readable through ti_v2_last_error().
 *  - Dimension order is M,N,K (unlike the legacy ABI, which is m,k,n).
 */
#ifndef TINYINFER_BACKEND_V2_H
#define TINYINFER_BACKEND_V2_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
/* reference backend/include/tinyinfer_backend_v2.h:7-9 */
enum ti_v2_status { TI_V2_OK = 0, TI_V2_INVALID_ARGUMENT = 1, TI_V2_DEVICE_MISMATCH = 2,
                    TI_V2_UNSUPPORTED_CONFIG = 3, TI_V2_CUDA_ERROR = 4 };
enum ti_v2_output_dtype { TI_V2_FP16 = 0, TI_V2_FP32 = 1 };

/* Returns 2 (reference backend/runtime_v2.cu:31). */
int ti_v2_abi_version(void);
/* Thread-local message of the last failing call on this thread; cleared at the
 * start of every entry point (reference backend/runtime_v2.cu:11-12,20,32). */
const char* ti_v2_last_error(void);
/* The 12-entry GEMM catalog JSON, byte-identical to reference
 * backend/runtime_v2.cu:33-53 (NativeOps compares it, llm/native_ops.py:57-62). */
const char* ti_v2_gemm_catalog_json(void);

/* C[M,N] = A[M,K] fp16 x B[K,N] fp16 (+ bias fp16[N]); fp32 accumulation; output
 * fp16 (output_dtype 0) or fp32 (1).  Fused-epilogue configs 0..5 only.
 * Replaces reference backend/runtime_v2.cu:54-57. */
int ti_v2_gemm_f16(const uint16_t* a, const uint16_t* b, const uint16_t* bias, void* y,
                   int m, int n, int k, int output_dtype, int config, uintptr_t stream, int device);
/* W8A16: B[k,n] = fp16_rn(float(q[k,n]) * scales[n]); q int8 [K,N], scales fp32 [N].
 * Replaces reference backend/runtime_v2.cu:58-61. */
int ti_v2_gemm_i8(const uint16_t* a, const int8_t* q, const float* scales, const uint16_t* bias,
                  void* y, int m, int n, int k, int output_dtype, int config, uintptr_t stream,
                  int device);
/* _ex variants take the caller-owned fp32[M,N] workspace that configs 6..11
 * ("separate" epilogue) require; null for configs 0..5.
 * Replace reference backend/runtime_v2.cu:62-76. */
int ti_v2_gemm_ex_f16(const uint16_t* a, const uint16_t* b, const uint16_t* bias, void* y,
                      float* workspace, int m, int n, int k, int output_dtype, int config,
                      uintptr_t stream, int device);
int ti_v2_gemm_ex_i8(const uint16_t* a, const int8_t* q, const float* scales, const uint16_t* bias,
                     void* y, float* workspace, int m, int n, int k, int output_dtype, int config,
                     uintptr_t stream, int device);
/* FP32 C[M,N] = A[M,K] B[K,N].  Replaces reference backend/runtime_v2.cu:77-81. */
int ti_v2_legacy_gemm_f32(const float* a, const float* b, float* y, int m, int n, int k,
                          uintptr_t stream, int device);
/* q[B,H,Q,D], k/v[B,H,K,D] fp16, metadata int32[B] (device).  Rows whose query
 * is padded or sees no key are exactly 0.  D in {64,128}; config in {0,1}.
 * Replaces reference backend/runtime_v2.cu:82-90. */
int ti_v2_attention_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* y,
                        const int32_t* q_lengths, const int32_t* kv_lengths,
                        const int32_t* query_offsets, int batch, int heads, int q_len, int kv_len,
                        int head_dim, int causal, int config, uintptr_t stream, int device);
/* Row LayerNorm, fp16 in/out, fp32 statistics.  Replaces backend/runtime_v2.cu:91-97. */
int ti_v2_layernorm_f16(const uint16_t* x, const uint16_t* gamma, const uint16_t* beta,
                        uint16_t* y, int rows, int cols, float eps, uintptr_t stream, int device);
/* tanh-GELU, fp16 in/out.  Replaces reference backend/runtime_v2.cu:98-102. */
int ti_v2_gelu_new_f16(const uint16_t* x, uint16_t* y, int64_t count, uintptr_t stream,
                       int device);
/* Last-axis softmax, fp16 in/out.  Replaces reference backend/runtime_v2.cu:103-107. */
int ti_v2_softmax_f16(const uint16_t* x, uint16_t* y, int rows, int cols, uintptr_t stream,
                      int device);
#ifdef __cplusplus
}
#endif
#endif
