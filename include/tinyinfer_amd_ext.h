/* libtinyinfer_backend.so — entry points with no counterpart in the reference ABI.
 *
 * ti_amd_gemm_i8_fused: the W8A16 linear with the epilogues the GPT-2 runtime
 * fuses into the GEMM (the reference runs them as separate kernels:
 * reference llm/src/runtime.cu:149-153 residual adds, :151 gelu_new):
 *   epilogue 0: y = fp16_rn(acc + bias)
 *   epilogue 1: y = fp16_rn(gelu_tanh(fp16_rn(acc + bias)))
 *   epilogue 2: y = fp16_rn(residual + fp16_rn(acc + bias))   (residual may equal y)
 * a fp16 [M,K], q int8 [K,N], scales fp32 [N], bias fp16 [N] or null, y fp16 [M,N].
 * For callers that want the fused decode/prefill kernels standalone (the
 * configs[1] sweep, tests).  Validation and status codes as ti_v2_gemm_ex_i8. */
#ifndef TINYINFER_AMD_EXT_H
#define TINYINFER_AMD_EXT_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
int ti_amd_gemm_i8_fused(const uint16_t* a, const int8_t* q, const float* scales,
                         const uint16_t* bias, uint16_t* y, const uint16_t* residual, int m,
                         int n, int k, int epilogue, uintptr_t stream, int device);

/* ti_amd_legacy_gemm_f32_variant: the three FP32 GEMM variants behind
 * ikernels.cuda_bench_matmul(variant, ...) (reference
 * kernels/src/cuda/bench_api.cu:43-51 over kernels/src/cuda/matmul.cu:7-80):
 * 0 naive, 1 LDS-tiled, 2 register-tiled (what ti_cuda_gemm and
 * ti_v2_legacy_gemm_f32 run).  y[M,N] = a[M,K] @ b[K,N] in fp32, device
 * pointers, v2 status codes (3 for an unknown variant). */
int ti_amd_legacy_gemm_f32_variant(int variant, const float* a, const float* b, float* y, int m, int n, int k,
                                   uintptr_t stream, int device);

/* ti_amd_gemm_ex_i8_noalloc: no counterpart in the reference.  For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): ti_v2_gemm_ex_i8 with the same
 * arguments, validation, status codes and result bits.  It calls no hipMalloc,
 * hipFree or allocating library routine, and neither does ti_v2_gemm_ex_i8
 * any more: split-K work is finished by the last workgroup of the same launch,
 * with its fp32 partials in static device arrays of the library, one 4 MiB
 * slot per hardware queue (32 slots per GPU, held until the process ends).
 * Limit: a plan is only split when its partials fit the slot (1 Mi floats,
 * 1024 output tiles); larger shapes run unsplit, so no shape is refused.
 * Dispatches on one hardware queue never overlap, so calls on one stream, or
 * on streams that share a queue, do not race, and calls that overlap on
 * different queues use different slots; only with more than 32 hardware
 * queues in use on one GPU can two queues share a slot and overlapping calls
 * on them race. */
int ti_amd_gemm_ex_i8_noalloc(const uint16_t* a, const int8_t* b, const float* scales,
                              const uint16_t* bias, void* y, float* workspace, int m, int n, int k,
                              int dtype, int config, uintptr_t stream, int device);

/* Panel-packed int8 weights for the decode GEMV (M <= 32).  The reference keeps
 * q row-major [K,N] (reference kernels/src/cuda/tc/gemm.cu:21 reads
 * q[r*n + c]); the runtime packs every linear once at load so that each wave
 * load is one contiguous KiB already in MFMA B-operand order:
 *   record (cb, kc) at byte (cb * ceil(K/64) + kc) * 1024, cb = column block of
 *   16, kc = K chunk of 64; lane l's 16 bytes = column cb*16 + (l & 15), rows
 *   kc*64 + 8*(l >> 4) + 0..7 then kc*64 + 32 + 8*(l >> 4) + 0..7; zero past K/N.
 * ti_amd_packed_w8_bytes: size of the packed copy (0 for an invalid shape).
 * ti_amd_pack_w8: device q int8 [K,N] -> packed (16-byte aligned), on `stream`.
 * ti_amd_gemm_w8p_fused: ti_amd_gemm_i8_fused over packed weights, K % 64 == 0,
 * A and packed 16-byte aligned; M <= 32 runs the decode GEMV, M > 32 the
 * multistage MFMA GEMM (64x64 tiles, operands streamed HBM -> LDS with
 * global_load_lds).  Same arithmetic:
 * Y = epilogue(sum_k A[m,k] * fp16_rn(float(q[k,n]) * scales[n]) + bias[n]). */
int64_t ti_amd_packed_w8_bytes(int k, int n);
int ti_amd_pack_w8(const int8_t* q, int k, int n, void* packed, uintptr_t stream, int device);
int ti_amd_gemm_w8p_fused(const uint16_t* a, const void* packed, const float* scales,
                          const uint16_t* bias, uint16_t* y, const uint16_t* residual, int m, int n,
                          int k, int epilogue, uintptr_t stream, int device);

/* Pre-dequantised fp16 weights for the prefill GEMM (M > 32): every weight
 * fp16_rn(float(q[k,n]) * scales[n]) -- the values the int8 kernels compute on
 * the fly (reference kernels/src/cuda/tc/gemm.cu:21,24) -- stored once, so the
 * GEMM is a plain fp16 MFMA GEMM.  Layout: for column block cb (16 columns) and
 * K group kk (32 rows), 1 KiB at (cb * ceil(K/32) + kk) * 1024 bytes, lane l's
 * 16 bytes = column cb*16 + (l & 15), rows kk*32 + 8*(l >> 4) + 0..7; zero past
 * K/N.  ti_amd_packed_w16_bytes: its size; ti_amd_pack_w16: device q int8 [K,N]
 * + scales fp32 [N] -> packed; ti_amd_gemm_w16p_fused: Y = epilogue(A @ W +
 * bias) with the epilogues of ti_amd_gemm_i8_fused, M > 32, K % 32 == 0, A and
 * packed 16-byte aligned. */
int64_t ti_amd_packed_w16_bytes(int k, int n);
int ti_amd_pack_w16(const int8_t* q, const float* scales, int k, int n, void* packed, uintptr_t stream,
                    int device);
int ti_amd_gemm_w16p_fused(const uint16_t* a, const void* packed16, const uint16_t* bias, uint16_t* y,
                           const uint16_t* residual, int m, int n, int k, int epilogue, uintptr_t stream,
                           int device);

/* ti_amd_gemm_w8p_ln_fused: the decode GEMV with the LayerNorm that precedes
 * every GPT-2 linear fed from the residual stream (reference
 * llm/src/runtime.cu:143 ln_1 -> c_attn, :150 ln_2 -> c_fc) computed in its
 * prologue:
 *   Y = epilogue(sum_k LN(A)[m,k] * fp16_rn(float(q[k,n]) * scales[n]) + bias[n]),
 *   LN(A)[m,:] = fp16_rn((A[m,:] * inv - mean * inv) * gamma + beta),
 *   inv = rsqrt(var + eps),
 * mean and var (population, two passes) in fp32 over the K columns of row m,
 * as ti_v2_layernorm_f16 up to fp32 rounding.  The runtime uses it for decode;
 * a caller with many workgroups per row set (the LM head) is better served by
 * one ti_v2_layernorm_f16 pass, since every workgroup normalizes all M rows.  1 <= M <= 32, K % 64 == 0, K <= 2048; A, gamma, beta
 * and packed 16-byte aligned; epilogues as ti_amd_gemm_i8_fused. */
int ti_amd_gemm_w8p_ln_fused(const uint16_t* a, const uint16_t* gamma, const uint16_t* beta, float eps,
                             const void* packed, const float* scales, const uint16_t* bias, uint16_t* y,
                             const uint16_t* residual, int m, int n, int k, int epilogue,
                             uintptr_t stream, int device);

/* FP32 row LayerNorm / last-axis Softmax on a caller stream: the kernels behind
 * ti_cuda_layernorm / ti_cuda_softmax (reference backend/runtime.cpp:10-12),
 * with the v2 conventions (device pointers, stream, device check, status code
 * instead of abort) so they can be ordered with other work or graph-captured.
 * Validation as ti_v2_layernorm_f16 / ti_v2_softmax_f16 with 4-byte alignment. */
int ti_amd_layernorm_f32(const float* x, const float* gamma, const float* beta, float* y,
                         int rows, int cols, float eps, uintptr_t stream, int device);
int ti_amd_softmax_f32(const float* x, float* y, int rows, int cols, uintptr_t stream, int device);
/* y = softmax(LayerNorm(x; gamma, beta, eps)) over the last axis, FP32, one
 * pass per row: the LayerNorm -> Softmax graph that tinyc's norm_softmax issues
 * as ti_cuda_layernorm then ti_cuda_softmax (reference bench/integrated.py:87-92,
 * backend/runtime.cpp:10-12), with the same values as those two calls at half
 * the memory traffic.  Validation as ti_amd_layernorm_f32; y must not overlap x. */
int ti_amd_layernorm_softmax_f32(const float* x, const float* gamma, const float* beta, float* y,
                                 int rows, int cols, float eps, uintptr_t stream, int device);
#ifdef __cplusplus
}
#endif
#endif
