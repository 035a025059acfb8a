// libtinyinfer_backend.so: the v2 C ABI (declared in include/tinyinfer_backend_v2.h).
//
// Each entry point checks its arguments with the rules of reference
// backend/include/tinyinfer_host_validation.hpp:23-70 (device match first, as
// reference backend/runtime_v2.cu:19-25), enqueues nothing when a check fails,
// and otherwise launches the gfx950 kernels on the caller's stream.
#include <cmath>
#include <cstdio>
#include <initializer_list>
#include <limits>

#include "../../include/tinyinfer_amd_ext.h"
#include "../../include/tinyinfer_backend_v2.h"
#include "kernels.hpp"

namespace {

thread_local char error_text[256] = "";

int fail(int status, const char* text) {
  std::snprintf(error_text, sizeof(error_text), "%s", text);
  return status;
}
int hip_status(hipError_t e) { return e == hipSuccess ? TI_V2_OK : fail(TI_V2_CUDA_ERROR, hipGetErrorString(e)); }

int begin(int device) {
  error_text[0] = '\0';
  if (device < 0) return fail(TI_V2_INVALID_ARGUMENT, "device must be nonnegative");
  int current = -1;
  const hipError_t e = hipGetDevice(&current);
  if (e != hipSuccess) return hip_status(e);
  return current == device ? TI_V2_OK : fail(TI_V2_DEVICE_MISMATCH, "caller must select the supplied HIP device");
}

bool aligned(const void* p, size_t bytes) { return p && reinterpret_cast<uintptr_t>(p) % bytes == 0; }
bool shape_fits(std::initializer_list<int> dims, size_t bytes) {
  uint64_t product = bytes;
  for (int d : dims) {
    if (d <= 0 || product > uint64_t(std::numeric_limits<int64_t>::max()) / uint64_t(d)) return false;
    product *= uint64_t(d);
  }
  return true;
}

// Catalog semantics of reference kernels/src/cuda/tc/catalog.cuh:8-15; this
// build compiles every configuration (only_config = -1).
bool config_available(int id) { return id >= 0 && id < 12; }
int config_tile(int id) { return id % 3; }
bool config_separate(int id) { return id >= 6; }

int check_gemm(const void* a, const void* b, const void* bias, const void* y, int m, int n, int k,
               int dtype, int config, bool int8) {
  if (!config_available(config))
    return fail(TI_V2_UNSUPPORTED_CONFIG, "GEMM config absent from this compiled allow-list");
  const int bm = config_tile(config) == 0 ? 32 : 64;
  if ((dtype != 0 && dtype != 1) || !aligned(a, 2) || !aligned(b, int8 ? 1 : 2) ||
      !aligned(y, dtype == 0 ? 2 : 4) || (bias && !aligned(bias, 2)) || !shape_fits({m, k}, 2) ||
      !shape_fits({k, n}, int8 ? 1 : 2) || !shape_fits({m, n}, dtype == 0 ? 2 : 4) ||
      (m - 1) / bm + 1 > 65535)
    return fail(TI_V2_INVALID_ARGUMENT, "invalid GEMM shape, pointers, alignment, output dtype or grid");
  return TI_V2_OK;
}
int check_workspace(const void* p, int m, int n, int config) {
  if (config_separate(config) && (!aligned(p, 4) || !shape_fits({m, n}, 4)))
    return fail(TI_V2_INVALID_ARGUMENT, "separate epilogue requires caller-owned FP32[M,N] workspace");
  return TI_V2_OK;
}

// Split-K partials go to the calling queue's slot of the library's static pool
// and are finished in the same launch: nothing is allocated, and the call can
// be captured into a graph on any stream.
int run_gemm(const uint16_t* a, const void* w, bool int8, const float* scales, const uint16_t* bias,
             void* y, float* workspace, int m, int n, int k, int dtype, int config, uintptr_t stream) {
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  tia::GemmArgs g;
  g.a = a;
  g.lda = k;
  g.w = w;
  g.w_int8 = int8;
  g.scales = scales;
  g.m = m;
  g.n = n;
  g.k = k;
  const bool separate = config_separate(config);
  if (separate) {
    g.epi.kind = tia::EPI_RAW_F32;
    g.epi.y = workspace;
  } else {
    g.epi.kind = dtype == 1 ? tia::EPI_F32 : tia::EPI_F16;
    g.epi.bias = bias;
    g.epi.y = y;
  }
  g.epi.ldy = n;
  hipError_t err = tia::gemm(g, tia::queue_pool_scratch(), st);
  if (err == hipSuccess && separate) err = tia::bias_epilogue(workspace, bias, y, int64_t(m) * n, n, dtype, st);
  return hip_status(err);
}

}  // namespace

extern "C" int ti_v2_abi_version(void) { return 2; }
extern "C" const char* ti_v2_last_error(void) { return error_text; }
extern "C" const char* ti_v2_gemm_catalog_json(void) {
  return "{\"schema_version\":1,\"only_config\":-1,\"configs\":["
         "{\"id\":0,\"tile\":[32,32,16,4],\"stages\":2,\"epilogue\":\"fused\"},"
         "{\"id\":1,\"tile\":[64,32,32,8],\"stages\":2,\"epilogue\":\"fused\"},"
         "{\"id\":2,\"tile\":[64,64,32,8],\"stages\":2,\"epilogue\":\"fused\"},"
         "{\"id\":3,\"tile\":[32,32,16,4],\"stages\":1,\"epilogue\":\"fused\"},"
         "{\"id\":4,\"tile\":[64,32,32,8],\"stages\":1,\"epilogue\":\"fused\"},"
         "{\"id\":5,\"tile\":[64,64,32,8],\"stages\":1,\"epilogue\":\"fused\"},"
         "{\"id\":6,\"tile\":[32,32,16,4],\"stages\":2,\"epilogue\":\"separate\"},"
         "{\"id\":7,\"tile\":[64,32,32,8],\"stages\":2,\"epilogue\":\"separate\"},"
         "{\"id\":8,\"tile\":[64,64,32,8],\"stages\":2,\"epilogue\":\"separate\"},"
         "{\"id\":9,\"tile\":[32,32,16,4],\"stages\":1,\"epilogue\":\"separate\"},"
         "{\"id\":10,\"tile\":[64,32,32,8],\"stages\":1,\"epilogue\":\"separate\"},"
         "{\"id\":11,\"tile\":[64,64,32,8],\"stages\":1,\"epilogue\":\"separate\"}]}";
}

extern "C" int ti_v2_gemm_ex_f16(const uint16_t* a, const uint16_t* b, const uint16_t* bias, void* y,
                                 float* workspace, int m, int n, int k, int dtype, int config,
                                 uintptr_t stream, int device) {
  int status = begin(device);
  if (status) return status;
  if ((status = check_gemm(a, b, bias, y, m, n, k, dtype, config, false))) return status;
  if ((status = check_workspace(workspace, m, n, config))) return status;
  return run_gemm(a, b, false, nullptr, bias, y, workspace, m, n, k, dtype, config, stream);
}

extern "C" int ti_v2_gemm_ex_i8(const uint16_t* a, const int8_t* b, const float* scales,
                                const uint16_t* bias, void* y, float* workspace, int m, int n, int k,
                                int dtype, int config, uintptr_t stream, int device) {
  int status = begin(device);
  if (status) return status;
  if ((status = check_gemm(a, b, bias, y, m, n, k, dtype, config, true))) return status;
  if (!aligned(scales, 4)) return fail(TI_V2_INVALID_ARGUMENT, "scales pointer must be nonnull aligned FP32[N]");
  if ((status = check_workspace(workspace, m, n, config))) return status;
  return run_gemm(a, b, true, scales, bias, y, workspace, m, n, k, dtype, config, stream);
}

// ti_amd_gemm_ex_i8_noalloc: ti_v2_gemm_ex_i8 for callers that must not
// allocate.  Every entry point of this library is allocation-free (split
// work goes to the queue pool), so it is the same call: same arguments,
// validation, status codes and bits.
extern "C" int ti_amd_gemm_ex_i8_noalloc(const uint16_t* a, const int8_t* b, const float* scales,
                                         const uint16_t* bias, void* y, float* workspace, int m, int n,
                                         int k, int dtype, int config, uintptr_t stream, int device) {
  return ti_v2_gemm_ex_i8(a, b, scales, bias, y, workspace, m, n, k, dtype, config, stream, device);
}

extern "C" int ti_v2_gemm_f16(const uint16_t* a, const uint16_t* b, const uint16_t* bias, void* y,
                              int m, int n, int k, int dtype, int config, uintptr_t stream, int device) {
  return ti_v2_gemm_ex_f16(a, b, bias, y, nullptr, m, n, k, dtype, config, stream, device);
}

extern "C" int ti_v2_gemm_i8(const uint16_t* a, const int8_t* b, const float* scales,
                             const uint16_t* bias, void* y, int m, int n, int k, int dtype, int config,
                             uintptr_t stream, int device) {
  return ti_v2_gemm_ex_i8(a, b, scales, bias, y, nullptr, m, n, k, dtype, config, stream, device);
}

extern "C" int ti_v2_legacy_gemm_f32(const float* a, const float* b, float* y, int m, int n, int k,
                                     uintptr_t stream, int device) {
  int status = begin(device);
  if (status) return status;
  if (!aligned(a, 4) || !aligned(b, 4) || !aligned(y, 4) || !shape_fits({m, k}, 4) ||
      !shape_fits({k, n}, 4) || !shape_fits({m, n}, 4) || (m - 1) / 64 + 1 > 65535)
    return fail(TI_V2_INVALID_ARGUMENT, "invalid FP32 GEMM arguments");
  return hip_status(tia::legacy_gemm_f32(a, b, y, m, n, k, reinterpret_cast<hipStream_t>(stream)));
}

extern "C" int ti_amd_legacy_gemm_f32_variant(int variant, const float* a, const float* b, float* y, int m, int n,
                                              int k, uintptr_t stream, int device) {
  int status = begin(device);
  if (status) return status;
  if (variant < 0 || variant > 2) return fail(TI_V2_UNSUPPORTED_CONFIG, "FP32 GEMM variant must be 0, 1 or 2");
  if (!aligned(a, 4) || !aligned(b, 4) || !aligned(y, 4) || !shape_fits({m, k}, 4) || !shape_fits({k, n}, 4) ||
      !shape_fits({m, n}, 4) || (m - 1) / 16 + 1 > 65535)
    return fail(TI_V2_INVALID_ARGUMENT, "invalid FP32 GEMM arguments");
  return hip_status(tia::legacy_gemm_f32_variant(variant, a, b, y, m, n, k, reinterpret_cast<hipStream_t>(stream)));
}

extern "C" int ti_v2_attention_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* y,
                                   const int32_t* ql, const int32_t* kl, const int32_t* offsets, int b,
                                   int h, int nq, int nk, int d, int causal, int config,
                                   uintptr_t stream, int device) {
  int status = begin(device);
  if (status) return status;
  if (config < 0 || config > 1) return fail(TI_V2_UNSUPPORTED_CONFIG, "attention config must be 0,1");
  if ((d != 64 && d != 128) || (causal != 0 && causal != 1) || b > 65535 || h > 65535 ||
      !shape_fits({b, h, nq, d}, 2) || !shape_fits({b, h, nk, d}, 2) || !aligned(q, 2) ||
      !aligned(k, 2) || !aligned(v, 2) || !aligned(y, 2) || !aligned(ql, 4) || !aligned(kl, 4) ||
      !aligned(offsets, 4))
    return fail(TI_V2_INVALID_ARGUMENT, "invalid attention arguments");
  tia::AttnArgs a;
  a.q = q;
  a.q_sq = d;
  a.q_sh = int64_t(nq) * d;
  a.q_sb = int64_t(h) * nq * d;
  a.k = k;
  a.v = v;
  a.kv_sh = int64_t(nk) * d;
  a.kv_sb = int64_t(h) * nk * d;
  a.out = y;
  a.o_sq = a.q_sq;
  a.o_sh = a.q_sh;
  a.o_sb = a.q_sb;
  a.q_lengths = ql;
  a.kv_lengths = kl;
  a.offsets = offsets;
  a.batch = b;
  a.heads = h;
  a.q_len = nq;
  a.kv_len = nk;
  a.head_dim = d;
  a.causal = causal != 0;
  // A long single-query call splits its keys across workgroups, the chunk
  // states in the calling queue's slot of the library's static pool (merged in
  // the same launch; the choice follows the shape alone).
  return hip_status(tia::attention(a, reinterpret_cast<hipStream_t>(stream), tia::queue_pool_scratch()));
}

extern "C" int ti_v2_layernorm_f16(const uint16_t* x, const uint16_t* g, const uint16_t* b, uint16_t* y,
                                   int rows, int cols, float eps, uintptr_t stream, int device) {
  int status = begin(device);
  if (status) return status;
  if (!shape_fits({rows, cols}, 2) || !std::isfinite(eps) || eps <= 0.f || !aligned(x, 2) ||
      !aligned(g, 2) || !aligned(b, 2) || !aligned(y, 2))
    return fail(TI_V2_INVALID_ARGUMENT, "invalid LayerNorm arguments");
  return hip_status(tia::layernorm_f16(x, g, b, y, rows, cols, eps, reinterpret_cast<hipStream_t>(stream)));
}

extern "C" int ti_v2_gelu_new_f16(const uint16_t* x, uint16_t* y, int64_t count, uintptr_t stream,
                                  int device) {
  int status = begin(device);
  if (status) return status;
  if (count <= 0 || count > std::numeric_limits<int64_t>::max() / 2 || !aligned(x, 2) || !aligned(y, 2))
    return fail(TI_V2_INVALID_ARGUMENT, "invalid GELU arguments");
  return hip_status(tia::gelu_f16(x, y, count, reinterpret_cast<hipStream_t>(stream)));
}

extern "C" int ti_v2_softmax_f16(const uint16_t* x, uint16_t* y, int rows, int cols, uintptr_t stream,
                                 int device) {
  int status = begin(device);
  if (status) return status;
  if (!shape_fits({rows, cols}, 2) || !aligned(x, 2) || !aligned(y, 2))
    return fail(TI_V2_INVALID_ARGUMENT, "invalid softmax arguments");
  return hip_status(tia::softmax_f16(x, y, rows, cols, reinterpret_cast<hipStream_t>(stream)));
}

extern "C" int ti_amd_gemm_i8_fused(const uint16_t* a, const int8_t* q, const float* scales,
                                    const uint16_t* bias, uint16_t* y, const uint16_t* residual,
                                    int m, int n, int k, int epilogue, uintptr_t stream, int device) {
  int status = begin(device);
  if (status) return status;
  if ((status = check_gemm(a, q, bias, y, m, n, k, 0, 0, true))) return status;
  if (!aligned(scales, 4)) return fail(TI_V2_INVALID_ARGUMENT, "scales pointer must be nonnull aligned FP32[N]");
  if (epilogue < 0 || epilogue > 2 || (epilogue == 2 && !aligned(residual, 2)))
    return fail(TI_V2_INVALID_ARGUMENT, "epilogue must be 0 (bias), 1 (bias+GELU) or 2 (bias+residual)");
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  tia::GemmArgs g;
  g.a = a;
  g.lda = k;
  g.w = q;
  g.w_int8 = true;
  g.scales = scales;
  g.m = m;
  g.n = n;
  g.k = k;
  g.epi.kind = epilogue == 1 ? tia::EPI_GELU : (epilogue == 2 ? tia::EPI_RESIDUAL : tia::EPI_F16);
  g.epi.bias = bias;
  g.epi.y = y;
  g.epi.ldy = n;
  g.epi.residual = residual;
  g.epi.ldr = n;
  return hip_status(tia::gemm(g, tia::queue_pool_scratch(), st));
}

extern "C" int64_t ti_amd_packed_w8_bytes(int k, int n) {
  if (!shape_fits({k, n}, 1)) return 0;
  return int64_t(tia::packed_w8_bytes(k, n));
}

extern "C" int ti_amd_pack_w8(const int8_t* q, int k, int n, void* packed, uintptr_t stream, int device) {
  int status = begin(device);
  if (status) return status;
  if (!q || !aligned(packed, 16) || !shape_fits({k, n}, 1))
    return fail(TI_V2_INVALID_ARGUMENT, "pack_w8 needs int8 q[K,N] and a 16-byte aligned output");
  return hip_status(tia::pack_w8(q, n, k, n, packed, reinterpret_cast<hipStream_t>(stream)));
}

extern "C" int64_t ti_amd_packed_w16_bytes(int k, int n) {
  if (!shape_fits({k, n}, 2)) return 0;
  return int64_t(tia::packed_w16_bytes(k, n));
}

extern "C" int ti_amd_pack_w16(const int8_t* q, const float* scales, int k, int n, void* packed, uintptr_t stream,
                               int device) {
  int status = begin(device);
  if (status) return status;
  if (!q || !aligned(scales, 4) || !aligned(packed, 16) || !shape_fits({k, n}, 2))
    return fail(TI_V2_INVALID_ARGUMENT, "pack_w16 needs int8 q[K,N], fp32 scales[N] and a 16-byte aligned output");
  return hip_status(tia::pack_w16(q, n, scales, k, n, packed, reinterpret_cast<hipStream_t>(stream)));
}

extern "C" int ti_amd_gemm_w16p_fused(const uint16_t* a, const void* packed16, const uint16_t* bias, uint16_t* y,
                                      const uint16_t* residual, int m, int n, int k, int epilogue, uintptr_t stream,
                                      int device) {
  int status = begin(device);
  if (status) return status;
  if (m <= 32 || !aligned(a, 16) || !aligned(packed16, 16) || !aligned(y, 2) || (bias && !aligned(bias, 2)) ||
      k % 32 != 0 || !shape_fits({m, k}, 2) || !shape_fits({m, n}, 2) || !shape_fits({k, n}, 2))
    return fail(TI_V2_INVALID_ARGUMENT,
                "fp16-packed GEMM needs M > 32, K % 32 == 0 and 16-byte aligned A and packed weights");
  if (epilogue < 0 || epilogue > 2 || (epilogue == 2 && !aligned(residual, 2)))
    return fail(TI_V2_INVALID_ARGUMENT, "epilogue must be 0 (bias), 1 (bias+GELU) or 2 (bias+residual)");
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  tia::GemmArgs g;
  g.a = a;
  g.lda = k;
  g.w_f16p = packed16;
  g.w_int8 = true;
  g.m = m;
  g.n = n;
  g.k = k;
  g.epi.kind = epilogue == 1 ? tia::EPI_GELU : (epilogue == 2 ? tia::EPI_RESIDUAL : tia::EPI_F16);
  g.epi.bias = bias;
  g.epi.y = y;
  g.epi.ldy = n;
  g.epi.residual = residual;
  g.epi.ldr = n;
  return hip_status(tia::gemm(g, tia::queue_pool_scratch(), st));
}

extern "C" int ti_amd_gemm_w8p_fused(const uint16_t* a, const void* packed, const float* scales,
                                     const uint16_t* bias, uint16_t* y, const uint16_t* residual, int m,
                                     int n, int k, int epilogue, uintptr_t stream, int device) {
  int status = begin(device);
  if (status) return status;
  if (!aligned(a, 16) || !aligned(packed, 16) || !aligned(scales, 4) || !aligned(y, 2) ||
      (bias && !aligned(bias, 2)) || k % 64 != 0 || !shape_fits({m, k}, 2) || !shape_fits({k, n}, 1) ||
      !shape_fits({m, n}, 2) || (int64_t(m) + 63) / 64 * ((int64_t(n) + 63) / 64) > (int64_t(1) << 30))
    return fail(TI_V2_INVALID_ARGUMENT,
                "packed GEMM needs K % 64 == 0 and 16-byte aligned A and packed weights");
  if (epilogue < 0 || epilogue > 2 || (epilogue == 2 && !aligned(residual, 2)))
    return fail(TI_V2_INVALID_ARGUMENT, "epilogue must be 0 (bias), 1 (bias+GELU) or 2 (bias+residual)");
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  tia::GemmArgs g;
  g.a = a;
  g.lda = k;
  g.w = packed;
  g.w_packed = packed;
  g.w_int8 = true;
  g.scales = scales;
  g.m = m;
  g.n = n;
  g.k = k;
  g.epi.kind = epilogue == 1 ? tia::EPI_GELU : (epilogue == 2 ? tia::EPI_RESIDUAL : tia::EPI_F16);
  g.epi.bias = bias;
  g.epi.y = y;
  g.epi.ldy = n;
  g.epi.residual = residual;
  g.epi.ldr = n;
  return hip_status(tia::gemm(g, tia::queue_pool_scratch(), st));
}

extern "C" int ti_amd_gemm_w8p_ln_fused(const uint16_t* a, const uint16_t* gamma, const uint16_t* beta, float eps,
                                        const void* packed, const float* scales, const uint16_t* bias, uint16_t* y,
                                        const uint16_t* residual, int m, int n, int k, int epilogue,
                                        uintptr_t stream, int device) {
  int status = begin(device);
  if (status) return status;
  if (!tia::gemm_ln_supported(m, k, n) || !aligned(a, 16) || !aligned(gamma, 16) || !aligned(beta, 16) ||
      !aligned(packed, 16) || !aligned(scales, 4) || !aligned(y, 2) || (bias && !aligned(bias, 2)) ||
      !std::isfinite(eps) || eps <= 0.f || !shape_fits({m, n}, 2) || !shape_fits({k, n}, 1))
    return fail(TI_V2_INVALID_ARGUMENT,
                "LayerNorm-prologue GEMM needs 1 <= M <= 32, K % 64 == 0, K <= 2048, eps > 0 and 16-byte "
                "aligned A, gamma, beta and packed weights");
  if (epilogue < 0 || epilogue > 2 || (epilogue == 2 && !aligned(residual, 2)))
    return fail(TI_V2_INVALID_ARGUMENT, "epilogue must be 0 (bias), 1 (bias+GELU) or 2 (bias+residual)");
  tia::GemmArgs g;
  g.a = a;
  g.lda = k;
  g.w = packed;
  g.w_packed = packed;
  g.w_int8 = true;
  g.scales = scales;
  g.m = m;
  g.n = n;
  g.k = k;
  g.ln_gamma = gamma;
  g.ln_beta = beta;
  g.ln_eps = eps;
  g.epi.kind = epilogue == 1 ? tia::EPI_GELU : (epilogue == 2 ? tia::EPI_RESIDUAL : tia::EPI_F16);
  g.epi.bias = bias;
  g.epi.y = y;
  g.epi.ldy = n;
  g.epi.residual = residual;
  g.epi.ldr = n;
  return hip_status(tia::gemm(g, nullptr, reinterpret_cast<hipStream_t>(stream)));
}

extern "C" int ti_amd_layernorm_f32(const float* x, const float* g, const float* b, float* y, int rows, int cols,
                                    float eps, uintptr_t stream, int device) {
  int status = begin(device);
  if (status) return status;
  if (!shape_fits({rows, cols}, 4) || !std::isfinite(eps) || eps <= 0.f || !aligned(x, 4) || !aligned(g, 4) ||
      !aligned(b, 4) || !aligned(y, 4))
    return fail(TI_V2_INVALID_ARGUMENT, "invalid LayerNorm arguments");
  return hip_status(tia::layernorm_f32(x, g, b, y, rows, cols, eps, reinterpret_cast<hipStream_t>(stream)));
}

extern "C" int ti_amd_layernorm_softmax_f32(const float* x, const float* g, const float* b, float* y, int rows,
                                            int cols, float eps, uintptr_t stream, int device) {
  int status = begin(device);
  if (status) return status;
  if (!shape_fits({rows, cols}, 4) || !std::isfinite(eps) || eps <= 0.f || !aligned(x, 4) || !aligned(g, 4) ||
      !aligned(b, 4) || !aligned(y, 4))
    return fail(TI_V2_INVALID_ARGUMENT, "invalid LayerNorm->softmax arguments");
  const int64_t bytes = int64_t(rows) * cols * 4;
  const auto xb = reinterpret_cast<uintptr_t>(x), yb = reinterpret_cast<uintptr_t>(y);
  if (rows > 0 && cols > 0 && xb < yb + uintptr_t(bytes) && yb < xb + uintptr_t(bytes))
    return fail(TI_V2_INVALID_ARGUMENT, "LayerNorm->softmax output must not overlap its input");
  return hip_status(tia::layernorm_softmax_f32(x, g, b, y, rows, cols, eps, reinterpret_cast<hipStream_t>(stream)));
}

extern "C" int ti_amd_softmax_f32(const float* x, float* y, int rows, int cols, uintptr_t stream, int device) {
  int status = begin(device);
  if (status) return status;
  if (!shape_fits({rows, cols}, 4) || !aligned(x, 4) || !aligned(y, 4))
    return fail(TI_V2_INVALID_ARGUMENT, "invalid softmax arguments");
  return hip_status(tia::softmax_f32(x, y, rows, cols, reinterpret_cast<hipStream_t>(stream)));
}
