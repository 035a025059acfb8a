// Internal launcher interface shared by the v2 C ABI (backend_v2.hip), the
// legacy ABI (backend_legacy.hip) and the GPT-2 runtime (llm_runtime.hip).
// Everything here enqueues on the given stream and returns the launch status.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tia {

// What a GEMM does with each finished fp32 accumulator C[m][n].
enum EpiKind : int {
  EPI_F16 = 0,       // y16[m][n] = fp16_rn(acc + bias[n])
  EPI_F32 = 1,       // y32[m][n] = acc + bias[n]
  EPI_GELU = 2,      // y16 = fp16_rn(gelu(fp16_rn(acc + bias)))
  EPI_RESIDUAL = 3,  // y16 = fp16_rn(res[m][n] + fp16_rn(acc + bias)); res may alias y
  EPI_RAW_F32 = 4,   // y32[m][n] = acc (the "separate" configs' workspace, no bias)
  EPI_QKV = 5,       // EPI_F16 into y, plus K/V columns scattered into the slot cache
};

struct Epilogue {
  int kind = EPI_F16;
  const uint16_t* bias = nullptr;  // fp16 [N] or null
  void* y = nullptr;
  int64_t ldy = 0;                 // row stride of y, elements
  const uint16_t* residual = nullptr;
  int64_t ldr = 0;
  // EPI_QKV: row m = b * qrows + t holds token t of request b; columns
  // [hidden, 2 hidden) are K and [2 hidden, 3 hidden) are V, head h at h*64.
  // Cache element ((((slot * layers + layer) * heads + h) * capacity + pos) * 64 + d),
  // pos = offsets[b] + t, written only when t < qlens[b].
  uint16_t* kcache = nullptr;
  uint16_t* vcache = nullptr;
  const int32_t* slots = nullptr;
  const int32_t* offsets = nullptr;
  const int32_t* qlens = nullptr;
  int qrows = 1, hidden = 0, heads = 0, layer = 0, layers = 0, capacity = 0;
  // Compact rows (a ragged prefill without padding): row row_start[b] + t holds
  // token t of request b, row_start[0..batch] ascending, row_start[batch] = M;
  // qrows is then ignored.
  const int32_t* row_start = nullptr;
  int batch = 0;
  // EPI_F16 / EPI_GELU / EPI_RESIDUAL: y (and residual) are P32 fragment-packed
  // (common.hpp p32_off) instead of row-major; ldy / ldr are ignored.
  bool p32 = false;
};

// Where split work goes.  Caller memory: split-K partial sums [splits][M][N]
// fp32 (and split-key attention states) finished by a second kernel or by the
// caller (a deferred GEMM); launches that share one such Scratch must be
// ordered (same stream).  queue_pool: no caller memory -- the split kernels use
// the calling hardware queue's slot of a static pool in the library and the
// last workgroup of each tile (or (b, h) row) finishes it in the same launch,
// so nothing is allocated and every call can be captured into a graph
// (queue_scratch.hpp); `partials` is then unused.
struct Scratch {
  float* partials = nullptr;
  size_t partial_floats = 0;
  bool queue_pool = false;
};
constexpr size_t kScratchPartialFloats = size_t(8) << 20;  // 32 MiB
// The scratch the C ABIs pass.
inline const Scratch* queue_pool_scratch() {
  static const Scratch s{nullptr, 0, true};
  return &s;
}

struct GemmArgs {
  const uint16_t* a = nullptr;  // fp16 [M, lda]
  int64_t lda = 0;
  const void* w = nullptr;      // int8 or fp16 [K, N] row-major
  bool w_int8 = true;
  const float* scales = nullptr;  // fp32 [N] for int8 weights
  int m = 0, n = 0, k = 0;
  int64_t ldw = 0;                // row stride of W in elements; 0 means n
  // Optional panel-packed copy of the int8 W (pack_w8).  When set, M <= 32,
  // K % 64 == 0 and A allows 16-byte loads, the GEMV over the packed records runs.
  const void* w_packed = nullptr;
  // Optional pre-dequantised fp16 copy of the int8 W (pack_w16): the M > 32
  // GEMM then runs as a plain fp16 MFMA GEMM over it (same values).
  const void* w_f16p = nullptr;
  // A is P32 fragment-packed (M <= 32, packed W; lda ignored).
  bool a_p32 = false;
  // Optional greedy partials (EPI_F32 logits): when the wide LM-head GEMV or a
  // one-split packed GEMV of up to 16 rows runs, it also writes each
  // workgroup's best (value, column) per row to amax_v/amax_i[row * groups +
  // group] (at most 32 * groups <= capacity entries; a row's partials are
  // contiguous) and sets *amax_groups = groups; otherwise *amax_groups = 0.
  // argmax_partials finishes them.
  float* amax_v = nullptr;
  int32_t* amax_i = nullptr;
  size_t amax_capacity = 0;
  int* amax_groups = nullptr;
  // Optional LayerNorm of the A rows (packed int8 W, M <= 32, gemm_ln_supported):
  // the GEMM multiplies fp16_rn((a - mean) * rsqrt(var + eps) * gamma + beta),
  // mean and var over the K columns of each row, as layernorm_f16 computes them.
  const uint16_t* ln_gamma = nullptr;
  const uint16_t* ln_beta = nullptr;
  float ln_eps = 1e-5f;
  // Batch-invariant sums (packed int8 or fp16-record weights): every
  // output element is accumulated in one order whatever M is -- K in 32-row
  // MFMA steps from 0 upward, no split-K -- so a prompt's rows come out the same
  // whether it is prefilled alone or beside others (the int8 panel and fp16
  // record kernels then agree bit for bit).
  bool canonical = false;
  // Decode rows of a caller that batches requests (the runtime): the kernel
  // family and K split are the same for every M up to 16, so a row's sums do
  // not depend on the batch (the single-row part-block GEMV is not used).
  bool decode_batches = false;
  // Another decode lane reads the same packed weights right after this launch
  // (the runtime's two-lane decode over cache-resident weights): the GEMV of
  // up to 16 rows reads them with cached loads instead of streaming them.
  bool weights_shared = false;
  // A deferred launch over packed weights splits K towards this many
  // workgroups (at least 4 K chunks per split, partials within the scratch).
  // The split count depends on the shape only, never on M.
  int defer_workgroups = 192;
  Epilogue epi;
};
// out[row] = the column of the largest value over the groups' partials (lowest
// column on ties, NaN never wins), rows <= 32.
hipError_t argmax_partials(const float* vals, const int32_t* idx, int groups, int rows, int32_t* out,
                           hipStream_t stream);
// Largest K / 64 a LayerNorm-prologue GEMM takes (one round of 8 waves x 4 chunks).
constexpr int kLnMaxChunks = 32;
bool gemm_ln_supported(int m, int k, int n);

// Panel-packed int8 weights: for column block cb (16 columns) and K chunk kc (64
// rows), a 1 KiB record at (cb * ceil(K/64) + kc) * 1024 bytes holding, for lane
// l = 0..63, column cb*16 + (l & 15) at rows kc*64 + 8*(l>>4) + 0..7 and
// kc*64 + 32 + 8*(l>>4) + 0..7 (16 bytes); entries past K or N are zero.
size_t packed_w8_bytes(int k, int n);
// fp16 B records of fp16_rn(float(q) * scale): for column block cb (16 columns)
// and K group kk (32 rows), 1 KiB at (cb * ceil(K/32) + kk) * 1024 bytes, lane l
// holding column cb*16 + (l & 15), rows kk*32 + 8*(l>>4) + 0..7; zero past K, N.
size_t packed_w16_bytes(int k, int n);
hipError_t pack_w16(const int8_t* q, int64_t ldq, const float* scales, int k, int n, void* out,
                    hipStream_t stream);
hipError_t pack_w8(const int8_t* q, int64_t ldq, int k, int n, void* out, hipStream_t stream);

// When `deferred` is non-null and the skinny (M <= 32) kernel runs, the epilogue
// is skipped: the raw fp32 sums are left in scratch->partials as [splits][M][N]
// and *deferred = splits (>= 1); the caller finishes them (e.g. with
// splitk_residual_layernorm).  Otherwise *deferred = 0 and the epilogue ran.
hipError_t gemm(const GemmArgs& args, const Scratch* scratch, hipStream_t stream,
                int* deferred = nullptr);
// Finishes a deferred GEMM whose N equals the row width `cols`, one wave per row:
//   x[r][c]    = fp16_rn(x[r][c] + fp16_rn(sum_s partials[s][r][c] + bias[c]))
//   norm[r][:] = LayerNorm(x[r][:]; gamma, beta, eps)   (fp16 out)
// i.e. the residual add of reference llm/src/runtime.cu:149/153 followed by the
// next ln (cols <= 2048).  p32: x and norm are P32 fragment-packed (rows <= 32,
// cols % 64 == 0); the partials stay row-major.
hipError_t splitk_residual_layernorm(const float* partials, int splits, int rows, int cols,
                                     const uint16_t* bias, uint16_t* x, const uint16_t* gamma,
                                     const uint16_t* beta, uint16_t* norm, float eps,
                                     hipStream_t stream, bool p32 = false);
// y = ws + bias (fp16 or fp32 output): the separate-epilogue pass of configs 6..11.
hipError_t bias_epilogue(const float* ws, const uint16_t* bias, void* y, int64_t count, int n,
                         int dtype, hipStream_t stream);
hipError_t legacy_gemm_f32(const float* a, const float* b, float* c, int m, int n, int k,
                           hipStream_t stream);
// Variant 0 naive, 1 LDS-tiled, 2 register-tiled (legacy_gemm_f32).
hipError_t legacy_gemm_f32_variant(int variant, const float* a, const float* b, float* c, int m, int n, int k,
                                   hipStream_t stream);

// Attention with generic strides (elements).  K/V of (b, h) start at
// k + slot(b) * kv_sb + h * kv_sh with consecutive keys D elements apart, where
// slot(b) = kv_slot ? kv_slot[b] : b.
struct AttnArgs {
  const uint16_t* q = nullptr;
  int64_t q_sb = 0, q_sh = 0, q_sq = 0;
  const uint16_t* k = nullptr;
  const uint16_t* v = nullptr;
  int64_t kv_sb = 0, kv_sh = 0;
  const int32_t* kv_slot = nullptr;
  uint16_t* out = nullptr;
  int64_t o_sb = 0, o_sh = 0, o_sq = 0;
  const int32_t* q_lengths = nullptr;
  const int32_t* kv_lengths = nullptr;
  const int32_t* offsets = nullptr;
  int batch = 0, heads = 0, q_len = 0, kv_len = 0, head_dim = 64;
  bool causal = true;
  // kv_lengths[b] is ignored and offsets[b] + q_lengths[b] used instead when set
  // (the runtime's slot cache: the visible length follows from the offset).
  bool kv_from_offsets = false;
  // Decode after a deferred QKV GEMM (q_len == 1, head_dim 64): q, k, v of the new
  // token of request b are fp16_rn(sum of qkv_partials[s][b][part * hidden + h*64 + d]
  // + qkv_bias[...]); the kernel stores k, v into the cache at position offsets[b]
  // and attends with q.  q and out strides are then ignored for q.
  const float* qkv_partials = nullptr;
  int qkv_splits = 0;
  const uint16_t* qkv_bias = nullptr;
  int hidden = 0;
  // Output row b * q_len + qi, columns h * head_dim + d, written P32
  // fragment-packed (rows < 32, heads * head_dim % 64 == 0); o_* ignored.
  bool out_p32 = false;
  // Several queries per request: one kernel variant whatever the grid, so a
  // query's result does not depend on the other requests of the call.
  bool batch_invariant = false;
  // Compact query rows (a ragged prefill without padding): query qi of request
  // b is q row q_row_start[b] + qi and out row likewise (q_sb / o_sb ignored),
  // and only its q_lengths[b] queries are written.
  const int32_t* q_row_start = nullptr;
};
// With the queue pool (queue_pool_scratch()), single-query attention over a
// long cache (kv_len 512 .. 4096 for head_dim 64, 256 .. 2048 for 128) in the
// ABI layout (no kv_slot, no lengths from offsets, no compact rows) splits the
// keys of each (b, h) across workgroups; the last chunk of a row to finish
// merges the row's chunk states in the same launch.
hipError_t attention(const AttnArgs& args, hipStream_t stream, const Scratch* scratch = nullptr);

hipError_t layernorm_f16(const uint16_t* x, const uint16_t* g, const uint16_t* b, uint16_t* y,
                         int rows, int cols, float eps, hipStream_t stream);
// The same over P32 fragment-packed x and y (rows <= 32, cols % 64 == 0).
hipError_t layernorm_f16_p32(const uint16_t* x, const uint16_t* g, const uint16_t* b, uint16_t* y,
                             int rows, int cols, float eps, hipStream_t stream);
hipError_t softmax_f16(const uint16_t* x, uint16_t* y, int rows, int cols, hipStream_t stream);
hipError_t gelu_f16(const uint16_t* x, uint16_t* y, int64_t count, hipStream_t stream);
hipError_t layernorm_f32(const float* x, const float* g, const float* b, float* y, int rows,
                         int cols, float eps, hipStream_t stream);
hipError_t softmax_f32(const float* x, float* y, int rows, int cols, hipStream_t stream);
// y = softmax(LayerNorm(x)) row by row in one pass (y may not alias x).
hipError_t layernorm_softmax_f32(const float* x, const float* g, const float* b, float* y, int rows,
                                int cols, float eps, hipStream_t stream);

}  // namespace tia
