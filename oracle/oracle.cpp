// ORACLE — test infrastructure, not product code.
//
// A plain C++ (host, OpenMP) restatement of the reference tinyinfer arithmetic
// on the GPT-2 INT8 hot path.  Only tests/, __graft_entry__.smoke() and the
// cpu_baseline leg of bench.py may load it, and only as the checker (or the
// timed CPU baseline); the product libraries never link or call it.
//
// Each function cites the reference file:line it restates.  What pins each
// function (golden vectors, the compiled reference under oracle/_ref, closed
// forms and invariants) is listed in tests/test_oracle.py; a function with no
// such check would be marked "parity unpinned" here — there is none.
//
// Rounding points mirror the reference: fp16 storage at every kernel boundary,
// fp32 arithmetic inside, fp16 round-to-nearest-even on store.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <memory>
#include <vector>
#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

// ---- IEEE binary16 <-> binary32, round-to-nearest-even (bit exact) ----------
float h2f_compute(uint16_t h) {
  const uint32_t sign = uint32_t(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 31u, man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) bits = sign;
    else {  // subnormal: value = man * 2^-24
      float v = float(man) * 5.9604644775390625e-08f;
      std::memcpy(&bits, &v, 4);
      bits |= sign;
    }
  } else if (exp == 31) bits = sign | 0x7f800000u | (man << 13);
  else bits = sign | ((exp + 112u) << 23) | (man << 13);
  float out;
  std::memcpy(&out, &bits, 4);
  return out;
}

// binary16 -> binary32 through a table of all 65 536 patterns, each computed by
// h2f_compute (the same values, without the branches per element).
struct HalfTable {
  float v[65536];
  HalfTable() {
    for (uint32_t i = 0; i < 65536; ++i) v[i] = h2f_compute(uint16_t(i));
  }
};
const HalfTable kHalf;
inline float h2f(uint16_t h) { return kHalf.v[h]; }

uint16_t f2h(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint16_t sign = uint16_t((x >> 16) & 0x8000u);
  const uint32_t absx = x & 0x7fffffffu;
  if (absx >= 0x7f800000u) return uint16_t(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0u));
  if (absx >= 0x477ff000u) return uint16_t(sign | 0x7c00u);  // rounds to >= 65520 -> inf
  if (absx < 0x38800000u) {  // below the smallest normal half: result is subnormal or zero
    if (absx < 0x33000000u) return sign;  // < 2^-25 rounds to zero (ties at 2^-25 -> even 0)
    const int e = int(absx >> 23);           // biased fp32 exponent
    const uint32_t m = (absx & 0x7fffffu) | 0x800000u;
    const int shift = 126 - e;  // value = m * 2^(e-150); half ulp 2^-24 -> m >> (126-e)
    const uint32_t base = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
    const uint32_t r = base + ((rem > half || (rem == half && (base & 1u))) ? 1u : 0u);
    return uint16_t(sign | r);
  }
  const uint32_t base = absx >> 13, rem = absx & 0x1fffu;
  uint32_t r = base + ((rem > 0x1000u || (rem == 0x1000u && (base & 1u))) ? 1u : 0u);
  r -= (112u << 10);  // re-bias exponent 127 -> 15
  return uint16_t(sign | r);
}

inline float rt16(float v) { return h2f(f2h(v)); }

float gelu_tanh(float z) {
  // reference kernels/src/cuda/tc/elementwise.cu:31
  return 0.5f * z * (1.f + std::tanh(0.7978845608028654f * (z + 0.044715f * z * z * z)));
}

}  // namespace

extern "C" {

// ---- fp16 conversions exposed for tests -------------------------------------
void or_f32_to_f16(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = f2h(x[i]);
}
void or_f16_to_f32(const uint16_t* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = h2f(x[i]);
}

// ---- INT8 weight-only codec ---------------------------------------------------
// Restates reference backend/host_codec.cpp:78-84 (== llm/quantization.py:27-42):
// scale[c] = float(double(max|w|)/127) or 1 for a zero column;
// q = clamp(round_half_even(double(w)/double(scale)), -127, 127).
int or_quantize(const uint16_t* w, int64_t rows, int64_t cols, int8_t* q, float* scales) {
  if (rows <= 0 || cols <= 0) return 1;
  for (int64_t i = 0; i < rows * cols; ++i)
    if ((w[i] & 0x7c00u) == 0x7c00u) return 1;
  for (int64_t c = 0; c < cols; ++c) {
    float mx = 0.f;
    for (int64_t r = 0; r < rows; ++r) mx = std::max(mx, std::fabs(h2f(w[r * cols + c])));
    scales[c] = mx != 0.f ? float(double(mx) / 127.0) : 1.0f;
  }
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) {
      const double v = std::nearbyint(double(h2f(w[r * cols + c])) / double(scales[c]));
      q[r * cols + c] = int8_t(std::max(-127.0, std::min(127.0, v)));
    }
  return 0;
}

// Restates reference tinyinfer_quantization_scalar.h:10-12 + gemm.cu:21,24:
// W = fp16_rn(float(q) * scale[col]).
void or_dequantize(const int8_t* q, const float* scales, int64_t rows, int64_t cols, uint16_t* out) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) out[r * cols + c] = f2h(float(q[r * cols + c]) * scales[c]);
}

// ---- W8A16 / FP16 linear ------------------------------------------------------
// Restates reference kernels/src/cuda/tc/gemm.cu:10-26,73-80 (+ bias_epilogue
// :118-124): y = A[M,K] * W[K,N] accumulated in fp32, + float(bias), stored as
// fp16_rn (dtype 0) or fp32 (dtype 1).  epilogue 1 adds the fused tanh-GELU of
// the fp16-rounded biased value (the reference's separate gelu pass over the
// fp16 GEMM output, runtime.cu:150-151).  W is given either as int8+scales
// (wf16 == nullptr) or as fp16 bits.  Accumulation runs over k in increasing
// order for every output element.
void or_linear(const uint16_t* a, const int8_t* q, const float* scales, const uint16_t* wf16,
               const uint16_t* bias, int M, int N, int K, int dtype, int epilogue, void* y) {
  std::vector<float> af(size_t(M) * K);
  for (size_t i = 0; i < af.size(); ++i) af[i] = h2f(a[i]);
  std::vector<float> acc(size_t(M) * N, 0.f);
#pragma omp parallel
  {
    std::vector<float> wrow;
#pragma omp for schedule(static)
    for (int n0 = 0; n0 < N; n0 += 256) {
      const int n1 = std::min(N, n0 + 256);
      wrow.resize(size_t(n1 - n0));
      for (int k = 0; k < K; ++k) {
        for (int n = n0; n < n1; ++n)
          wrow[n - n0] = wf16 ? h2f(wf16[size_t(k) * N + n])
                              : h2f(f2h(float(q[size_t(k) * N + n]) * scales[n]));
        for (int m = 0; m < M; ++m) {
          const float av = af[size_t(m) * K + k];
          float* out = &acc[size_t(m) * N];
          for (int n = n0; n < n1; ++n) out[n] += av * wrow[n - n0];
        }
      }
    }
  }
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < N; ++n) {
      float v = acc[size_t(m) * N + n] + (bias ? h2f(bias[n]) : 0.f);
      if (epilogue == 1) v = gelu_tanh(rt16(v));
      if (dtype == 1) static_cast<float*>(y)[size_t(m) * N + n] = v;
      else static_cast<uint16_t*>(y)[size_t(m) * N + n] = f2h(v);
    }
}

// Reference kernels/src/cpu/matmul.cpp:17-43 (matmul_blocked, 64x256x256 tiles,
// OpenMP over output tiles): the CPU FP32 GEMM used as the W8A16 CPU baseline
// over dequantized weights.
void or_matmul_blocked(const float* A, const float* B, float* C, int M, int N, int K) {
  constexpr int BM = 64, BK = 256, BN = 256;
  std::memset(C, 0, sizeof(float) * size_t(M) * N);
#pragma omp parallel for collapse(2) schedule(static)
  for (int i0 = 0; i0 < M; i0 += BM)
    for (int j0 = 0; j0 < N; j0 += BN) {
      const int iM = std::min(i0 + BM, M), jM = std::min(j0 + BN, N);
      for (int k0 = 0; k0 < K; k0 += BK) {
        const int kM = std::min(k0 + BK, K);
        for (int i = i0; i < iM; ++i) {
          float* __restrict__ c = C + size_t(i) * N;
          const float* __restrict__ ar = A + size_t(i) * K;
          for (int k = k0; k < kM; ++k) {
            const float aik = ar[k];
            const float* __restrict__ b = B + size_t(k) * N;
#pragma omp simd
            for (int j = j0; j < jM; ++j) c[j] += aik * b[j];
          }
        }
      }
    }
}

// ---- LayerNorm / Softmax / GELU, fp16 (v2 ABI) --------------------------------
// Restates reference kernels/src/cuda/tc/elementwise.cu:15-27: two-pass mean and
// variance, inv = rsqrt(var + eps), y = fp16_rn((x - mean) * inv * g + b).
// Statistics are formed in double and rounded to fp32 once.
void or_layernorm_f16(const uint16_t* x, const uint16_t* g, const uint16_t* b, uint16_t* y,
                      int rows, int cols, float eps) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const uint16_t* xr = x + size_t(r) * cols;
    double s = 0;
    for (int c = 0; c < cols; ++c) s += h2f(xr[c]);
    const float mean = float(s / cols);
    double ss = 0;
    for (int c = 0; c < cols; ++c) {
      const double d = double(h2f(xr[c])) - double(mean);
      ss += d * d;
    }
    const float inv = float(1.0 / std::sqrt(double(float(ss / cols)) + double(eps)));
    for (int c = 0; c < cols; ++c)
      y[size_t(r) * cols + c] = f2h((h2f(xr[c]) - mean) * inv * h2f(g[c]) + h2f(b[c]));
  }
}

// Restates reference kernels/src/cuda/tc/elementwise.cu:34-46: max, sum of
// exp(x - max), y = fp16_rn(exp(x - max) / sum).
void or_softmax_f16(const uint16_t* x, uint16_t* y, int rows, int cols) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const uint16_t* xr = x + size_t(r) * cols;
    float mx = -std::numeric_limits<float>::infinity();
    for (int c = 0; c < cols; ++c) mx = std::max(mx, h2f(xr[c]));
    double s = 0;
    for (int c = 0; c < cols; ++c) s += std::exp(double(h2f(xr[c])) - double(mx));
    for (int c = 0; c < cols; ++c)
      y[size_t(r) * cols + c] = f2h(float(std::exp(double(h2f(xr[c])) - double(mx)) / s));
  }
}

// Restates reference kernels/src/cuda/tc/elementwise.cu:28-33.
void or_gelu_f16(const uint16_t* x, uint16_t* y, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) y[i] = f2h(gelu_tanh(h2f(x[i])));
}

// ---- LayerNorm / Softmax, fp32 ---------------------------------------------
// Double-precision ground truth, restating reference kernels/tests/reference.hpp:29-53.
void or_layernorm_f32_exact(const float* x, const float* g, const float* b, float* y, int rows,
                            int cols, float eps) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + size_t(r) * cols;
    double mean = 0, var = 0;
    for (int c = 0; c < cols; ++c) mean += xr[c];
    mean /= cols;
    for (int c = 0; c < cols; ++c) var += (xr[c] - mean) * (xr[c] - mean);
    var /= cols;
    for (int c = 0; c < cols; ++c)
      y[size_t(r) * cols + c] = float((xr[c] - mean) / std::sqrt(var + double(eps)) * g[c] + b[c]);
  }
}
void or_softmax_f32_exact(const float* x, float* y, int rows, int cols) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + size_t(r) * cols;
    double m = -INFINITY, s = 0;
    for (int c = 0; c < cols; ++c) m = std::fmax(m, double(xr[c]));
    for (int c = 0; c < cols; ++c) s += std::exp(double(xr[c]) - m);
    for (int c = 0; c < cols; ++c) y[size_t(r) * cols + c] = float(std::exp(double(xr[c]) - m) / s);
  }
}
// The reference CPU algorithms timed as the FP32 CPU baseline:
// reference kernels/src/cpu/layernorm.cpp:22-40 (shifted single pass) and
// kernels/src/cpu/softmax.cpp:19-36 (max pass, exp+sum pass, scale pass).
void or_layernorm_f32_fused(const float* x, const float* g, const float* b, float* y, int rows,
                            int cols, float eps) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const float* __restrict__ xr = x + size_t(r) * cols;
    float* __restrict__ yr = y + size_t(r) * cols;
    const float shift = xr[0];
    float s = 0.f, ss = 0.f;
#pragma omp simd reduction(+ : s, ss)
    for (int c = 0; c < cols; ++c) {
      const float d = xr[c] - shift;
      s += d;
      ss += d * d;
    }
    const float mean_d = s / cols, var = ss / cols - mean_d * mean_d, mean = shift + mean_d;
    const float rstd = 1.f / std::sqrt((var > 0.f ? var : 0.f) + eps);
#pragma omp simd
    for (int c = 0; c < cols; ++c) yr[c] = (xr[c] - mean) * rstd * g[c] + b[c];
  }
}
void or_softmax_f32_fused(const float* x, float* y, int rows, int cols) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const float* __restrict__ xr = x + size_t(r) * cols;
    float* __restrict__ yr = y + size_t(r) * cols;
    float m = -std::numeric_limits<float>::infinity();
#pragma omp simd reduction(max : m)
    for (int c = 0; c < cols; ++c) m = xr[c] > m ? xr[c] : m;
    float s = 0.f;
#pragma omp simd reduction(+ : s)
    for (int c = 0; c < cols; ++c) {
      const float e = std::exp(xr[c] - m);
      yr[c] = e;
      s += e;
    }
    const float inv = 1.f / s;
#pragma omp simd
    for (int c = 0; c < cols; ++c) yr[c] *= inv;
  }
}

// ---- Attention ----------------------------------------------------------------
// Restates reference kernels/src/cuda/tc/attention.cu:29-56 for one (b, h, query):
// keys j < kv_valid (and j <= offset + qi when causal) in increasing order;
// s = dot(q, k_j) * (1/sqrt(D)); online m, l, acc in fp32 with alpha = 0 while
// l == 0; out = fp16_rn(acc / l), or 0 when no key is visible or the query is
// padding.  Generic strides let the same routine read the packed [B,H,K,D]
// ABI layout and the runtime's slot cache.
namespace {
void attend_one(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out, int nkeys,
                int D) {
  const float scale = float(1.0 / std::sqrt(double(D)));
  float m = -INFINITY, l = 0.f;
  std::vector<float> acc(D, 0.f), qf(D);
  for (int d = 0; d < D; ++d) qf[d] = h2f(q[d]);
  for (int j = 0; j < nkeys; ++j) {
    float s = 0.f;
    for (int d = 0; d < D; ++d) s += qf[d] * h2f(k[size_t(j) * D + d]);
    s *= scale;
    const float nx = std::max(m, s);
    const float alpha = l == 0.f ? 0.f : std::exp(m - nx), beta = std::exp(s - nx);
    for (int d = 0; d < D; ++d) acc[d] = acc[d] * alpha + beta * h2f(v[size_t(j) * D + d]);
    l = l * alpha + beta;
    m = nx;
  }
  for (int d = 0; d < D; ++d) out[d] = f2h(l > 0.f ? acc[d] / l : 0.f);
}
}  // namespace

void or_attention_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* y,
                      const int32_t* ql, const int32_t* kl, const int32_t* off, int B, int H,
                      int Q, int K, int D, int causal) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      const int qv = std::max(0, std::min(Q, ql[b])), kv = std::max(0, std::min(K, kl[b]));
      const size_t qb = (size_t(b) * H + h) * Q * D, kb = (size_t(b) * H + h) * K * D;
      for (int i = 0; i < Q; ++i) {
        int nk = 0;
        if (i < qv) {
          const int64_t bound = causal ? int64_t(off[b]) + i + 1 : int64_t(kv);
          nk = int(std::max<int64_t>(0, std::min<int64_t>(bound, kv)));
        }
        attend_one(q + qb + size_t(i) * D, k + kb, v + kb, y + qb + size_t(i) * D, nk, D);
      }
    }
}

// ---- GPT-2 forward / greedy ---------------------------------------------------
// Restates reference llm/src/runtime.cu:25-66,135-168,190-203 (composition,
// rounding points, greedy loop) on the host.  Weights are host arrays in the
// artifact layout (Conv1D [in,out] orientation, tied transposed head).
struct or_gpt2_weights {
  int layers, heads, hidden, vocab, ctx;
  const uint16_t* wte;  // [vocab, hidden] fp16
  const uint16_t* wpe;  // [ctx, hidden] fp16
  const uint16_t* lnf_g;
  const uint16_t* lnf_b;
  const uint16_t* const* ln1_g;  // per layer [hidden]
  const uint16_t* const* ln1_b;
  const uint16_t* const* ln2_g;
  const uint16_t* const* ln2_b;
  const int8_t* const* w[4];      // c_attn [H,3H], attn c_proj [H,H], c_fc [H,4H], mlp c_proj [4H,H]
  const float* const* s[4];       // scales per output column
  const uint16_t* const* bias[4];
  const int8_t* head_q;  // [hidden, vocab]
  const float* head_s;   // [vocab]
  // fp16-precision artifacts (reference runtime.cu:97-113, ti_v2_gemm_ex_f16):
  // when w16[0] is set the linears and the head are fp16 [K,N] bits, used as
  // they are (no scales) in place of w/s/head_q/head_s.
  const uint16_t* const* w16[4];
  const uint16_t* head16;
};
}  // extern "C"

namespace {
struct Gpt2 {
  int L, NH, Hd, V, ctx, slots, cap;
  std::vector<uint16_t> wte, wpe, lnf_g, lnf_b;
  std::vector<std::vector<uint16_t>> ln1_g, ln1_b, ln2_g, ln2_b, bias[4];
  std::vector<std::vector<float>> w[4];  // dequantized fp16 values widened to fp32, [K,N]
  std::vector<float> head;               // [hidden, vocab]
  std::vector<uint16_t> kc, vc;          // [slot][layer][head][pos][64]
  std::vector<int> lengths;

  size_t cache_index(int slot, int layer, int h, int pos) const {
    return ((((size_t(slot) * L + layer) * NH + h) * cap + pos) * 64);
  }

  // fp32-accumulated linear over pre-dequantized weights; fp16 rounding of the
  // result as the reference's TI_V2_FP16 output (runtime.cu:143,148,150,152).
  // `active` lists the rows to compute (null: all); the others stay 0 (the
  // padding rows of a ragged prefill, which no real row reads).
  static void linear(const std::vector<float>& x, int rows, int K, const std::vector<float>& W,
                     int N, const uint16_t* bias, std::vector<float>& out, bool round16,
                     const std::vector<int>* active = nullptr) {
    out.assign(size_t(rows) * N, 0.f);
    std::vector<int> all;
    if (!active) {
      all.resize(rows);
      for (int r = 0; r < rows; ++r) all[r] = r;
      active = &all;
    }
    const int count = int(active->size());
    // Rows in blocks of 16 share each loaded weight row (a 128-column slice of W
    // is read once per 16 rows instead of once per row); every output still
    // sums k in increasing order, one fma per k.
    constexpr int RB = 16;
#pragma omp parallel for schedule(dynamic) collapse(2)
    for (int n0 = 0; n0 < N; n0 += 128) {
      for (int i0 = 0; i0 < count; i0 += RB) {
        const int n1 = std::min(N, n0 + 128), i1 = std::min(count, i0 + RB);
        for (int k = 0; k < K; ++k) {
          const float* wr = &W[size_t(k) * N];
          for (int i = i0; i < i1; ++i) {
            const int r = (*active)[i];
            const float av = x[size_t(r) * K + k];
            float* o = &out[size_t(r) * N];
#pragma omp simd
            for (int n = n0; n < n1; ++n) o[n] += av * wr[n];
          }
        }
        for (int i = i0; i < i1; ++i) {
          float* o = &out[size_t((*active)[i]) * N];
          for (int n = n0; n < n1; ++n) {
            const float v = o[n] + (bias ? h2f(bias[n]) : 0.f);
            o[n] = round16 ? rt16(v) : v;
          }
        }
      }
    }
  }

  // x = fp16_rn(x + proj), elementwise.
  static void residual(std::vector<float>& x, const std::vector<float>& proj) {
    const int64_t n = int64_t(x.size());
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) x[i] = rt16(x[i] + proj[i]);
  }

  void layernorm(const std::vector<float>& x, int rows, const std::vector<uint16_t>& g,
                 const std::vector<uint16_t>& b, std::vector<float>& y) const {
    std::vector<uint16_t> xin(x.size()), yo(x.size());
    const int64_t n = int64_t(x.size());
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) xin[i] = f2h(x[i]);
    or_layernorm_f16(xin.data(), g.data(), b.data(), yo.data(), rows, Hd, 1e-5f);
    y.resize(x.size());
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) y[i] = h2f(yo[i]);
  }

  // One forward over rows [b, qlen] of new tokens; returns the fp16 ln_f output of
  // every row (values held as float).  Mirrors transform(), runtime.cu:135-156.
  void transform(const std::vector<int>& slot, const std::vector<int>& tokens,
                 const std::vector<int>& lens, int B, int Q, std::vector<float>& xout) {
    const int rows = B * Q, H3 = 3 * Hd, H4 = 4 * Hd;
    std::vector<float> x(size_t(rows) * Hd, 0.f), norm, qkv, attn(size_t(rows) * Hd, 0.f), proj, mlp;
    std::vector<int> offs(B), real;
    for (int b = 0; b < B; ++b) offs[b] = lengths[slot[b]];
    for (int b = 0; b < B; ++b)
      for (int t = 0; t < lens[b]; ++t) real.push_back(b * Q + t);
    for (int b = 0; b < B; ++b)  // embed: fp16(wte[id] + wpe[off + t]), padded rows 0 (:25-30)
      for (int t = 0; t < lens[b]; ++t) {
        const int id = tokens[size_t(b) * Q + t], pos = offs[b] + t;
        for (int c = 0; c < Hd; ++c)
          x[(size_t(b) * Q + t) * Hd + c] = rt16(h2f(wte[size_t(id) * Hd + c]) + h2f(wpe[size_t(pos) * Hd + c]));
      }
    for (int l = 0; l < L; ++l) {
      layernorm(x, rows, ln1_g[l], ln1_b[l], norm);
      linear(norm, rows, Hd, w[0][l], H3, bias[0][l].data(), qkv, true, &real);
      // split_scatter (:34-42): q | k | v thirds, head h at columns h*64..h*64+63
      for (int b = 0; b < B; ++b)
        for (int t = 0; t < lens[b]; ++t)
          for (int h = 0; h < NH; ++h)
            for (int d = 0; d < 64; ++d) {
              const size_t src = (size_t(b) * Q + t) * H3 + h * 64 + d;
              const size_t dst = cache_index(slot[b], l, h, offs[b] + t) + d;
              kc[dst] = f2h(qkv[src + Hd]);
              vc[dst] = f2h(qkv[src + 2 * Hd]);
            }
      // attention over the slot cache (:146-147), causal with offset = old length
      std::fill(attn.begin(), attn.end(), 0.f);
#pragma omp parallel for collapse(2) schedule(static)
      for (int b = 0; b < B; ++b)
        for (int h = 0; h < NH; ++h) {
          std::vector<uint16_t> qh(64), oh(64);
          for (int t = 0; t < lens[b]; ++t) {
            for (int d = 0; d < 64; ++d) qh[d] = f2h(qkv[(size_t(b) * Q + t) * H3 + h * 64 + d]);
            const int nk = offs[b] + t + 1;
            attend_one(qh.data(), &kc[cache_index(slot[b], l, h, 0)], &vc[cache_index(slot[b], l, h, 0)],
                       oh.data(), nk, 64);
            for (int d = 0; d < 64; ++d) attn[(size_t(b) * Q + t) * Hd + h * 64 + d] = h2f(oh[d]);
          }
        }
      linear(attn, rows, Hd, w[1][l], Hd, bias[1][l].data(), proj, true, &real);
      residual(x, proj);  // res = x + proj (:149)
      layernorm(x, rows, ln2_g[l], ln2_b[l], norm);
      linear(norm, rows, Hd, w[2][l], H4, bias[2][l].data(), mlp, true, &real);
      {  // gelu_new over the fp16 c_fc output (:151)
        const int64_t n = int64_t(mlp.size());
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < n; ++i) mlp[i] = rt16(gelu_tanh(mlp[i]));
      }
      linear(mlp, rows, H4, w[3][l], Hd, bias[3][l].data(), proj, true, &real);
      residual(x, proj);  // x = res + proj (:153)
    }
    layernorm(x, rows, lnf_g, lnf_b, xout);  // ln_f (:155)
  }

  // forward(): runtime.cu:157-168 — last_rows, fp32 lm_head without bias, argmax
  // with the lowest id on ties; lengths advance afterwards.
  void forward(const int* s, const int* tok, const int* lens, int B, int stride, float* logits,
               int* next) {
    int Q = 0;
    for (int b = 0; b < B; ++b) Q = std::max(Q, lens[b]);
    std::vector<int> slot(s, s + B), ll(lens, lens + B), dense(size_t(B) * Q, 0);
    for (int b = 0; b < B; ++b)
      for (int t = 0; t < lens[b]; ++t) dense[size_t(b) * Q + t] = tok[size_t(b) * stride + t];
    std::vector<float> xo;
    transform(slot, dense, ll, B, Q, xo);
    if (logits || next) {
      std::vector<float> last(size_t(B) * Hd), lg;
      for (int b = 0; b < B; ++b)
        std::copy(&xo[(size_t(b) * Q + lens[b] - 1) * Hd], &xo[(size_t(b) * Q + lens[b]) * Hd], &last[size_t(b) * Hd]);
      linear(last, B, Hd, head, V, nullptr, lg, false);
      if (logits) std::copy(lg.begin(), lg.end(), logits);
      if (next)
        for (int b = 0; b < B; ++b) {
          int best = 0;
          for (int j = 1; j < V; ++j)
            if (lg[size_t(b) * V + j] > lg[size_t(b) * V + best]) best = j;
          next[b] = best;
        }
    }
    for (int b = 0; b < B; ++b) lengths[s[b]] += lens[b];
  }
};

std::vector<uint16_t> copy16(const uint16_t* p, size_t n) { return std::vector<uint16_t>(p, p + n); }
std::vector<float> widen16(const uint16_t* w, size_t n) {
  std::vector<float> out(n);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < int64_t(n); ++i) out[i] = h2f(w[i]);
  return out;
}
std::vector<float> dequant_f32(const int8_t* q, const float* s, int K, int N) {
  std::vector<float> out(size_t(K) * N);
#pragma omp parallel for schedule(static)
  for (int k = 0; k < K; ++k)
    for (int n = 0; n < N; ++n) out[size_t(k) * N + n] = rt16(float(q[size_t(k) * N + n]) * s[n]);
  return out;
}
}  // namespace

extern "C" {
void* or_gpt2_create(const or_gpt2_weights* w, int slots, int capacity) {
  auto m = std::make_unique<Gpt2>();
  m->L = w->layers; m->NH = w->heads; m->Hd = w->hidden; m->V = w->vocab; m->ctx = w->ctx;
  m->slots = slots; m->cap = capacity;
  const int H = w->hidden;
  m->wte = copy16(w->wte, size_t(w->vocab) * H);
  m->wpe = copy16(w->wpe, size_t(w->ctx) * H);
  m->lnf_g = copy16(w->lnf_g, H);
  m->lnf_b = copy16(w->lnf_b, H);
  const int KN[4][2] = {{H, 3 * H}, {H, H}, {H, 4 * H}, {4 * H, H}};
  for (int l = 0; l < w->layers; ++l) {
    m->ln1_g.push_back(copy16(w->ln1_g[l], H)); m->ln1_b.push_back(copy16(w->ln1_b[l], H));
    m->ln2_g.push_back(copy16(w->ln2_g[l], H)); m->ln2_b.push_back(copy16(w->ln2_b[l], H));
    for (int i = 0; i < 4; ++i) {
      m->w[i].push_back(w->w16[0] ? widen16(w->w16[i][l], size_t(KN[i][0]) * KN[i][1])
                                  : dequant_f32(w->w[i][l], w->s[i][l], KN[i][0], KN[i][1]));
      m->bias[i].push_back(copy16(w->bias[i][l], KN[i][1]));
    }
  }
  m->head = w->w16[0] ? widen16(w->head16, size_t(H) * w->vocab) : dequant_f32(w->head_q, w->head_s, H, w->vocab);
  const size_t cache = size_t(slots) * w->layers * w->heads * capacity * 64;
  m->kc.assign(cache, 0);
  m->vc.assign(cache, 0);
  m->lengths.assign(slots, 0);
  return m.release();
}
void or_gpt2_destroy(void* p) { delete static_cast<Gpt2*>(p); }
void or_gpt2_reset(void* p, int slot) { static_cast<Gpt2*>(p)->lengths[slot] = 0; }
int or_gpt2_length(void* p, int slot) { return static_cast<Gpt2*>(p)->lengths[slot]; }
void or_gpt2_forward(void* p, const int* slots, const int* tokens, const int* lens, int B, int stride,
                     float* logits, int* next) {
  static_cast<Gpt2*>(p)->forward(slots, tokens, lens, B, stride, logits, next);
}
// Greedy loop of reference runtime.cu:190-203: the prefill returns token 1, then
// one single-token forward per step for still-active requests; the final
// generated token is not appended.  output[B, out_stride].
void or_gpt2_greedy(void* p, const int* slots, const int* prompts, const int* plens,
                    const int* requested, int B, int stride, int* output, int out_stride) {
  auto* m = static_cast<Gpt2*>(p);
  std::vector<int> next(B), done(B, 1);
  std::fill(output, output + size_t(B) * out_stride, -1);
  m->forward(slots, prompts, plens, B, stride, nullptr, next.data());
  for (int b = 0; b < B; ++b) output[size_t(b) * out_stride] = next[b];
  for (;;) {
    std::vector<int> act, ids, ones, owner;
    for (int b = 0; b < B; ++b)
      if (done[b] < requested[b]) { act.push_back(slots[b]); ids.push_back(next[b]); ones.push_back(1); owner.push_back(b); }
    if (act.empty()) break;
    std::vector<int> gen(act.size());
    m->forward(act.data(), ids.data(), ones.data(), int(act.size()), 1, nullptr, gen.data());
    for (size_t j = 0; j < owner.size(); ++j) {
      const int b = owner[j];
      next[b] = gen[j];
      output[size_t(b) * out_stride + done[b]] = next[b];
      ++done[b];
    }
  }
}
int or_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
}  // extern "C"
