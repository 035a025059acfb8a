// W8A16 / FP16-weight linear layers for gfx950.
//
// Two kernels cover the M range of GPT-2 inference:
//  * skinny (M <= 32, decode): every wave streams weight fragments straight from
//    HBM into MFMA B-operand registers (no LDS for weights), dequantises them in
//    registers as fp16_rn(float(q) * scale[n]) and runs v_mfma_f32_16x16x32_f16
//    with A padded to 16/32 rows.  A lane loads one dword (4 consecutive output
//    columns) from 8 consecutive K rows, so the MFMA for "column slot" c covers
//    columns {n0 + 4j + c}; the 4 waves of a workgroup split K, reduce through
//    LDS, and workgroups split K further: each writes fp32 partials and a
//    second kernel sums them in split order and runs the fused epilogue (bias /
//    GELU / residual / KV scatter).  (A single-kernel last-arrival reduction
//    needs agent-scope release/acquire fences, which on the multi-XCD part
//    write back and invalidate the whole L2 in every workgroup.)
//  * tiled (M > 32, prefill): 64x64x32 tiles, A and the dequantised weight tile
//    staged in LDS (weights transposed to [n][k] so both MFMA operands are one
//    ds_read_b128 per lane), double buffered, same fused epilogues.
// Dequantisation mirrors reference kernels/src/cuda/tc/gemm.cu:21,24 and the
// bias epilogue mirrors gemm.cu:73-80 / :118-124; accumulation is fp32.
#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

#include "common.hpp"
#include "kernels.hpp"

namespace tia {
namespace {

__device__ __forceinline__ void apply_epilogue(const Epilogue& e, int m, int n, float acc) {
  switch (e.kind) {
    case EPI_RAW_F32:
      static_cast<float*>(e.y)[int64_t(m) * e.ldy + n] = acc;
      return;
    case EPI_F32:
      static_cast<float*>(e.y)[int64_t(m) * e.ldy + n] = acc + (e.bias ? h2f(e.bias[n]) : 0.f);
      return;
    case EPI_GELU: {
      const float h = rt16(acc + (e.bias ? h2f(e.bias[n]) : 0.f));
      static_cast<uint16_t*>(e.y)[int64_t(m) * e.ldy + n] = f2h(gelu_tanh(h));
      return;
    }
    case EPI_RESIDUAL: {
      const float h = rt16(acc + (e.bias ? h2f(e.bias[n]) : 0.f));
      const float r = h2f(e.residual[int64_t(m) * e.ldr + n]);
      static_cast<uint16_t*>(e.y)[int64_t(m) * e.ldy + n] = f2h(r + h);
      return;
    }
    case EPI_QKV: {
      const uint16_t hv = f2h(acc + (e.bias ? h2f(e.bias[n]) : 0.f));
      static_cast<uint16_t*>(e.y)[int64_t(m) * e.ldy + n] = hv;
      if (n >= e.hidden) {
        const int b = m / e.qrows, t = m - b * e.qrows;
        if (t < e.qlens[b]) {
          const int part = n >= 2 * e.hidden ? 2 : 1;
          const int c = n - part * e.hidden, h = c >> 6, d = c & 63;
          const int64_t pos = int64_t(e.offsets[b]) + t;
          const int64_t idx =
              (((int64_t(e.slots[b]) * e.layers + e.layer) * e.heads + h) * e.capacity + pos) * 64 + d;
          (part == 1 ? e.kcache : e.vcache)[idx] = hv;
        }
      }
      return;
    }
    default:  // EPI_F16
      static_cast<uint16_t*>(e.y)[int64_t(m) * e.ldy + n] = f2h(acc + (e.bias ? h2f(e.bias[n]) : 0.f));
      return;
  }
}

// ---------------------------------------------------------------------------
// Skinny kernel
// ---------------------------------------------------------------------------
struct SkinnyParams {
  const uint16_t* a;
  int64_t lda;
  const void* w;
  const float* scales;
  int m, n, k;
  int64_t ldw;         // row stride of W in elements (>= n)
  int ntile;           // ceil(N / 64)
  int steps;           // ceil(K / 32)
  int steps_per_block; // K steps owned by one workgroup (its waves take every 4th)
  int splits;
  bool defer;          // always leave fp32 partials (even for one split), no epilogue
  Epilogue epi;
  float* partials;     // [splits][M][N]
};

constexpr int kSkinnyThreads = 256;

// Weight fragment of one lane for one 32-row K step: rows k0 + 8g + r (r = 0..7),
// columns col..col+3.  int8: one dword per row; fp16: two dwords per row.
template <bool INT8>
struct WFrag {
  uint32_t d[INT8 ? 8 : 16];
};

template <bool INT8, bool WVEC>
__device__ __forceinline__ void load_wfrag(WFrag<INT8>& f, const void* w, int K, int N, int64_t LDW, int krow,
                                           int col) {
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int k = krow + r;
    if constexpr (INT8) {
      const int8_t* p = static_cast<const int8_t*>(w);
      uint32_t v = 0;
      if (k < K) {
        if constexpr (WVEC) {
          if (col < N) v = *reinterpret_cast<const uint32_t*>(p + int64_t(k) * LDW + col);
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (col + c < N) v |= uint32_t(uint8_t(p[int64_t(k) * LDW + col + c])) << (8 * c);
        }
      }
      f.d[r] = v;
    } else {
      const uint16_t* p = static_cast<const uint16_t*>(w);
      uint32_t v0 = 0, v1 = 0;
      if (k < K) {
        if constexpr (WVEC) {
          if (col < N) {
            const uint2 u = *reinterpret_cast<const uint2*>(p + int64_t(k) * LDW + col);
            v0 = u.x;
            v1 = u.y;
          }
        } else {
          uint16_t h[4] = {0, 0, 0, 0};
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (col + c < N) h[c] = p[int64_t(k) * LDW + col + c];
          v0 = uint32_t(h[0]) | (uint32_t(h[1]) << 16);
          v1 = uint32_t(h[2]) | (uint32_t(h[3]) << 16);
        }
      }
      f.d[2 * r] = v0;
      f.d[2 * r + 1] = v1;
    }
  }
}

// B operand of MFMA column slot c: the 8 K values of column col + c.
template <bool INT8>
__device__ __forceinline__ half8_t bfrag(const WFrag<INT8>& f, int c, float scale) {
  half8_t out;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    if constexpr (INT8) {
      const int8_t q = int8_t(f.d[r] >> (8 * c));
      out[r] = f16(float(q) * scale);  // fp16_rn(float(q) * scale[n])
    } else {
      const uint32_t word = f.d[2 * r + (c >> 1)];
      out[r] = __builtin_bit_cast(f16, uint16_t(word >> (16 * (c & 1))));
    }
  }
  return out;
}

template <bool AVEC>
__device__ __forceinline__ half8_t afrag(const uint16_t* a, int64_t lda, int M, int K, int m,
                                         int kk) {
  half8_t out;
  if constexpr (AVEC) {
    if (m < M && kk < K) return *reinterpret_cast<const half8_t*>(a + int64_t(m) * lda + kk);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = f16(0.f);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      out[i] = (m < M && kk + i < K) ? __builtin_bit_cast(f16, a[int64_t(m) * lda + kk + i]) : f16(0.f);
  }
  return out;
}

template <bool INT8, int MT, bool WVEC, bool AVEC>
__global__ __launch_bounds__(kSkinnyThreads) void skinny_kernel(SkinnyParams p) {
  __shared__ float red[4][MT * 16][65];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;

  // Blocks are dispatched round-robin over the 8 XCDs; hand each XCD a
  // contiguous range of (tile, split) work so column tiles that share 128-byte
  // weight lines are read through the same L2.
  const int nb = gridDim.x, bid = blockIdx.x;
  const int logical = (nb % 8 == 0) ? (bid % 8) * (nb / 8) + bid / 8 : bid;
  const int tile = logical % p.ntile, split = logical / p.ntile;
  const int n0 = tile * 64, col = n0 + 4 * j;

  float sc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) sc[c] = (INT8 && col + c < p.n) ? p.scales[col + c] : 0.f;

  float4_t acc[MT][4];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[t][c] = float4_t{0.f, 0.f, 0.f, 0.f};

  const int s_begin = split * p.steps_per_block;
  const int s_end = min(p.steps, s_begin + p.steps_per_block);
  // Each wave takes every 4th step; two steps are loaded before either is used.
  for (int st = s_begin + wave; st < s_end; st += 8) {
    WFrag<INT8> f0, f1;
    const int k0 = st * 32, k1 = (st + 4) * 32;
    const bool has1 = st + 4 < s_end;
    load_wfrag<INT8, WVEC>(f0, p.w, p.k, p.n, p.ldw, k0 + 8 * g, col);
    if (has1) load_wfrag<INT8, WVEC>(f1, p.w, p.k, p.n, p.ldw, k1 + 8 * g, col);
    half8_t a0[MT], a1[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) a0[t] = afrag<AVEC>(p.a, p.lda, p.m, p.k, 16 * t + j, k0 + 8 * g);
    if (has1) {
#pragma unroll
      for (int t = 0; t < MT; ++t) a1[t] = afrag<AVEC>(p.a, p.lda, p.m, p.k, 16 * t + j, k1 + 8 * g);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const half8_t b = bfrag<INT8>(f0, c, sc[c]);
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[t][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0[t], b, acc[t][c], 0, 0, 0);
    }
    if (has1) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const half8_t b = bfrag<INT8>(f1, c, sc[c]);
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1[t], b, acc[t][c], 0, 0, 0);
      }
    }
  }

  // MFMA output: lane holds rows 4g + v (v = 0..3) of column j of each 16x16 block.
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[wave][16 * t + 4 * g + v][4 * j + c] = acc[t][c][v];
  __syncthreads();

  constexpr int kElems = MT * 16 * 64;
  for (int e = threadIdx.x; e < kElems; e += kSkinnyThreads) {
    const int row = e >> 6, cc = e & 63, n = n0 + cc;
    if (row < p.m && n < p.n) {
      const float s = red[0][row][cc] + red[1][row][cc] + red[2][row][cc] + red[3][row][cc];
      if (p.splits == 1 && !p.defer) apply_epilogue(p.epi, row, n, s);
      else p.partials[(int64_t(split) * p.m + row) * p.n + n] = s;
    }
  }
}

// Second pass of a split-K launch: C[m][n] = sum of the split partials in split
// order, then the epilogue.  The kernel boundary orders it after every partial.
// Each workgroup covers 64 consecutive outputs with 4 waves; wave w sums splits
// w, w + 4, ... so all splits of an output are in flight at once, and wave 0
// adds the four group sums in a fixed order.
__global__ __launch_bounds__(256) void splitk_epilogue_kernel(const float* partials, int splits, int m,
                                                              int n, Epilogue epi) {
  __shared__ float red[4][64];
  const int lane = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int64_t total = int64_t(m) * n;
  for (int64_t base = int64_t(blockIdx.x) * 64; base < total; base += int64_t(gridDim.x) * 64) {
    const int64_t i = base + lane;
    float s = 0.f;
    if (i < total) {
#pragma unroll 4
      for (int sp = grp; sp < splits; sp += 4) s += partials[i + sp * total];
    }
    red[grp][lane] = s;
    __syncthreads();
    if (grp == 0 && i < total) {
      const int row = int(i / n), col = int(i - int64_t(row) * n);
      apply_epilogue(epi, row, col, ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane]);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Tiled kernel (M > 32)
// ---------------------------------------------------------------------------
struct TiledParams {
  const uint16_t* a;
  int64_t lda;
  const void* w;
  const float* scales;
  int m, n, k;
  int64_t ldw;
  Epilogue epi;
};
constexpr int TBM = 64, TBN = 64, TBK = 32, TPAD = 40;  // LDS row pitch in halves

template <bool INT8, bool WVEC, bool AVEC>
__global__ __launch_bounds__(256) void tiled_kernel(TiledParams p) {
  __shared__ __attribute__((aligned(16))) f16 As[2][TBM][TPAD];
  __shared__ __attribute__((aligned(16))) f16 Bs[2][TBN][TPAD];  // transposed: [n][k]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * TBM, n0 = blockIdx.x * TBN;

  // A staging: thread -> row tid/4, k segment (tid%4)*8.
  const int a_row = tid >> 2, a_kseg = (tid & 3) * 8;
  // W staging: thread -> columns c4..c4+3, K rows kr, kr+1.
  const int w_c4 = (tid & 15) * 4, w_kr = (tid >> 4) * 2;
  float sc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) sc[c] = (INT8 && n0 + w_c4 + c < p.n) ? p.scales[n0 + w_c4 + c] : 0.f;

  half8_t areg;
  f16 wreg[2][4];

  auto load_global = [&](int k0) {
    areg = afrag<AVEC>(p.a, p.lda, p.m, p.k, m0 + a_row, k0 + a_kseg);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int k = k0 + w_kr + r, col = n0 + w_c4;
      if constexpr (INT8) {
        const int8_t* wp = static_cast<const int8_t*>(p.w);
        int8_t q[4] = {0, 0, 0, 0};
        if (k < p.k) {
          if (WVEC && col < p.n) {
            const uint32_t v = *reinterpret_cast<const uint32_t*>(wp + int64_t(k) * p.ldw + col);
#pragma unroll
            for (int c = 0; c < 4; ++c) q[c] = int8_t(v >> (8 * c));
          } else if (!WVEC) {
#pragma unroll
            for (int c = 0; c < 4; ++c)
              if (col + c < p.n) q[c] = wp[int64_t(k) * p.ldw + col + c];
          }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) wreg[r][c] = f16(float(q[c]) * sc[c]);
      } else {
        const uint16_t* wp = static_cast<const uint16_t*>(p.w);
        uint16_t h[4] = {0, 0, 0, 0};
        if (k < p.k) {
          if (WVEC && col < p.n) {
            const uint2 u = *reinterpret_cast<const uint2*>(wp + int64_t(k) * p.ldw + col);
            h[0] = uint16_t(u.x); h[1] = uint16_t(u.x >> 16); h[2] = uint16_t(u.y); h[3] = uint16_t(u.y >> 16);
          } else if (!WVEC) {
#pragma unroll
            for (int c = 0; c < 4; ++c)
              if (col + c < p.n) h[c] = wp[int64_t(k) * p.ldw + col + c];
          }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) wreg[r][c] = __builtin_bit_cast(f16, h[c]);
      }
    }
  };
  auto store_lds = [&](int s) {
    *reinterpret_cast<half8_t*>(&As[s][a_row][a_kseg]) = areg;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      half2_t pair;
      pair[0] = wreg[0][c];
      pair[1] = wreg[1][c];
      *reinterpret_cast<half2_t*>(&Bs[s][w_c4 + c][w_kr]) = pair;
    }
  };

  float4_t acc[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int c = 0; c < 2; ++c) acc[t][c] = float4_t{0.f, 0.f, 0.f, 0.f};

  const int steps = (p.k + TBK - 1) / TBK;
  load_global(0);
  store_lds(0);
  __syncthreads();
  for (int st = 0; st < steps; ++st) {
    const int cur = st & 1;
    if (st + 1 < steps) load_global((st + 1) * TBK);
    half8_t af[2], bf[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) af[t] = *reinterpret_cast<const half8_t*>(&As[cur][wm * 32 + 16 * t + j][8 * g]);
#pragma unroll
    for (int c = 0; c < 2; ++c) bf[c] = *reinterpret_cast<const half8_t*>(&Bs[cur][wn * 32 + 16 * c + j][8 * g]);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int c = 0; c < 2; ++c) acc[t][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t], bf[c], acc[t][c], 0, 0, 0);
    if (st + 1 < steps) {
      store_lds(cur ^ 1);
      __syncthreads();
    }
  }
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + wm * 32 + 16 * t + 4 * g + v, n = n0 + wn * 32 + 16 * c + j;
        if (m < p.m && n < p.n) apply_epilogue(p.epi, m, n, acc[t][c][v]);
      }
}

// ---------------------------------------------------------------------------
// Separate bias epilogue and the legacy FP32 GEMM
// ---------------------------------------------------------------------------
__global__ void bias_epilogue_kernel(const float* ws, const uint16_t* bias, void* y, int64_t count,
                                     int n, int dtype) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
       i += int64_t(gridDim.x) * blockDim.x) {
    const float v = ws[i] + (bias ? h2f(bias[i % n]) : 0.f);
    if (dtype == 1) static_cast<float*>(y)[i] = v;
    else static_cast<uint16_t*>(y)[i] = f2h(v);
  }
}

// 64x64 output tile per 256-thread block, 4x4 outputs per thread, K in 16-wide
// LDS slabs.
__global__ __launch_bounds__(256) void legacy_f32_kernel(const float* a, const float* b, float* c,
                                                         int m, int n, int k) {
  __shared__ float As[16][64 + 4];
  __shared__ float Bs[16][64 + 4];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int row0 = blockIdx.y * 64, col0 = blockIdx.x * 64;
  float acc[4][4] = {};
  for (int64_t k0 = 0; k0 < k; k0 += 16) {
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const int i = tid + l * 256;
      const int ar = i >> 4, ak = i & 15;  // A tile 64 x 16
      const int64_t gr = row0 + ar, gk = k0 + ak;
      As[ak][ar] = (gr < m && gk < k) ? a[gr * k + gk] : 0.f;
      const int bk = i >> 6, bc = i & 63;  // B tile 16 x 64
      const int64_t gk2 = k0 + bk, gc = col0 + bc;
      Bs[bk][bc] = (gk2 < k && gc < n) ? b[gk2 * n + gc] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      float av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) bv[jj] = Bs[kk][tx * 4 + jj];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) acc[i][jj] += av[i] * bv[jj];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int64_t r = row0 + ty * 4 + i, cc = col0 + tx * 4 + jj;
      if (r < m && cc < n) c[r * n + cc] = acc[i][jj];
    }
}

// ---------------------------------------------------------------------------
// Host-side dispatch
// ---------------------------------------------------------------------------
template <bool INT8, int MT>
hipError_t launch_skinny(const GemmArgs& g, bool wvec, bool avec, const Scratch* s,
                         hipStream_t stream, int* deferred) {
  SkinnyParams p{};
  p.a = g.a; p.lda = g.lda; p.w = g.w; p.scales = g.scales;
  p.m = g.m; p.n = g.n; p.k = g.k; p.epi = g.epi;
  p.ldw = g.ldw > 0 ? g.ldw : g.n;
  p.ntile = (g.n + 63) / 64;
  p.steps = (g.k + 31) / 32;
  // Number of K splits: aim for ~2 workgroups per CU (a 2.4 MB GEMV is
  // latency-bound, so every CU should have loads in flight), with the fp32
  // partials (splits * M * N * 4 bytes, L2/MALL traffic) at most twice the
  // weight bytes and within the scratch.
  int splits = 1;
  if (s && s->partials) {
    const int target = (2 * 256 + p.ntile - 1) / p.ntile;
    const int max_by_traffic = std::max(1, g.k / (2 * std::max(1, g.m)));
    splits = std::max(1, std::min(target, std::min(p.steps, max_by_traffic)));
    while (splits > 1 && size_t(splits) * g.m * g.n > s->partial_floats) --splits;
  }
  const int spb = (p.steps + splits - 1) / splits;
  splits = (p.steps + spb - 1) / spb;
  p.steps_per_block = spb;
  p.splits = splits;
  p.defer = deferred != nullptr;
  p.partials = s ? s->partials : nullptr;
  if (p.defer && (!p.partials || size_t(splits) * g.m * g.n > s->partial_floats)) return hipErrorInvalidValue;
  const dim3 grid(unsigned(p.ntile) * unsigned(splits));
#define TIA_SKINNY(WV, AV) hipLaunchKernelGGL((skinny_kernel<INT8, MT, WV, AV>), grid, dim3(kSkinnyThreads), 0, stream, p)
  if (wvec && avec) TIA_SKINNY(true, true);
  else if (wvec) TIA_SKINNY(true, false);
  else if (avec) TIA_SKINNY(false, true);
  else TIA_SKINNY(false, false);
#undef TIA_SKINNY
  if (p.defer) {
    *deferred = splits;
    return hipGetLastError();
  }
  if (splits > 1) {
    const int64_t total = int64_t(g.m) * g.n;
    const unsigned blocks = unsigned(std::min<int64_t>((total + 63) / 64, 8192));
    hipLaunchKernelGGL(splitk_epilogue_kernel, dim3(blocks), dim3(256), 0, stream, p.partials, splits, g.m,
                       g.n, g.epi);
  }
  return hipGetLastError();
}

template <bool INT8>
hipError_t launch_tiled(const GemmArgs& g, bool wvec, bool avec, hipStream_t stream) {
  TiledParams p{};
  p.a = g.a; p.lda = g.lda; p.w = g.w; p.scales = g.scales;
  p.m = g.m; p.n = g.n; p.k = g.k; p.epi = g.epi;
  p.ldw = g.ldw > 0 ? g.ldw : g.n;
  const dim3 grid(unsigned((g.n + TBN - 1) / TBN), unsigned((g.m + TBM - 1) / TBM));
#define TIA_TILED(WV, AV) hipLaunchKernelGGL((tiled_kernel<INT8, WV, AV>), grid, dim3(256), 0, stream, p)
  if (wvec && avec) TIA_TILED(true, true);
  else if (wvec) TIA_TILED(true, false);
  else if (avec) TIA_TILED(false, true);
  else TIA_TILED(false, false);
#undef TIA_TILED
  return hipGetLastError();
}

}  // namespace

hipError_t gemm(const GemmArgs& g, const Scratch* s, hipStream_t stream, int* deferred) {
  if (deferred) *deferred = 0;
  if (g.m <= 0 || g.n <= 0 || g.k <= 0) return hipErrorInvalidValue;
  const uintptr_t wp = reinterpret_cast<uintptr_t>(g.w), ap = reinterpret_cast<uintptr_t>(g.a);
  // Whole 4-column groups may be loaded when rows are 4-aligned and the row
  // pitch covers n rounded up to 4 (columns past n are padding, never stored).
  const int64_t ldw = g.ldw > 0 ? g.ldw : g.n;
  const bool wvec = ldw % 4 == 0 && ldw >= (int64_t(g.n) + 3) / 4 * 4 &&
                    (g.w_int8 ? wp % 4 == 0 : wp % 8 == 0);
  const bool avec = (g.lda % 8 == 0) && (ap % 16 == 0);
  if (g.m <= 16) return g.w_int8 ? launch_skinny<true, 1>(g, wvec, avec, s, stream, deferred)
                                 : launch_skinny<false, 1>(g, wvec, avec, s, stream, deferred);
  if (g.m <= 32) return g.w_int8 ? launch_skinny<true, 2>(g, wvec, avec, s, stream, deferred)
                                 : launch_skinny<false, 2>(g, wvec, avec, s, stream, deferred);
  return g.w_int8 ? launch_tiled<true>(g, wvec, avec, stream) : launch_tiled<false>(g, wvec, avec, stream);
}

const Scratch* library_scratch(int device, hipStream_t stream, hipError_t* err) {
  static std::mutex mu;
  static std::map<std::pair<int, hipStream_t>, Scratch> table;
  std::lock_guard<std::mutex> lock(mu);
  auto it = table.find({device, stream});
  if (it != table.end()) return &it->second;
  Scratch s;
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &capture) == hipSuccess && capture != hipStreamCaptureStatusNone) {
    // Allocation is not allowed under capture: the stream must run one call eagerly first.
    *err = hipErrorStreamCaptureUnsupported;
    return nullptr;
  }
  const hipError_t e = hipMalloc(&s.partials, kScratchPartialFloats * sizeof(float));
  if (e != hipSuccess) {
    *err = e;
    return nullptr;
  }
  s.partial_floats = kScratchPartialFloats;
  return &(table[{device, stream}] = s);
}

hipError_t bias_epilogue(const float* ws, const uint16_t* bias, void* y, int64_t count, int n,
                         int dtype, hipStream_t stream) {
  const int64_t blocks = std::min<int64_t>((count + 255) / 256, 65535);
  hipLaunchKernelGGL(bias_epilogue_kernel, dim3(unsigned(blocks)), dim3(256), 0, stream, ws, bias, y,
                     count, n, dtype);
  return hipGetLastError();
}

hipError_t legacy_gemm_f32(const float* a, const float* b, float* c, int m, int n, int k,
                           hipStream_t stream) {
  hipLaunchKernelGGL(legacy_f32_kernel, dim3(unsigned((n + 63) / 64), unsigned((m + 63) / 64)),
                     dim3(256), 0, stream, a, b, c, m, n, k);
  return hipGetLastError();
}

}  // namespace tia
