// W8A16 / FP16-weight linear layers for gfx950.
//
// Three kernels cover the M range of GPT-2 inference:
//  * packed GEMV (M <= 32, int8 weights in the panel layout the runtime builds
//    at load): a wave load is one contiguous KiB that is already two MFMA
//    B operands per lane, so weights go HBM -> VGPR with 16-byte loads; all
//    loads of a wave are in flight before its first wait, the waves of a
//    workgroup split K and reduce through LDS, and the epilogue runs in the
//    same kernel (K is split across workgroups only when the caller finishes
//    the partials itself).  A single row (M = 1) over at most 2048 columns
//    takes the part-block kernel instead when the caller does not batch rows
//    (standalone GEMV calls): no MFMA, 8 columns per workgroup, twice the
//    workgroups of the 16-column MFMA blocks.
//  * row GEMV / GEMM (M <= 1024, row-major weights of the C ABIs, aligned
//    operands): about 192 workgroups, each one 64-column tile of 16 (M <= 64)
//    or 32 rows over a range of 32-row K steps, every load of a wave's round
//    in flight at once, the skinny kernel's fragments and MFMAs; K splits
//    finish in the launch through the queue pool (rowgemv_kernel at M <= 16,
//    rowgemm_kernel above).
//  * skinny (M <= 32, row-major weights, where the row GEMV does not apply:
//    unaligned operands, no queue pool): every wave streams weight fragments straight from
//    HBM into MFMA B-operand registers (no LDS for weights), dequantises them in
//    registers as fp16_rn(float(q) * scale[n]) and runs v_mfma_f32_16x16x32_f16
//    with A padded to 16/32 rows.  A lane loads one dword (4 consecutive output
//    columns) from 8 consecutive K rows, so the MFMA for "column slot" c covers
//    columns {n0 + 4j + c}; the 4 waves of a workgroup split K, reduce through
//    LDS, and workgroups split K further: each writes fp32 partials, which
//    are summed in split order and finished with the fused epilogue (bias /
//    GELU / residual / KV scatter) either by a second kernel (callers that own
//    a scratch buffer: the runtime) or, for the C ABIs, by the last workgroup
//    of the tile in the same launch (partials in the queue's slot of a static
//    pool, written and read with agent-scope accesses, so no L2-wide
//    writeback or invalidate is needed; queue_scratch.hpp).
//  * tiled (M > 32 where the row GEMM does not apply, M > 1024): 64x64x32 tiles, A and the dequantised weight tile
//    staged in LDS (weights transposed to [n][k] so both MFMA operands are one
//    ds_read_b128 per lane), double buffered, same fused epilogues.
// Dequantisation mirrors reference kernels/src/cuda/tc/gemm.cu:21,24 and the
// bias epilogue mirrors gemm.cu:73-80 / :118-124; accumulation is fp32.
#include <algorithm>
#include <atomic>
#include <climits>
#include <type_traits>
#include <utility>

#include "common.hpp"
#include "kernels.hpp"
#include "queue_scratch.hpp"

namespace tia {
namespace {

// Split-K scratch of the C ABIs' GEMMs: per hardware queue, 4 MiB of fp32
// partials and 1024 tile arrival counters (a split plan is sized to fit).
constexpr size_t kPoolFloats = size_t(1) << 20;
constexpr int kPoolTiles = 1024;
TIA_QUEUE_POOL(gemm_pool, kPoolFloats, kPoolTiles)

struct PoolSlot {
  float* parts;
  unsigned* ctr;
};
// The calling dispatch's slot (a whole wave calls it).
__device__ __forceinline__ PoolSlot gemm_pool_slot() {
  const int lane = int(threadIdx.x & 63);
  const unsigned long long key = lane < kQueueSlots ? gemm_pool_keys[lane] : 0ull;
  const int s = queue_slot_resolve(gemm_pool_keys, key);
  return {gemm_pool_data[s], gemm_pool_ctr[s]};
}

// Most partials a finishing thread loads from the pool (one round of 16-byte
// loads, 64 registers); the launchers size pool split plans to it.
constexpr int kPoolLoads = 16;
// Pool split plans: at most this many splits of a tile whose finishing threads
// each hold `per_thread` float4s.
constexpr int pool_max_splits(int per_thread) { return kPoolLoads / per_thread; }
// Rounds of loads the tile finisher takes at most (its tile is read by one
// workgroup, so more splits mostly add bytes for one CU to fetch).
constexpr int kTileRounds = 2;
// Most K splits of a pool GEMV (M <= 32) launch.
constexpr int kPoolGemvSplits = 8;
// A pool split plan over `tiles` tiles of `tile_floats` floats: at most
// `max_splits` splits, the tile-contiguous partials within the slot, and
// rounded to whole ranges of `units` (K steps or chunks).
int pool_splits(int splits, int64_t tiles, int64_t tile_floats, int max_splits, int units) {
  splits = std::max(1, std::min(splits, max_splits));
  while (splits > 1 && tiles * splits * tile_floats > int64_t(kPoolFloats)) --splits;
  const int per = (units + splits - 1) / splits;
  return (units + per - 1) / per;
}

// A 16-bit load from global memory through a pointer the compiler cannot
// place (a select of two kernel-argument pointers): typed as global, it is a
// global_load, not a flat one, so later waits count it exactly (a pending flat
// load makes the next wait for any load wait for every load).
__device__ __forceinline__ uint16_t ldg_u16(const uint16_t* ptr) {
  return *(const uint16_t __attribute__((address_space(1)))*)ptr;
}

__device__ __forceinline__ float epilogue_bias(const Epilogue& e, int n) {
  return e.bias ? h2f(e.bias[n]) : 0.f;
}

// Element (m, n) of the fp16 output (and of the residual): row-major, or P32
// fragment-packed.
__device__ __forceinline__ int64_t y_off(const Epilogue& e, int m, int n) {
  return e.p32 ? p32_off(m, n) : int64_t(m) * e.ldy + n;
}
__device__ __forceinline__ int64_t r_off(const Epilogue& e, int m, int n) {
  return e.p32 ? p32_off(m, n) : int64_t(m) * e.ldr + n;
}

// Request b and token t of row m of an EPI_QKV output: m = b * qrows + t, or
// m = row_start[b] + t over compact rows (a binary search of row_start).
__device__ __forceinline__ void qkv_row(const Epilogue& e, int m, int& b, int& t) {
  if (e.row_start) {
    int lo = 0, hi = e.batch;  // row_start[lo] <= m < row_start[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (e.row_start[mid] <= m) lo = mid;
      else hi = mid;
    }
    b = lo;
    t = m - e.row_start[lo];
  } else {
    b = m / e.qrows;
    t = m - b * e.qrows;
  }
}

// EPI_QKV element (m, n) = acc + bias of token t of request b: fp16 into y,
// and for the K and V columns of a real token the same bits into the slot
// cache.
__device__ __forceinline__ void qkv_store_bt(const Epilogue& e, int b, int t, int m, int n, float val) {
  const uint16_t hv = f2h(val);
  static_cast<uint16_t*>(e.y)[int64_t(m) * e.ldy + n] = hv;
  if (n >= e.hidden) {
    if (t < e.qlens[b]) {
      const int part = n >= 2 * e.hidden ? 2 : 1;
      const int c = n - part * e.hidden, h = c >> 6, d = c & 63;
      const int64_t pos = int64_t(e.offsets[b]) + t;
      const int64_t idx = (((int64_t(e.slots[b]) * e.layers + e.layer) * e.heads + h) * e.capacity + pos) * 64 + d;
      (part == 1 ? e.kcache : e.vcache)[idx] = hv;
    }
  }
}

__device__ __forceinline__ void qkv_store(const Epilogue& e, int m, int n, float val) {
  int b, t;
  qkv_row(e, m, b, t);
  qkv_store_bt(e, b, t, m, n, val);
}

// `bias` is epilogue_bias(e, n) (callers may load it early); EPI_RAW_F32 ignores it.
// `resid` is residual[m][n] for EPI_RESIDUAL (likewise loaded by the caller).
// Element (m, n) of epilogue kind K (EPI_F16 for any kind not listed).
template <int K>
__device__ __forceinline__ void epilogue_k(const Epilogue& e, int m, int n, float acc, float bias, float resid) {
  if constexpr (K == EPI_RAW_F32) {
    static_cast<float*>(e.y)[int64_t(m) * e.ldy + n] = acc;
  } else if constexpr (K == EPI_F32) {
    static_cast<float*>(e.y)[int64_t(m) * e.ldy + n] = acc + bias;
  } else if constexpr (K == EPI_GELU) {
    static_cast<uint16_t*>(e.y)[y_off(e, m, n)] = f2h(gelu_tanh(rt16(acc + bias)));
  } else if constexpr (K == EPI_RESIDUAL) {
    static_cast<uint16_t*>(e.y)[y_off(e, m, n)] = f2h(resid + rt16(acc + bias));
  } else if constexpr (K == EPI_QKV) {
    qkv_store(e, m, n, acc + bias);
  } else {
    static_cast<uint16_t*>(e.y)[y_off(e, m, n)] = f2h(acc + bias);
  }
}

// Calls f(std::integral_constant<int, kind>) for the epilogue kind of e, so a
// loop written inside f is compiled once per kind with no switch per element.
template <typename F>
__device__ __forceinline__ void with_epilogue_kind(const Epilogue& e, F&& f) {
  switch (e.kind) {
    case EPI_RAW_F32: f(std::integral_constant<int, EPI_RAW_F32>{}); return;
    case EPI_F32: f(std::integral_constant<int, EPI_F32>{}); return;
    case EPI_GELU: f(std::integral_constant<int, EPI_GELU>{}); return;
    case EPI_RESIDUAL: f(std::integral_constant<int, EPI_RESIDUAL>{}); return;
    case EPI_QKV: f(std::integral_constant<int, EPI_QKV>{}); return;
    default: f(std::integral_constant<int, EPI_F16>{}); return;
  }
}

__device__ __forceinline__ void apply_epilogue(const Epilogue& e, int m, int n, float acc, float bias,
                                               float resid) {
  with_epilogue_kind(e, [&](auto k) { epilogue_k<decltype(k)::value>(e, m, n, acc, bias, resid); });
}

__device__ __forceinline__ void apply_epilogue(const Epilogue& e, int m, int n, float acc, float bias) {
  apply_epilogue(e, m, n, acc, bias, e.kind == EPI_RESIDUAL ? h2f(e.residual[r_off(e, m, n)]) : 0.f);
}
__device__ __forceinline__ void apply_epilogue(const Epilogue& e, int m, int n, float acc) {
  apply_epilogue(e, m, n, acc, e.kind == EPI_RAW_F32 ? 0.f : epilogue_bias(e, n));
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
  int rblocks;         // row blocks (rowgemm_kernel)
  int steps;           // ceil(K / 32)
  int steps_per_block; // K steps owned by one workgroup (its waves take every 4th)
  int splits;
  bool defer;          // always leave fp32 partials (even for one split), no epilogue
  bool pool;           // splits > 1 finish in this launch through the queue pool
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
      out[r] = f16r(float(q) * scale);  // fp16_rn(float(q) * scale[n])
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

// POOL: this instantiation finishes splits > 1 in the launch through the queue
// pool (the C ABIs); the other keeps its registers free of the finisher.
template <bool INT8, int MT, bool WVEC, bool AVEC, bool POOL = false>
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
  if (POOL && p.splits > 1) {
    // This split's sums to the queue's pool slot, tile-contiguous: thread t
    // holds columns 4 (t % 16) .. + 3 of row t / 16 (+ 16 in pass 1); the
    // tile's last split to arrive loads every split's float4s of the rows
    // below M in one round of loads spread over its threads, sums them in
    // split order and runs the epilogue.
    const PoolSlot slot = gemm_pool_slot();
    const auto rs = agent_rsrc(slot.parts, uint32_t(kPoolFloats * sizeof(float)));
    const int t = int(threadIdx.x), c4 = t & 15, r0 = t >> 4;
    auto off = [&](int sp, int pass, int idx) {
      return uint32_t(((int64_t(tile) * p.splits + sp) * MT + pass) * kSkinnyThreads + idx) * 16u;
    };
#pragma unroll
    for (int pass = 0; pass < MT; ++pass) {
      const int row = r0 + 16 * pass;
      f32x4_t v;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        v[c] = red[0][row][4 * c4 + c] + red[1][row][4 * c4 + c] + red[2][row][4 * c4 + c] + red[3][row][4 * c4 + c];
      st_agent4(rs, off(split, pass, t), v);
    }
    if (!wg_arrive_last(slot.ctr + tile * kCounterStride, p.splits)) return;
    // Group gi of the G groups of 16 R threads (R = rows below M in a pass)
    // sums splits [gi spg, (gi + 1) spg) in order, group sums meet in LDS and
    // group 0 adds them in group order, then runs the epilogue.
    constexpr int SMAX = pool_max_splits(MT);
    __shared__ f32x4_t gsum[kSkinnyThreads][MT];
    const int rr = min(p.m, 16), per = 16 * rr, ng = max(1, kSkinnyThreads / per);
    const int spg = (p.splits + ng - 1) / ng;
    const int gi = t / per, wi = t - gi * per;
    f32x4_t v[MT][SMAX];
#pragma unroll
    for (int pass = 0; pass < MT; ++pass)
#pragma unroll
      for (int u = 0; u < SMAX; ++u) {
        const int sp = gi * spg + u;
        v[pass][u] = (gi < ng && u < spg && sp < p.splits && (wi >> 4) + 16 * pass < p.m) ? ld_agent4(rs, off(sp, pass, wi))
                                                                                          : f32x4_t{};
      }
    depart(slot.ctr + tile * kCounterStride);
#pragma unroll
    for (int pass = 0; pass < MT; ++pass) {
      f32x4_t acc = v[pass][0];
#pragma unroll
      for (int u = 1; u < SMAX; ++u)
        if (u < spg && gi * spg + u < p.splits) acc += v[pass][u];
      if (gi < ng) gsum[t][pass] = acc;
    }
    __syncthreads();
    if (gi != 0) return;
    with_epilogue_kind(p.epi, [&](auto kind) {
      constexpr int K = decltype(kind)::value;
#pragma unroll
      for (int pass = 0; pass < MT; ++pass) {
        const int row = (wi >> 4) + 16 * pass;
        if (row >= p.m) continue;
        f32x4_t acc = gsum[wi][pass];
        for (int q = 1; q < ng && q * spg < p.splits; ++q) acc += gsum[q * per + wi][pass];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int n = n0 + 4 * (wi & 15) + c;
          if (n >= p.n) continue;
          const float bias = K == EPI_RAW_F32 ? 0.f : epilogue_bias(p.epi, n);
          const float resid = K == EPI_RESIDUAL ? h2f(p.epi.residual[r_off(p.epi, row, n)]) : 0.f;
          epilogue_k<K>(p.epi, row, n, acc[c], bias, resid);
        }
      }
    });
    return;
  }
  for (int e = threadIdx.x; e < kElems; e += kSkinnyThreads) {
    const int row = e >> 6, cc = e & 63, n = n0 + cc;
    if (row < p.m && n < p.n) {
      const float s = red[0][row][cc] + red[1][row][cc] + red[2][row][cc] + red[3][row][cc];
      if (p.splits == 1 && !p.defer) apply_epilogue(p.epi, row, n, s);
      else p.partials[(int64_t(split) * p.m + row) * p.n + n] = s;
    }
  }
}

// Row-major int8 GEMV of the C ABIs at M <= 16 (q [K][N] as the reference
// keeps it, reference kernels/src/cuda/tc/gemm.cu:21): workgroup (tile, split)
// covers one 64-column tile over at most W * S 32-row K steps; wave w takes
// steps w, w + W, ... with every load of the wave in flight before its first
// MFMA (the skinny kernel's fragments and dequantisation).  The waves meet in
// LDS; with one split the workgroup runs the epilogue, otherwise each split's
// sums go to the queue's pool slot and the tile's last split to arrive adds
// them in split order (one round of loads) and runs it.  The plan depends on N
// and K only, so a row's result does not depend on M.
constexpr int kRowSplits = 16;
template <int W, int S>
__global__ __launch_bounds__(W * 64) void rowgemv_kernel(SkinnyParams p) {
  __shared__ float red[W][16][65];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  // Consecutive (tile, split) ids per XCD (blocks go round-robin over the 8
  // XCDs): the two tiles that share a 128-byte weight line read it through one L2.
  const int nb = gridDim.x, bid = blockIdx.x;
  const int logical = (nb % 8 == 0) ? (bid % 8) * (nb / 8) + bid / 8 : bid;
  const int tile = logical % p.ntile, split = logical / p.ntile;
  const int s0 = split * p.steps_per_block, s1 = min(p.steps, s0 + p.steps_per_block);
  const int n0 = tile * 64, col = n0 + 4 * j;
  float sc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) sc[c] = col + c < p.n ? p.scales[col + c] : 0.f;
  WFrag<true> f[S];
  half8_t a[S];
#pragma unroll
  for (int i = 0; i < S; ++i) {
    const int st = s0 + wave + W * i;
    if (st < s1) {
      load_wfrag<true, true>(f[i], p.w, p.k, p.n, p.ldw, st * 32 + 8 * g, col);
      a[i] = afrag<true>(p.a, p.lda, p.m, p.k, j, st * 32 + 8 * g);
    }
  }
  float4_t acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < S; ++i) {
    if (s0 + wave + W * i < s1) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], bfrag<true>(f[i], c, sc[c]), acc[c], 0, 0, 0);
    }
  }
  // MFMA output: lane holds rows 4g + v (v = 0..3) of column j of each 16x16 block.
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int v = 0; v < 4; ++v) red[wave][4 * g + v][4 * j + c] = acc[c][v];
  __syncthreads();
  auto wave_sum = [&](int row, int cc) {
    float s = red[0][row][cc];
#pragma unroll
    for (int w = 1; w < W; ++w) s += red[w][row][cc];
    return s;
  };
  if (p.splits == 1) {
    for (int e = threadIdx.x; e < p.m * 64; e += W * 64) {
      const int row = e >> 6, cc = e & 63, n = n0 + cc;
      if (n < p.n) apply_epilogue(p.epi, row, n, wave_sum(row, cc));
    }
    return;
  }
  // Split sp of the tile at parts + sp * 1024 + (row * 64 + column).
  const PoolSlot slot = gemm_pool_slot();
  float* parts = slot.parts + int64_t(tile) * p.splits * 1024;
  for (int e = threadIdx.x; e < p.m * 64; e += W * 64) st_agent(parts + split * 1024 + e, wave_sum(e >> 6, e & 63));
  if (!wg_arrive_last(slot.ctr + tile * kCounterStride, p.splits)) return;
  for (int e = threadIdx.x; e < p.m * 64; e += W * 64) {
    float v[kRowSplits];
#pragma unroll
    for (int u = 0; u < kRowSplits; ++u) v[u] = u < p.splits ? ld_agent(parts + u * 1024 + e) : 0.f;
    float s = v[0];
#pragma unroll
    for (int u = 1; u < kRowSplits; ++u)
      if (u < p.splits) s += v[u];
    const int n = n0 + (e & 63);
    if (n < p.n) apply_epilogue(p.epi, e >> 6, n, s);
  }
  depart(slot.ctr + tile * kCounterStride);
}

// Row-major int8 GEMM of the C ABIs at 16 < M <= 1024 (q [K][N] as the reference
// keeps it, reference kernels/src/cuda/tc/gemm.cu:21), built like the skinny
// kernel (weight fragments from HBM straight into MFMA B registers, dequantised
// there, no LDS staging): workgroup (tile, row block, split) covers one
// 64-column tile and 16 * MT rows over a range of 32-row K steps; wave w takes
// steps w, w + W, ..., S of them per round with every load of the round in
// flight before its first MFMA.  The waves meet in LDS; with one split the
// workgroup runs the epilogue, otherwise each split's sums go to the queue's
// pool slot as float4s and the unit's last split to arrive adds them in split
// order (one round of loads) and runs it.  Row blocks are 16 rows up to M = 64,
// then 32; the K split follows the count of (tile, row block) units, so unlike
// the M <= 16 GEMV a row's sums may differ between M values (the reference ABI
// promises no batch invariance; the runtime never takes this path).
template <int MT, int W, int S>
__global__ __launch_bounds__(W * 64) void rowgemm_kernel(SkinnyParams p) {
  constexpr int R = 16 * MT, NT = W * 64;
  constexpr int OUT4 = (R * 16 + NT - 1) / NT;  // float4 outputs of a finishing thread
  constexpr int SMAX = kPoolLoads / OUT4;       // splits its one round of loads covers
  __shared__ float red[W][R][65];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  // Consecutive ids per XCD (blocks go round-robin over the 8 XCDs), column
  // tile fastest: the two tiles that share a 128-byte weight line, and the
  // tiles that share a row block's A rows, are read through one L2.
  const int nb = gridDim.x, bid = blockIdx.x;
  const int logical = (nb % 8 == 0) ? (bid % 8) * (nb / 8) + bid / 8 : bid;
  const int tile = logical % p.ntile, rest = logical / p.ntile;
  const int rb = rest % p.rblocks, split = rest / p.rblocks;
  const int m0 = rb * R, rows = min(R, p.m - m0);
  const int s0 = split * p.steps_per_block, s1 = min(p.steps, s0 + p.steps_per_block);
  const int n0 = tile * 64, col = n0 + 4 * j;
  float sc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) sc[c] = col + c < p.n ? p.scales[col + c] : 0.f;
  float4_t acc[MT][4];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[t][c] = float4_t{0.f, 0.f, 0.f, 0.f};
  for (int base = s0 + wave; base < s1; base += W * S) {
    WFrag<true> f[S];
    half8_t a[S][MT];
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int st = base + W * i;
      if (st < s1) {
        load_wfrag<true, true>(f[i], p.w, p.k, p.n, p.ldw, st * 32 + 8 * g, col);
#pragma unroll
        for (int t = 0; t < MT; ++t) a[i][t] = afrag<true>(p.a, p.lda, p.m, p.k, m0 + 16 * t + j, st * 32 + 8 * g);
      }
    }
#pragma unroll
    for (int i = 0; i < S; ++i) {
      if (base + W * i < s1) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const half8_t b = bfrag<true>(f[i], c, sc[c]);
#pragma unroll
          for (int t = 0; t < MT; ++t) acc[t][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i][t], b, acc[t][c], 0, 0, 0);
        }
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
  // float4 output q of the unit: row q / 16, columns 4 (q % 16) .. + 3.
  const int tid = int(threadIdx.x), nq = rows * 16;
  auto wave_sum4 = [&](int q) {
    const int r = q >> 4, c0 = 4 * (q & 15);
    f32x4_t v;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float x = red[0][r][c0 + c];
#pragma unroll
      for (int w = 1; w < W; ++w) x += red[w][r][c0 + c];
      v[c] = x;
    }
    return v;
  };
  auto epilogue4 = [&](int q, const f32x4_t& v) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int n = n0 + 4 * (q & 15) + c;
      if (n < p.n) apply_epilogue(p.epi, m0 + (q >> 4), n, v[c]);
    }
  };
  if (p.splits == 1) {
    for (int q = tid; q < nq; q += NT) epilogue4(q, wave_sum4(q));
    return;
  }
  const PoolSlot slot = gemm_pool_slot();
  const auto rs = agent_rsrc(slot.parts, uint32_t(kPoolFloats * sizeof(float)));
  const int unit = tile * p.rblocks + rb;
  auto off = [&](int sp, int q) { return uint32_t(((int64_t(unit) * p.splits + sp) * (R * 16) + q) * 16); };
  for (int q = tid; q < nq; q += NT) st_agent4(rs, off(split, q), wave_sum4(q));
  if (!wg_arrive_last(slot.ctr + unit * kCounterStride, p.splits)) return;
  f32x4_t v[OUT4][SMAX];
#pragma unroll
  for (int o = 0; o < OUT4; ++o)
#pragma unroll
    for (int u = 0; u < SMAX; ++u) {
      const int q = tid + o * NT;
      v[o][u] = q < nq && u < p.splits ? ld_agent4(rs, off(u, q)) : f32x4_t{};
    }
  depart(slot.ctr + unit * kCounterStride);
#pragma unroll
  for (int o = 0; o < OUT4; ++o) {
    const int q = tid + o * NT;
    if (q >= nq) continue;
    f32x4_t sum = v[o][0];
#pragma unroll
    for (int u = 1; u < SMAX; ++u)
      if (u < p.splits) sum += v[o][u];
    epilogue4(q, sum);
  }
}
// Most splits of a rowgemm_kernel<MT, W, S> plan.
constexpr int rowgemm_max_splits(int mt, int w) { return kPoolLoads / ((16 * mt * 16 + w * 64 - 1) / (w * 64)); }

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
  // One loop per epilogue kind (the kind is uniform over the launch).
  with_epilogue_kind(epi, [&](auto kind) {
    constexpr int K = decltype(kind)::value;
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
        const float bias = K == EPI_RAW_F32 ? 0.f : epilogue_bias(epi, col);
        const float resid = K == EPI_RESIDUAL ? h2f(epi.residual[r_off(epi, row, col)]) : 0.f;
        epilogue_k<K>(epi, row, col, ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane], bias, resid);
      }
      __syncthreads();
    }
  });
}

// ---------------------------------------------------------------------------
// Panel-packed int8 weights and the decode GEMV over them (M <= 32)
// ---------------------------------------------------------------------------
// Panel layout: column block cb (16 columns), K chunk kc (64 rows) is one 1 KiB
// record at ((cb * KC + kc) * 64 + lane) * 16 bytes; lane's 16 bytes are column
// cb*16 + (lane & 15), rows kc*64 + 8*(lane >> 4) + r (bytes 0..7) and
// kc*64 + 32 + 8*(lane >> 4) + r (bytes 8..15), r = 0..7: the B operands of two
// consecutive v_mfma_f32_16x16x32_f16 steps.  Entries past K or N are 0.
__global__ void pack_w8_kernel(const int8_t* q, int64_t ldq, int k, int n, int kc, int64_t total16,
                               u32x4_t* out) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total16;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int lane = int(i & 63);
    const int64_t rec = i >> 6;
    const int chunk = int(rec % kc), cb = int(rec / kc);
    const int col = cb * 16 + (lane & 15), g = lane >> 4;
    uint32_t d[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t v = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int r = (w & 1) * 4 + b;
        const int row = chunk * 64 + (w >> 1) * 32 + 8 * g + r;
        const uint8_t byte = (row < k && col < n) ? uint8_t(q[int64_t(row) * ldq + col]) : uint8_t(0);
        v |= uint32_t(byte) << (8 * b);
      }
      d[w] = v;
    }
    out[i] = u32x4_t{d[0], d[1], d[2], d[3]};
  }
}

struct PackedParams {
  const uint16_t* a;
  int64_t lda;
  const u32x4_t* w;     // panel-packed records
  const float* scales;  // fp32 [N]
  int m, n, k;
  int nb, kc;           // column blocks, K chunks
  int chunks_per_split, splits;
  bool defer;
  Epilogue epi;
  float* partials;      // [splits][M][N]
  const uint16_t* ln_gamma;  // A = LayerNorm(a rows; gamma, beta, eps) when set
  const uint16_t* ln_beta;
  float ln_eps;
  // MT = 1, one split, fp32 epilogue: when set, per (workgroup, row) best
  // output and its column, as the wide GEMV leaves them for greedy decoding.
  float* amax_v;
  int32_t* amax_i;
  int rblocks;          // RB launches: row blocks of 16 * MT rows
};


// fp16_rn(float(q) * scale) of the 8 bytes in (lo, hi): one MFMA B operand.
__device__ __forceinline__ half8_t dequant8(uint32_t lo, uint32_t hi, float scale) {
  half8_t out;
#pragma unroll
  for (int r = 0; r < 4; ++r) out[r] = f16r(float(int8_t(lo >> (8 * r))) * scale);
#pragma unroll
  for (int r = 0; r < 4; ++r) out[4 + r] = f16r(float(int8_t(hi >> (8 * r))) * scale);
  return out;
}

// One workgroup of W waves owns CBG consecutive column blocks and the K chunks
// of one split; wave w takes chunks w, w + W, ... and issues the loads of up to
// CPW of them (CBG weight records and the A fragments of each chunk) before the
// first MFMA, so a split is one memory round trip, and each A fragment feeds
// CBG column blocks (at M = 32 the A rows would otherwise be re-read for every
// 16 columns).  The W partial sums are reduced through LDS in wave order, then
// the epilogue runs (or fp32 partials are stored for a split/deferred launch).
// Loads use clamped chunk, row and column-block indices, never predicates
// (rows >= M, blocks >= nb are computed from valid data and never stored).
// LNA: A is LayerNorm(a) over its K = hidden columns, computed from the loaded
// fragments before the MFMAs; the launch then covers K in one round of one
// split (W * CPW >= kc).  PA: A is P32 fragment-packed (each A fragment one
// contiguous KiB).
// POOL (the C ABIs): a split launch finishes in the kernel -- every
// workgroup stores its reduced sums to the queue pool and the last of a column
// group's splits to arrive adds them in split order and runs the epilogue.
template <int MT, int W, int CPW, int CBG, bool LNA = false, bool PA = false, bool CW = false, bool POOL = false,
          bool RB = false>
__global__ __launch_bounds__(W * 64) void gemv_packed_kernel(PackedParams p) {
  __shared__ float red[W][CBG][MT * 256];
  __shared__ float stat[LNA ? W : 1][MT * 16];  // per-wave LayerNorm partial sums
  // LayerNorm gamma (q < CPW) and beta (q >= CPW) of chunk q % CPW of each
  // wave, 16 bytes at [wave][q * 8 + part]: one load per lane, not one per A
  // fragment and lane group.
  __shared__ half8_t gbl[LNA ? W : 1][LNA ? 16 * CPW : 1];
  // The wave index is uniform: chunk bounds below are scalar, so every load of a
  // round is issued before the first wait.
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int nbk = gridDim.x, bid = blockIdx.x;
  const int logical = (nbk % 8 == 0) ? (bid % 8) * (nbk / 8) + bid / 8 : bid;
  const int groups = (p.nb + CBG - 1) / CBG;
  // RB: row block rb (16 * MT rows from m0) varies fastest, so the row blocks
  // of a column group read its records through one XCD's L2.
  const int rb = RB ? logical % p.rblocks : 0;
  const int unit = RB ? logical / p.rblocks : logical;
  const int grp = unit % groups, split = unit / groups;
  const int m0 = RB ? rb * 16 * MT : 0, mrow = p.m - m0;
  const int cb0 = grp * CBG;
  const int c_begin = split * p.chunks_per_split;
  const int c_end = min(p.kc, c_begin + p.chunks_per_split);
  const bool epi_now = (POOL || p.splits == 1) && !p.defer;
  const bool has_bias = epi_now && p.epi.kind != EPI_RAW_F32 && p.epi.bias;

  const u32x4_t* wb[CBG];
  const float* scp[CBG];
  float colmask[CBG];
  uint16_t bias_raw[CBG];
  // Unconditional load (of A's first element when there is no bias) whose value
  // is converted only in the epilogue: a conditional load here would be waited
  // for at once, before the weight loads are issued.
  const uint16_t* bsrc = has_bias ? p.epi.bias : p.a;
#pragma unroll
  for (int r = 0; r < CBG; ++r) {
    const int cb = min(cb0 + r, p.nb - 1), col = cb * 16 + j;
    wb[r] = p.w + int64_t(cb) * p.kc * 64 + lane;
    scp[r] = p.scales + min(col, p.n - 1);
    colmask[r] = (cb0 + r < p.nb && col < p.n) ? 1.f : 0.f;
    // Every output this thread finishes in block r is in column (cb0 + r) * 16 +
    // (threadIdx.x & 15): its bias is fetched now, not after the reduction.
    bias_raw[r] = ldg_u16(bsrc + (has_bias ? min((cb0 + r) * 16 + int(threadIdx.x & 15), p.n - 1) : 0));
  }
  const uint16_t* arow[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) arow[t] = p.a + (int64_t(m0) + min(16 * t + j, mrow - 1)) * p.lda + 8 * g;
  // PA: lane offset inside a fragment, rows past M clamped to row M - 1 like
  // the row-major path (at M = 1 a fragment load then touches one cache line).
  int pa_lane[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) pa_lane[t] = (min(16 * t + j, mrow - 1) - 16 * t + 16 * g) * 8;

  // Outputs of this thread in the epilogue: o = threadIdx.x + it * W * 64 over
  // CBG blocks of rows x 16.  Their residuals are loaded now, unconditionally
  // (A's first element stands in), like the bias.
  constexpr int kOutIters = (CBG * MT * 256 + W * 64 - 1) / (W * 64);
  const int rows = min(mrow, MT * 16), per_block = rows * 16;
  const bool has_res = epi_now && p.epi.kind == EPI_RESIDUAL;
  const uint16_t* rsrc = has_res ? p.epi.residual : p.a;
  // Output o of the epilogue: block r = o / per_block, element rem (with one
  // block, o itself: no division).
  auto block_of = [&](int o, int& r, int& rem) {
    if constexpr (CBG == 1) {
      r = 0;
      rem = o;
    } else {
      r = o / per_block;
      rem = o - r * per_block;
    }
  };
  uint16_t res_raw[kOutIters];
#pragma unroll
  for (int it = 0; it < kOutIters; ++it) {
    // The offset arithmetic only under a residual epilogue (a uniform branch);
    // the load itself stays unconditional.
    int64_t roff = 0;
    if (has_res) {
      const int o = threadIdx.x + it * W * 64;
      int r, rem;
      block_of(o, r, rem);
      const int n = (cb0 + r) * 16 + (rem & 15);
      if (o < CBG * per_block && cb0 + r < p.nb && n < p.n) roff = r_off(p.epi, m0 + (rem >> 4), n);
    }
    res_raw[it] = ldg_u16(rsrc + roff);
  }

  float4_t acc[MT][CBG];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < CBG; ++r) acc[t][r] = float4_t{0.f, 0.f, 0.f, 0.f};

  // One round: the loads of chunks c0, c0 + W, ... (CPW of them), then the MFMAs.
  auto round = [&](int c0) {
    u32x4_t wf[CPW][CBG];
    half8_t af[CPW][2][MT];
    half8_t gbv;
    // CW: cached loads, for two decode lanes that stream the same records
    // microseconds apart, the second finding them in cache (b = 32 decode as
    // two 16-row lanes: 102 K against 92 K tok/s with nontemporal loads);
    // otherwise the records stream past the caches (GPT-2 XL decode, whose
    // 1.6 GB do not stay cached: 12.06 K against 11.81 K tok/s with cached
    // loads).
    auto load_w = [&](int i) {
      const int c = min(c0 + i * W, c_end - 1);
#pragma unroll
      for (int r = 0; r < CBG; ++r)
        wf[i][r] = CW ? wb[r][int64_t(c) * 64] : __builtin_nontemporal_load(wb[r] + int64_t(c) * 64);
    };
    auto load_a = [&](int i) {
      const int c = min(c0 + i * W, c_end - 1);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
#pragma unroll
        for (int t = 0; t < MT; ++t)
          af[i][s][t] = PA ? *reinterpret_cast<const half8_t*>(p.a + ((int64_t(c) * 2 + t) * 2 + s) * 512 + pa_lane[t])
                           : *reinterpret_cast<const half8_t*>(arow[t] + c * 64 + 32 * s);
      }
    };
    // Lanes past 16 * CPW repeat the last (q, part) pair: same address, same
    // LDS slot, same value.
    const int gb_q = min(lane >> 3, 2 * CPW - 1), gb_slot = gb_q * 8 + (lane & 7);
    if constexpr (LNA) {
      // gamma/beta and A first: the LayerNorm below needs only them (loads
      // complete in order), so it runs while the weight records are in flight.
      const int c = min(c0 + (gb_q % CPW) * W, c_end - 1);
      gbv = *reinterpret_cast<const half8_t*>((gb_q < CPW ? p.ln_gamma : p.ln_beta) + c * 64 + (lane & 7) * 8);
#pragma unroll
      for (int i = 0; i < CPW; ++i) load_a(i);
#pragma unroll
      for (int i = 0; i < CPW; ++i) load_w(i);
    } else {
#pragma unroll
      for (int i = 0; i < CPW; ++i) {
        load_w(i);
        load_a(i);
      }
    }
    // The scales are loaded after the round's weights and A (and waited for
    // with them); the scheduling barrier keeps every load of the round ahead of
    // the first wait.
    float sc[CBG];
#pragma unroll
    for (int r = 0; r < CBG; ++r) sc[r] = *scp[r];
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (LNA) {
      // LayerNorm of the A rows over the K = hidden columns: two-pass fp32
      // mean and variance as the row kernel (sum of x, then of (x - mean)^2),
      // rsqrt(var + eps), fp16_rn((x * inv - mean * inv) * gamma + beta).  Every
      // chunk of K is in this workgroup's single round, spread over the waves
      // and the 4 k-groups of a row's lanes.  The first pass sums fp16 pairs
      // with dot2 (exact products, fp32 sums) and the normalization reads x,
      // gamma and beta as fp16 operands of mixed-precision fmas.
      float mean[MT], inv[MT], shift[MT];
      gbl[wave][gb_slot] = gbv;  // read after the barriers below
      const half2_t ones = {f16(1.f), f16(1.f)};
      // An opaque 1.0: fma(x, one, -mean) stays one mixed-precision fma (the
      // compiler would turn a literal 1.0 into a conversion and a subtraction).
      float one = 1.f;
      asm volatile("" : "+v"(one));
#pragma unroll
      for (int pass = 0; pass < 2; ++pass) {
        float part[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          part[t] = 0.f;
#pragma unroll
          for (int i = 0; i < CPW; ++i) {
            float pc = 0.f;
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
              for (int e = 0; e < 8; e += 2) {
                if (pass == 0) {
                  pc = __builtin_amdgcn_fdot2(half2_t{af[i][s][t][e], af[i][s][t][e + 1]}, ones, pc, false);
                } else {
                  const float d0 = fmaf(float(af[i][s][t][e]), one, -mean[t]);
                  const float d1 = fmaf(float(af[i][s][t][e + 1]), one, -mean[t]);
                  pc = fmaf(d1, d1, fmaf(d0, d0, pc));
                }
              }
            // A chunk past the end re-read the last one: it is not counted.
            part[t] += c0 + i * W < c_end ? pc : 0.f;
          }
          part[t] += __shfl_xor(part[t], 16, 64);
          part[t] += __shfl_xor(part[t], 32, 64);
          // The 4 lanes of row j hold the same sum (branch-free store: the
          // LayerNorm stays one basic block, so the scheduling barriers hold).
          stat[wave][16 * t + j] = part[t];
        }
        lds_barrier();
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          float tot = 0.f;
#pragma unroll
          for (int w = 0; w < W; ++w) tot += stat[w][16 * t + j];
          if (pass == 0) mean[t] = tot / float(p.k);
          else inv[t] = rsqrtf(tot / float(p.k) + p.ln_eps);
        }
        lds_barrier();
      }
#pragma unroll
      for (int t = 0; t < MT; ++t) shift[t] = -mean[t] * inv[t];
#pragma unroll
      for (int i = 0; i < CPW; ++i)
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const half8_t gam = gbl[wave][i * 8 + 4 * s + g], bet = gbl[wave][(CPW + i) * 8 + 4 * s + g];
#pragma unroll
          for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int e = 0; e < 8; ++e)
              af[i][s][t][e] =
                  f16r(fmaf(fmaf(float(af[i][s][t][e]), inv[t], shift[t]), float(gam[e]), float(bet[e])));
        }
      // Keep the weight dequantization (which waits for the records) after the
      // LayerNorm.
      __builtin_amdgcn_sched_barrier(0);
    }
    // A chunk past the split's end re-read the last chunk; its scale is 0 so
    // its B operands are +-0 and the MFMAs leave the sums unchanged.
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
      const bool live = c0 + i * W < c_end;
#pragma unroll
      for (int r = 0; r < CBG; ++r) {
        const float si = live ? sc[r] * colmask[r] : 0.f;
        const half8_t b0 = dequant8(wf[i][r][0], wf[i][r][1], si);
        const half8_t b1 = dequant8(wf[i][r][2], wf[i][r][3], si);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          acc[t][r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i][0][t], b0, acc[t][r], 0, 0, 0);
          acc[t][r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i][1][t], b1, acc[t][r], 0, 0, 0);
        }
      }
    }
  };
  if constexpr (LNA) {
    // Every wave runs the single round (its barriers included), chunks or not.
    round(c_begin + wave);
  } else {
    for (int c0 = c_begin + wave; c0 < c_end; c0 += W * CPW) round(c0);
  }

  // MFMA output: lane holds rows 4g + v of column j of each 16x16 block.
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < CBG; ++r)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[wave][r][(16 * t + 4 * g + v) * 16 + j] = acc[t][r][v];
  __syncthreads();
  // The epilogue recomputes its indices (an opaque copy of the thread index
  // keeps the compiler from holding those of the residual loads live through
  // the main loop).
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  if constexpr (POOL) {
    if (p.splits > 1) {
      // Split s of column group grp at ((grp * splits + s) * kTileOut + o), o
      // the output index of the epilogue loop; the finisher loads every
      // split of its outputs in one round.
      constexpr int kTileOut = CBG * MT * 256, SMAX = kPoolLoads / kOutIters;
      const PoolSlot slot = gemm_pool_slot();
      const float* tile_parts = slot.parts + int64_t(grp) * p.splits * kTileOut;
#pragma unroll
      for (int it = 0; it < kOutIters; ++it) {
        const int o = tid + it * W * 64;
        int r, rem;
        block_of(o, r, rem);
        if (o >= CBG * per_block) continue;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) v += red[w][r][rem];
        st_agent(const_cast<float*>(tile_parts) + int64_t(split) * kTileOut + o, v);
      }
      if (!wg_arrive_last(slot.ctr + grp * kCounterStride, p.splits)) return;
      float part[kOutIters][SMAX];
#pragma unroll
      for (int it = 0; it < kOutIters; ++it) {
        const int o = tid + it * W * 64;
#pragma unroll
        for (int u = 0; u < SMAX; ++u)
          part[it][u] = (u < p.splits && o < CBG * per_block) ? ld_agent(tile_parts + int64_t(u) * kTileOut + o) : 0.f;
      }
      depart(slot.ctr + grp * kCounterStride);
#pragma unroll
      for (int it = 0; it < kOutIters; ++it) {
        const int o = tid + it * W * 64;
        int r, rem;
        block_of(o, r, rem);
        const int row = rem >> 4, n = (cb0 + r) * 16 + (rem & 15);
        if (o >= CBG * per_block || cb0 + r >= p.nb || n >= p.n) continue;
        float v = part[it][0];
#pragma unroll
        for (int u = 1; u < SMAX; ++u)
          if (u < p.splits) v += part[it][u];
        uint16_t braw = bias_raw[0];
#pragma unroll
        for (int q = 1; q < CBG; ++q) braw = r == q ? bias_raw[q] : braw;
        apply_epilogue(p.epi, m0 + row, n, v, has_bias ? h2f(braw) : 0.f, has_res ? h2f(res_raw[it]) : 0.f);
      }
      return;
    }
  }
  float amax_val = -__builtin_huge_valf();  // MT = 1: this thread's (single) output
  int amax_col = INT_MAX;
#pragma unroll
  for (int it = 0; it < kOutIters; ++it) {
    const int o = tid + it * W * 64;
    int r, rem;
    block_of(o, r, rem);
    const int row = rem >> 4, n = (cb0 + r) * 16 + (rem & 15);
    if (o >= CBG * per_block || cb0 + r >= p.nb || n >= p.n) continue;
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) s += red[w][r][rem];
    uint16_t braw = bias_raw[0];
#pragma unroll
    for (int q = 1; q < CBG; ++q) braw = r == q ? bias_raw[q] : braw;
    const float bias = has_bias ? h2f(braw) : 0.f;
    if (epi_now) apply_epilogue(p.epi, m0 + row, n, s, bias, has_res ? h2f(res_raw[it]) : 0.f);
    else p.partials[(int64_t(split) * p.m + m0 + row) * p.n + n] = s;
    if (MT == 1) {
      amax_val = s + bias;  // the EPI_F32 value
      amax_col = n;
    }
  }
  if constexpr (MT == 1) {
    // Argmax partials: thread o holds row o / 16, column o % 16 of the single
    // block (CBG = 1, one output per thread), so a row's 16 columns are 16
    // consecutive lanes of one wave.
    static_assert(MT != 1 || (CBG == 1 && kOutIters == 1), "one output per thread");
    if (!p.amax_v) return;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1)
      amax_merge(amax_val, amax_col, __shfl_xor(amax_val, o, 64), __shfl_xor(amax_col, o, 64));
    if ((tid & 15) == 0 && tid < per_block) {
      p.amax_v[(tid >> 4) * groups + grp] = amax_val;
      p.amax_i[(tid >> 4) * groups + grp] = amax_col;
    }
  }
}

// ---------------------------------------------------------------------------
// Part-block GEMV for a single row of A (M = 1) over the panel-packed weights,
// without MFMA.  A workgroup owns QC in {4, 8} columns of a 16-column block, so
// N = 768 runs on 96 (QC 8) or 192 (QC 4) workgroups instead of 48, each
// streaming a part of the bytes (a single-row product has no use for the
// 16-row MFMA shape).  QC 4 reads half cache lines and measured slower; the
// launcher uses QC 8.  In a record the QC columns of part h sit in lanes
// QC*h .. QC*h + QC - 1 of each 16-lane group, four runs of 16*QC bytes; a wave
// load takes those runs of 16 / QC consecutive records.  Lane L holds column
// 16 cb + QC h + (L % QC) at the 16 rows of lane group (L / QC) % 4 of record
// (16 / QC) * step + L / (4 QC).  Products are fp16_rn(float(q) * scale) times
// A in fp16 (dot2, fp32 sums); the lanes of a column, then the W waves
// (through LDS), are summed and the epilogue runs in the kernel (or the fp32
// sums go to partials split 0 for a deferred launch).  Wave w takes record
// steps w, w + W, ... and issues LPW of them before the first wait; records
// past the end are clamped to the last one and weighted 0.
template <int W, int LPW, int QC>
__global__ __launch_bounds__(W * 64) void gemv_part_kernel(PackedParams p) {
  static_assert(QC == 4 || QC == 8, "4 or 8 columns per workgroup");
  constexpr int RPL = 16 / QC;  // records per wave load
  __shared__ float red[W][QC];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane % QC, g = (lane / QC) & 3, r = lane / (4 * QC);
  const int cb = blockIdx.x / RPL, h = blockIdx.x % RPL;
  const int col = cb * 16 + QC * h + c;
  const bool epi_now = !p.defer;
  const bool has_bias = epi_now && p.epi.kind != EPI_RAW_F32 && p.epi.bias;
  const bool has_res = epi_now && p.epi.kind == EPI_RESIDUAL;
  // Epilogue operands of output column cb*16 + QC h + threadIdx.x % QC, loaded
  // first and unconditionally (A's first element stands in), converted at use.
  const int ecol = min(cb * 16 + QC * h + int(threadIdx.x % QC), p.n - 1);
  const uint16_t bias_raw = ldg_u16(has_bias ? p.epi.bias + ecol : p.a);
  const uint16_t res_raw = ldg_u16(has_res ? p.epi.residual + r_off(p.epi, 0, ecol) : p.a);
  // Masked only at use: an arithmetic use here would wait for this load before
  // the weight loads below are issued.
  const float scale = p.scales[min(col, p.n - 1)];
  const bool col_ok = col < p.n;
  const u32x4_t* wb = p.w + int64_t(cb) * p.kc * 64 + g * 16 + QC * h + c;
  const uint16_t* arow = p.a + 8 * g;
  const int steps = (p.kc + RPL - 1) / RPL;
  float acc = 0.f;
  for (int s0 = wave; s0 < steps; s0 += W * LPW) {
    u32x4_t wf[LPW];
    half8_t af[LPW][2];
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int kc = min(RPL * min(s0 + i * W, steps - 1) + r, p.kc - 1);
      wf[i] = __builtin_nontemporal_load(wb + int64_t(kc) * 64);
      af[i][0] = *reinterpret_cast<const half8_t*>(arow + kc * 64);
      af[i][1] = *reinterpret_cast<const half8_t*>(arow + kc * 64 + 32);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const bool live = s0 + i * W < steps && RPL * (s0 + i * W) + r < p.kc;
      const float si = live && col_ok ? scale : 0.f;
      const half8_t b0 = dequant8(wf[i][0], wf[i][1], si);
      const half8_t b1 = dequant8(wf[i][2], wf[i][3], si);
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        acc = __builtin_amdgcn_fdot2(half2_t{af[i][0][e], af[i][0][e + 1]}, half2_t{b0[e], b0[e + 1]}, acc, false);
        acc = __builtin_amdgcn_fdot2(half2_t{af[i][1][e], af[i][1][e + 1]}, half2_t{b1[e], b1[e + 1]}, acc, false);
      }
    }
  }
#pragma unroll
  for (int o = QC; o < 64; o <<= 1) acc += __shfl_xor(acc, o, 64);
  if (lane < QC) red[wave][lane] = acc;
  __syncthreads();
  if (threadIdx.x >= QC || cb * 16 + QC * h + int(threadIdx.x) >= p.n) return;
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < W; ++w) s += red[w][threadIdx.x];
  if (epi_now) apply_epilogue(p.epi, 0, ecol, s, has_bias ? h2f(bias_raw) : 0.f, has_res ? h2f(res_raw) : 0.f);
  else p.partials[ecol] = s;
}

// ---------------------------------------------------------------------------
// Wide decode GEMV (the LM head): 17..32 rows against many 16-column blocks.
// Two workgroups per CU over per = ceil(blocks / (2 CUs)), clamped to 6..16,
// consecutive column blocks (no CU takes a third turn; on the GPT-2 head 449
// workgroups of 7 waves: 15.2 us at M = 32 against 17.1 with one workgroup of
// 13 per CU and 20.7 with 9..12 waves, whose workgroups no longer fit twice),
// one block per wave over the full K, so the accumulators go straight to the
// epilogue (no reduction across waves) and A is read once per workgroup (the
// split-K GEMV re-reads all of A for every one or two column blocks: 1571
// workgroups x 48 KiB for the 38.6 MB GPT-2 head at M = 32).  A wave issues
// its share of the A copy, then its block's scale, bias and K chunks in K
// order (scheduling barriers hold the order: loads return in issue order and a
// wait names a count, not a load), so A lands first and goes to LDS while the
// weights stream, and chunk c is multiplied as soon as it has arrived.  EK is
// the epilogue kind.
struct WideParams {
  const uint16_t* a;    // P32 fragment-packed [32][K], or row-major [M][lda] (AP32 false)
  int64_t lda;
  const u32x4_t* w;     // panel-packed records
  const float* scales;  // fp32 [N]
  int m, n, nb, per;    // rows, columns, column blocks, blocks (waves) per workgroup
  Epilogue epi;
  float* amax_v;        // when set: per (workgroup, row) best logit and its column
  int32_t* amax_i;
};

constexpr int kWideWaves = 16, kWideMinWaves = 6;

template <int MT, int KC, int EK, bool AP32>
__global__ __launch_bounds__(kWideWaves * 64) void gemv_wide_kernel(WideParams p) {
  constexpr int W = kWideWaves;
  // A as MFMA fragments ((c * MT + t) * 2 + s) * 64 + lane: rows 16t + (lane & 15),
  // columns 64c + 32s + 8 (lane >> 4) .. + 7 (for MT = 2, the P32 layout).
  constexpr int kFrags = KC * MT * 2 * 64, kACopy = (kFrags + kWideMinWaves * 64 - 1) / (kWideMinWaves * 64);
  static_assert(AP32 ? MT == 2 : true, "P32 A holds 32 rows");
  const int nt = blockDim.x;  // p.per waves, kWideMinWaves <= p.per <= W
  __shared__ half8_t a_lds[kFrags];
  __shared__ float sv[W][32];
  __shared__ int si[W][32];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int cb = blockIdx.x * p.per + wave;
  // The last workgroup's waves past the last block load that block again
  // (the second request finds the first's lines); their sums are never stored.
  const int cbl = min(cb, p.nb - 1), col = cb * 16 + j, colc = min(cbl * 16 + j, p.n - 1);
  const bool active = cb < p.nb;
  const bool has_bias = EK != EPI_RAW_F32 && p.epi.bias;

  half8_t ar[kACopy];
#pragma unroll
  for (int i = 0; i < kACopy; ++i) {
    const int f = min(i * nt + int(threadIdx.x), kFrags - 1);  // fragment f / 64, lane f % 64
    if constexpr (AP32) {
      ar[i] = reinterpret_cast<const half8_t*>(p.a)[f];
    } else {
      // Rows past M repeat row M - 1 (their sums are never stored).
      const int fl = f & 63, frag = f >> 6, s2 = frag & 1, t = (frag >> 1) % MT, c = (frag >> 1) / MT;
      const int row = min(16 * t + (fl & 15), p.m - 1), acol = 64 * c + 32 * s2 + 8 * (fl >> 4);
      ar[i] = *reinterpret_cast<const half8_t*>(p.a + int64_t(row) * p.lda + acol);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  const float scale = p.scales[colc];
  const uint16_t bias_raw = ldg_u16(has_bias ? p.epi.bias + colc : p.a);
  u32x4_t wr[KC];
  const u32x4_t* wb = p.w + int64_t(cbl) * KC * 64 + lane;
#pragma unroll
  for (int c = 0; c < KC; ++c) {
    __builtin_amdgcn_sched_barrier(0);
    wr[c] = __builtin_nontemporal_load(wb + c * 64);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < kACopy; ++i)  // clamped like the loads: a repeated index stores the same value
    a_lds[min(i * nt + int(threadIdx.x), kFrags - 1)] = ar[i];
  __syncthreads();

  // Four sums, chunk c into sum c % 4, added in that order at the end: the K
  // order of the 4-wave packed GEMV over the same KC (wave w takes chunks w,
  // w + 4, ...; the waves are added in order), which serves 1..16 rows, so a
  // row's logits do not depend on the batch size.
  float4_t acc[4][MT];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[q][t] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < KC; ++c) {
    const half8_t b0 = dequant8(wr[c][0], wr[c][1], scale);
    const half8_t b1 = dequant8(wr[c][2], wr[c][3], scale);
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      float4_t& ac = acc[c % 4][t];
      ac = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_lds[((c * MT + t) * 2) * 64 + lane], b0, ac, 0, 0, 0);
      ac = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_lds[((c * MT + t) * 2 + 1) * 64 + lane], b1, ac, 0, 0, 0);
    }
    // One chunk's LDS reads and dequantisation at a time.
    __builtin_amdgcn_sched_barrier(0);
  }
  const float bias = has_bias ? h2f(bias_raw) : 0.f;
  float vals[MT * 4];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float sum = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) sum += acc[q][t][v];
      vals[t * 4 + v] = sum;
    }
  if (active && col < p.n) {
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * t + 4 * g + v;
        if (row >= p.m) continue;
        const float sum = vals[t * 4 + v];
        if constexpr (EK == EPI_F32) {
          static_cast<float*>(p.epi.y)[int64_t(row) * p.epi.ldy + col] = sum + bias;
        } else if constexpr (EK == EPI_GELU) {
          static_cast<uint16_t*>(p.epi.y)[int64_t(row) * p.epi.ldy + col] = f2h(gelu_tanh(rt16(sum + bias)));
        } else if constexpr (EK == EPI_RESIDUAL) {
          const float r = h2f(p.epi.residual[int64_t(row) * p.epi.ldr + col]);
          static_cast<uint16_t*>(p.epi.y)[int64_t(row) * p.epi.ldy + col] = f2h(r + rt16(sum + bias));
        } else {
          static_cast<uint16_t*>(p.epi.y)[int64_t(row) * p.epi.ldy + col] = f2h(sum + bias);
        }
      }
  }
  if constexpr (EK == EPI_F32) {
    if (!p.amax_v) return;
    // Argmax partials: across the 16 column lanes of each row, then across the
    // waves (blocks in column order) through LDS; one (value, column) per row
    // per workgroup, the lowest column on ties.
    const bool live = active && col < p.n;
#pragma unroll
    for (int r = 0; r < MT * 4; ++r) {
      float bv = live ? vals[r] + bias : -__builtin_huge_valf();
      int bi = live ? col : INT_MAX;
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) amax_merge(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
      if (j == 0) {
        sv[wave][16 * (r >> 2) + 4 * g + (r & 3)] = bv;
        si[wave][16 * (r >> 2) + 4 * g + (r & 3)] = bi;
      }
    }
    __syncthreads();
    if (threadIdx.x < 32 && int(threadIdx.x) < p.m) {
      float v = sv[0][threadIdx.x];
      int i = si[0][threadIdx.x];
#pragma unroll
      for (int w = 1; w < W; ++w)
        if (w < p.per) amax_merge(v, i, sv[w][threadIdx.x], si[w][threadIdx.x]);
      p.amax_v[threadIdx.x * gridDim.x + blockIdx.x] = v;
      p.amax_i[threadIdx.x * gridDim.x + blockIdx.x] = i;
    }
  }
}

// Greedy id of each row from the wide GEMV's per-workgroup partials: one wave
// per row, lanes stride over the groups, same tie rule.
__global__ __launch_bounds__(64) void argmax_partials_kernel(const float* vals, const int32_t* idx, int groups,
                                                            int32_t* out) {
  const int row = blockIdx.x, lane = threadIdx.x;
  float v = -__builtin_huge_valf();
  int i = INT_MAX;
  for (int gi = lane; gi < groups; gi += 64) amax_merge(v, i, vals[row * groups + gi], idx[row * groups + gi]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) amax_merge(v, i, __shfl_xor(v, o, 64), __shfl_xor(i, o, 64));
  if (lane == 0) out[row] = i;
}

// ---------------------------------------------------------------------------
// Multistage MFMA GEMM over panel-packed weights (prefill, M > 32)
// ---------------------------------------------------------------------------
// Tile BM x BN = (WM * MT * 16) x (WN * R * 16), 4 waves as WM x WN, K in chunks of
// 64.  Every operand moves HBM/L2 -> LDS with global_load_lds_dwordx4 (no
// registers), one 1 KiB wave instruction per A fragment (16 rows x 32 K, lanes
// in MFMA A order) and per packed weight record (already in MFMA B order), so
// each wave later reads its operands with conflict-free ds_read_b128 at
// lane * 16.  S LDS stages: while chunk c is multiplied, chunks c+1 .. c+S-2
// are in flight and c+S-1 is being issued.  Per chunk: wait for this wave's
// loads of chunk c (vmcnt), barrier (everyone's loads of c landed and everyone
// finished chunk c-1), issue chunk c+S-1 into the stage of c-1, compute c.
using global_ptr = const void __attribute__((address_space(1)))*;
using lds_ptr = void __attribute__((address_space(3)))*;

struct PanelParams {
  const uint16_t* a;
  int64_t lda;
  const u32x4_t* w;     // panel-packed records
  const float* scales;  // fp32 [N]
  int m, n, k;
  int nb, kc;           // column blocks, K chunks
  int tiles_n, tiles;   // tiles per row of tiles, tiles per split
  int group_m;          // tile rows per group of the tile order
  int chunks_per_split, splits;
  bool defer;
  bool pool;            // splits > 1 finish in this launch through the queue pool
  Epilogue epi;
  float* partials;      // [splits][M][N] when splits > 1 or defer
};

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// Wait until at most `outstanding` chunks of this wave's loads (LPW each) are in
// flight: vmcnt needs an immediate, so the uniform count selects one of MAX + 1.
template <int LPW, int I, int MAX>
__device__ __forceinline__ void wait_chunk(int outstanding) {
  if constexpr (I >= MAX) {
    wait_vmcnt<MAX * LPW>();
  } else {
    if (outstanding <= I) {
      wait_vmcnt<I * LPW>();
      return;
    }
    wait_chunk<LPW, I + 1, MAX>(outstanding);
  }
}

// Row pitch (floats) of the fp32 tiles the MFMA GEMMs stage their sums in for
// the epilogue: rows stay 16-byte aligned, and the accumulator stores (lane
// (j, g) of a 16-column block writes rows 4g + v, column j) hit 64 distinct
// banks.
constexpr int tile_pitch(int bn) { return bn + 4; }

// In-launch split-K finish of a TR x BN fp32 tile staged in LDS at pitch
// tile_pitch(BN), in tile_epilogue's thread mapping (thread t holds RPT
// float4s: columns 4 (t % (BN / 4)) .. + 3 of tile rows t / (BN / 4) + i RS).
// This split's float4s go to the queue's pool slot, tile-contiguous in the
// threads' own order (float4 i of thread t of split s at ((tile splits + s)
// RPT + i) NT + t), so every store and load is a coalesced 16-byte access; the
// last split of the tile to arrive loads every split's float4s in one round
// (splits <= pool_max_splits(RPT)), adds them in split order back into the
// LDS tile and returns true, and the caller then runs tile_epilogue on it;
// every other workgroup returns false.
template <int TR, int BN, int NT>
__device__ bool tile_split_finish(float* ctile, int split, int splits, int tile) {
  constexpr int CG = BN / 4, RS = NT / CG, RPT = TR / RS, SMAX = pool_max_splits(RPT);
  static_assert(SMAX >= 1, "a finishing thread's float4s fit one round of loads");
  // (splits <= kTileRounds * SMAX: the finish takes up to kTileRounds rounds.)
  const int t = int(threadIdx.x), c4 = t % CG, rl0 = t / CG;
  const PoolSlot slot = gemm_pool_slot();
  const auto rs = agent_rsrc(slot.parts, uint32_t(kPoolFloats * sizeof(float)));
  auto off = [&](int sp, int i) { return uint32_t(((int64_t(tile) * splits + sp) * RPT + i) * NT + t) * 16u; };
#pragma unroll
  for (int i = 0; i < RPT; ++i)
    st_agent4(rs, off(split, i), *reinterpret_cast<const f32x4_t*>(ctile + (rl0 + i * RS) * tile_pitch(BN) + 4 * c4));
  if (!wg_arrive_last(slot.ctr + tile * kCounterStride, splits)) return false;
  f32x4_t acc[RPT];
  for (int r0 = 0; r0 < splits; r0 += SMAX) {
    f32x4_t v[RPT][SMAX];
#pragma unroll
    for (int i = 0; i < RPT; ++i)
#pragma unroll
      for (int sp = 0; sp < SMAX; ++sp) v[i][sp] = r0 + sp < splits ? ld_agent4(rs, off(r0 + sp, i)) : f32x4_t{};
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      if (r0 == 0) acc[i] = v[i][0];
      else acc[i] += v[i][0];
#pragma unroll
      for (int sp = 1; sp < SMAX; ++sp)
        if (r0 + sp < splits) acc[i] += v[i][sp];
    }
  }
#pragma unroll
  for (int i = 0; i < RPT; ++i) *reinterpret_cast<f32x4_t*>(ctile + (rl0 + i * RS) * tile_pitch(BN) + 4 * c4) = acc[i];
  depart(slot.ctr + tile * kCounterStride);
  return true;
}

// The 4 bias values of columns col .. col + 3 (0 past N or without a bias),
// loaded early: used only by the tile epilogue.  Without a bias the loads
// read `any`, a valid fp16 address (A's first element), and are discarded.
__device__ __forceinline__ void load_bias4(const Epilogue& e, int col, int n, const uint16_t* any,
                                           float (&bias)[4]) {
  const bool has = e.kind != EPI_RAW_F32 && e.bias;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const uint16_t raw = ldg_u16(has ? e.bias + min(col + c, n - 1) : any);
    bias[c] = has && col + c < n ? h2f(raw) : 0.f;
  }
}

// Epilogue of TR rows x BN columns of fp32 sums staged in LDS at pitch
// tile_pitch(BN): thread t of NT takes columns col = n0 + 4 (t % (BN / 4))
// .. + 3 (its bias4) of tile rows t / (BN / 4) + i NT / (BN / 4), tile row 0
// being output row r0.  The epilogue kind is switched once, outside the
// loops, so each kind runs straight-line code (a switch per element cost ~70
// VALU and ~20 scalar instructions per output); residuals are loaded before
// any result is computed; a group of 4 columns inside the matrix goes out as
// one 8-byte (fp16) or 16-byte (fp32) store when the layout allows it.
// partials != null: the raw sums go to partials[(split m + row) n + col]
// (split-K or a deferred finisher) instead.
template <int TR, int BN, int NT>
__device__ __forceinline__ void tile_epilogue(const Epilogue& e, const float* ctile, int r0, int n0, int m, int n,
                                              const float (&bias)[4], float* partials, int split) {
  constexpr int CG = BN / 4, RS = NT / CG, RPT = TR / RS;
  static_assert(NT % CG == 0 && TR % RS == 0 && RPT >= 1, "whole row groups per thread");
  const int c4 = int(threadIdx.x) % CG, rl0 = int(threadIdx.x) / CG;
  const int col = n0 + 4 * c4;
  if (col >= n) return;
  const bool full = col + 4 <= n;
  // Row i of this thread: output row r0 + rl0 + i RS, its 4 sums from LDS.
  auto row_of = [&](int i) { return r0 + rl0 + i * RS; };
  auto sums = [&](int i) {
    return *reinterpret_cast<const float4_t*>(ctile + (rl0 + i * RS) * tile_pitch(BN) + 4 * c4);
  };
  auto aligned = [](const void* ptr, int bytes) { return reinterpret_cast<uintptr_t>(ptr) % bytes == 0; };
  // fp32 rows at base + row * ld (+ col): one 16-byte store per row when it can.
  auto store_f32 = [&](float* base, int64_t ld, auto&& f) {
    const bool vec = full && ld % 4 == 0 && aligned(base, 16);
#pragma unroll 1
    for (int i = 0; i < RPT; ++i) {
      const int row = row_of(i);
      if (row >= m) break;
      const float4_t v = sums(i);
      float* dst = base + int64_t(row) * ld + col;
      if (vec) {
        *reinterpret_cast<float4_t*>(dst) = float4_t{f(v[0], 0), f(v[1], 1), f(v[2], 2), f(v[3], 3)};
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (col + c < n) dst[c] = f(v[c], c);
      }
    }
  };
  if (partials) {
    store_f32(partials + int64_t(split) * m * n, n, [](float x, int) { return x; });
    return;
  }
  switch (e.kind) {
    case EPI_RAW_F32:
      store_f32(static_cast<float*>(e.y), e.ldy, [](float x, int) { return x; });
      return;
    case EPI_F32:
      store_f32(static_cast<float*>(e.y), e.ldy, [&](float x, int c) { return x + bias[c]; });
      return;
    case EPI_QKV: {
      // Per row: the request, its token and cache position once; a full
      // 4-column group (one head: hidden % 64 == 0) goes to y and, for a K or
      // V column of a real token, to the slot cache as one 8-byte store each.
      uint16_t* y = static_cast<uint16_t*>(e.y);
      const bool vec = full && e.ldy % 4 == 0 && aligned(y, 8) && aligned(e.kcache, 8) && aligned(e.vcache, 8) &&
                       e.hidden % 64 == 0;
#pragma unroll 1
      for (int i = 0; i < RPT; ++i) {
        const int row = row_of(i);
        if (row >= m) break;
        const float4_t v = sums(i);
        int rb, rt;
        qkv_row(e, row, rb, rt);
        if (!vec) {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (col + c < n) qkv_store_bt(e, rb, rt, row, col + c, v[c] + bias[c]);
          continue;
        }
        const half4_t h4 = {f16r(v[0] + bias[0]), f16r(v[1] + bias[1]), f16r(v[2] + bias[2]), f16r(v[3] + bias[3])};
        *reinterpret_cast<half4_t*>(y + int64_t(row) * e.ldy + col) = h4;
        if (col >= e.hidden && rt < e.qlens[rb]) {
          const int part = col >= 2 * e.hidden ? 2 : 1;
          const int c = col - part * e.hidden, hd = c >> 6, d = c & 63;
          const int64_t pos = int64_t(e.offsets[rb]) + rt;
          const int64_t idx =
              (((int64_t(e.slots[rb]) * e.layers + e.layer) * e.heads + hd) * e.capacity + pos) * 64 + d;
          *reinterpret_cast<half4_t*>((part == 1 ? e.kcache : e.vcache) + idx) = h4;
        }
      }
      return;
    }
    default:
      break;
  }
  // fp16 outputs (EPI_F16, EPI_GELU, EPI_RESIDUAL), row-major or P32: the 4
  // columns col .. col + 3 (col % 4 == 0) of a row are contiguous in both
  // layouts, at y_off(row, col) + c.
  uint16_t* y = static_cast<uint16_t*>(e.y);
  const bool vec = full && (e.p32 || e.ldy % 4 == 0) && aligned(y, 8);
  auto store_f16 = [&](int row, float o0, float o1, float o2, float o3) {
    uint16_t* dst = y + y_off(e, row, col);
    if (vec) {
      *reinterpret_cast<half4_t*>(dst) = half4_t{f16r(o0), f16r(o1), f16r(o2), f16r(o3)};
    } else {
      const float o[4] = {o0, o1, o2, o3};
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (col + c < n) dst[c] = f2h(o[c]);
    }
  };
  if (e.kind == EPI_RESIDUAL) {
    // Every residual of the thread in flight before the first result.
    const bool rvec = full && (e.p32 || e.ldr % 4 == 0) && aligned(e.residual, 8);
    half4_t rs[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const uint16_t* src = e.residual + r_off(e, min(row_of(i), m - 1), col);
      if (rvec) {
        rs[i] = *reinterpret_cast<const half4_t*>(src);
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) rs[i][c] = __builtin_bit_cast(f16, src[min(c, n - 1 - col)]);
      }
    }
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int row = row_of(i);
      if (row >= m) break;
      const float4_t v = sums(i);
      float o[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] = float(rs[i][c]) + rt16(v[c] + bias[c]);
      store_f16(row, o[0], o[1], o[2], o[3]);
    }
    return;
  }
  auto rows_f16 = [&](auto&& f) {
#pragma unroll 1
    for (int i = 0; i < RPT; ++i) {
      const int row = row_of(i);
      if (row >= m) break;
      const float4_t v = sums(i);
      store_f16(row, f(v[0], 0), f(v[1], 1), f(v[2], 2), f(v[3], 3));
    }
  };
  if (e.kind == EPI_GELU) rows_f16([&](float x, int c) { return gelu_tanh(rt16(x + bias[c])); });
  else rows_f16([&](float x, int c) { return x + bias[c]; });
}

// Workgroup -> (split, tile row, tile column).  Workgroups are dispatched to
// the 8 XCDs round-robin by id, so ids are first regrouped into 8 contiguous
// runs (one per XCD); within a split, tiles are walked in groups of GM tile
// rows, column by column, so the workgroups one XCD runs together share GM
// A row panels and a few weight column panels in that XCD's L2 instead of
// each streaming every weight column panel (gm_max = 1: row-major order).
__device__ __forceinline__ void tile_of_block(int gm_max, int tiles_n, int tiles, int& split, int& tm, int& tn) {
  const int nbk = gridDim.x, bid = blockIdx.x;
  const int logical = (nbk % 8 == 0) ? (bid % 8) * (nbk / 8) + bid / 8 : bid;
  const int tile = logical % tiles, tiles_m = tiles / tiles_n;
  split = logical / tiles;
  const int per_group = gm_max * tiles_n, group = tile / per_group, first = group * gm_max;
  const int gm = min(tiles_m - first, gm_max), r = tile - group * per_group;
  tm = first + r % gm;
  tn = r / gm;
}

template <int WM, int WN, int MT, int R, int S, bool POOL = false>
__global__ __launch_bounds__(256) void panel_gemm_kernel(PanelParams p) {
  constexpr int BM = WM * MT * 16, BN = WN * R * 16;
  constexpr int NA = (BM / 16) * 2, NB = BN / 16, NL = NA + NB;
  static_assert(NL % 4 == 0, "loads must split evenly over the waves");
  constexpr int LPW = NL / 4;
  constexpr int STAGE = NL * 1024;
  static_assert(WM * WN == 4 && S >= 3 && (S - 2) * LPW < 64, "4 waves; in-flight loads within vmcnt");
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];  // S * STAGE bytes

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int wm = wave / WN, wn = wave % WN;
  int split, tm, tn;
  tile_of_block(p.group_m, p.tiles_n, p.tiles, split, tm, tn);
  const int m0 = tm * BM, cb0 = tn * NB;
  const int c_begin = split * p.chunks_per_split;
  const int kc = min(p.kc - c_begin, p.chunks_per_split);  // chunks of this split (>= 1)

  // This wave's LPW loads per chunk: load id < NA is A fragment (t, s) = (id/2,
  // id%2): lane (j, g) reads row m0 + 16t + j (clamped), k = 64c + 32s + 8g;
  // otherwise packed record cb0 + id - NA (clamped): lane reads its 16 bytes.
  const char* src[LPW];
  int stride[LPW];
#pragma unroll
  for (int l = 0; l < LPW; ++l) {
    const int id = wave * LPW + l;
    if (id < NA) {
      const int t = id >> 1, s = id & 1;
      const int row = min(m0 + 16 * t + j, p.m - 1);
      src[l] = reinterpret_cast<const char*>(p.a + int64_t(row) * p.lda + 64 * c_begin + 32 * s + 8 * g);
      stride[l] = 128;
    } else {
      const int cb = min(cb0 + id - NA, p.nb - 1);
      src[l] = reinterpret_cast<const char*>(p.w + (int64_t(cb) * p.kc + c_begin) * 64 + lane);
      stride[l] = 1024;
    }
  }
  auto issue = [&](int chunk, int stage) {
#pragma unroll
    for (int l = 0; l < LPW; ++l)
      __builtin_amdgcn_global_load_lds((global_ptr)(src[l] + int64_t(chunk) * stride[l]),
                                       (lds_ptr)(lds + stage * STAGE + (wave * LPW + l) * 1024), 16, 0, 0);
  };

  // The tile's BN fp32 scales reach LDS (past the stages) by the same DMA path
  // (4-byte elements land at lane * 4), issued by wave 0 before its chunk-0
  // loads, so the chunk-0 wait and barrier cover them: nothing loaded into a
  // register is used in the loop (the compiler would otherwise wait for every
  // prologue load up front).  The bias is loaded into registers now and used
  // only after the loop; a null bias reads A's first element, scaled by 0.
  static_assert(BN % 64 == 0 && BN / 64 <= 4, "one 64-lane scale load per 64 columns");
  const float* scale_lds = reinterpret_cast<const float*>(lds + S * STAGE);
  if (wave < BN / 64)
    __builtin_amdgcn_global_load_lds((global_ptr)(p.scales + min(cb0 * 16 + 64 * wave + lane, p.n - 1)),
                                     (lds_ptr)(lds + S * STAGE + 256 * wave), 4, 0, 0);
  // The epilogue gives thread t columns 4 (t % (BN / 4)) .. + 3 of the tile:
  // their bias is loaded now (used only after the loop).
  const bool epi_now = p.splits == 1 && !p.defer;
  float bias[4];
  load_bias4(p.epi, cb0 * 16 + 4 * int(threadIdx.x % (BN / 4)), p.n, p.a, bias);
  float4_t acc[MT][R];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[t][r] = float4_t{0.f, 0.f, 0.f, 0.f};

  // Prologue: chunks 0 .. S-2 (a split shorter than that re-reads its last chunk
  // into stages it never uses; the waits below stay conservative).
#pragma unroll
  for (int c = 0; c < S - 1; ++c) issue(min(c, kc - 1), c);
  for (int c = 0; c < kc; ++c) {
    wait_chunk<LPW, 0, S - 2>(min(c + S - 2, kc - 1) - c);
    __builtin_amdgcn_s_barrier();
    if (c + S - 1 < kc) issue(c + S - 1, (c + S - 1) % S);
    const uint8_t* st = lds + (c % S) * STAGE;
    // Every LDS read of the chunk is issued first (scales and records, then
    // the A fragments; LDS reads return in order, so each use waits for its
    // own read only): the dequantisation runs while the A fragments arrive.
    float sc[R];
    u32x4_t raw[R];
    half8_t af[MT][2];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      sc[r] = scale_lds[(wn * R + r) * 16 + j];
      raw[r] = *reinterpret_cast<const u32x4_t*>(st + (NA + wn * R + r) * 1024 + lane * 16);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int s = 0; s < 2; ++s)
        af[t][s] = *reinterpret_cast<const half8_t*>(st + (((wm * MT + t) * 2 + s) * 1024) + lane * 16);
    __builtin_amdgcn_sched_barrier(0);
    half8_t bq[R][2];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      bq[r][0] = dequant8(raw[r][0], raw[r][1], sc[r]);
      bq[r][1] = dequant8(raw[r][2], raw[r][3], sc[r]);
    }
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int r = 0; r < R; ++r)
          acc[t][r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t][s], bq[r][s], acc[t][r], 0, 0, 0);
  }
  wait_vmcnt<0>();

  // Epilogue through LDS (the stages are free once every wave is past the last
  // chunk): the accumulators land in a BM x BN fp32 tile, which tile_epilogue
  // finishes 4 columns per thread.
  static_assert(BM * tile_pitch(BN) * 4 <= S * STAGE, "fp32 tile fits the stages");
  __syncthreads();
  float* ctile = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        ctile[((wm * MT + t) * 16 + 4 * g + v) * tile_pitch(BN) + (wn * R + r) * 16 + j] = acc[t][r][v];
  __syncthreads();
  if (POOL && p.splits > 1) {
    if (tile_split_finish<BM, BN, 256>(ctile, split, p.splits, tm * p.tiles_n + tn))
      tile_epilogue<BM, BN, 256>(p.epi, ctile, m0, cb0 * 16, p.m, p.n, bias, nullptr, split);
    return;
  }
  tile_epilogue<BM, BN, 256>(p.epi, ctile, m0, cb0 * 16, p.m, p.n, bias, epi_now ? nullptr : p.partials, split);
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
  // Split-K (gridDim.z > 1): split z takes K steps [z * steps_per_split, ...)
  // and stores raw fp32 sums at partials[(z * m + row) * n + col], or with
  // `pool` in the queue pool slot, finished by the tile's last split.
  int steps_per_split;
  float* partials;
  bool pool;
};
constexpr int TBM = 64, TBN = 64, TBK = 32, TPAD = 40;  // LDS row pitch in halves

template <bool INT8, bool WVEC, bool AVEC, bool POOL = false>
__global__ __launch_bounds__(256) void tiled_kernel(TiledParams p) {
  // A and W^T double buffers; after the K loop the same bytes hold the fp32
  // output tile for the epilogue.
  constexpr size_t kStage = size_t(2) * (TBM + TBN) * TPAD * sizeof(f16);
  constexpr size_t kTile = size_t(TBM) * tile_pitch(TBN) * sizeof(float);
  __shared__ __attribute__((aligned(16))) uint8_t smem[kStage > kTile ? kStage : kTile];
  auto As = reinterpret_cast<f16(*)[TBM][TPAD]>(smem);
  auto Bs = reinterpret_cast<f16(*)[TBN][TPAD]>(smem + size_t(2) * TBM * TPAD * sizeof(f16));  // transposed: [n][k]
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

  // Staged K step: the A fragment and the raw W bytes (int8: 4 per K row,
  // fp16: 4 halves in two words), dequantised only when stored to LDS, so a
  // step's loads stay in flight while earlier steps compute.
  struct Staged {
    half8_t a;
    uint32_t w[2][2];
  };
  auto load_global = [&](Staged& r_, int k0) {
    r_.a = afrag<AVEC>(p.a, p.lda, p.m, p.k, m0 + a_row, k0 + a_kseg);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int k = k0 + w_kr + r, col = n0 + w_c4;
      uint32_t lo = 0, hi = 0;
      if (k < p.k) {
        if constexpr (INT8) {
          const int8_t* wp = static_cast<const int8_t*>(p.w) + int64_t(k) * p.ldw + col;
          if (WVEC && col < p.n) {
            lo = *reinterpret_cast<const uint32_t*>(wp);
          } else if (!WVEC) {
#pragma unroll
            for (int c = 0; c < 4; ++c)
              if (col + c < p.n) lo |= uint32_t(uint8_t(wp[c])) << (8 * c);
          }
        } else {
          const uint16_t* wp = static_cast<const uint16_t*>(p.w) + int64_t(k) * p.ldw + col;
          if (WVEC && col < p.n) {
            const uint2 u = *reinterpret_cast<const uint2*>(wp);
            lo = u.x;
            hi = u.y;
          } else if (!WVEC) {
#pragma unroll
            for (int c = 0; c < 4; ++c)
              if (col + c < p.n) (c < 2 ? lo : hi) |= uint32_t(wp[c]) << (16 * (c & 1));
          }
        }
      }
      r_.w[r][0] = lo;
      r_.w[r][1] = hi;
    }
  };
  auto store_lds = [&](const Staged& r_, int s) {
    *reinterpret_cast<half8_t*>(&As[s][a_row][a_kseg]) = r_.a;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      half2_t pair;
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        if constexpr (INT8) pair[r] = f16r(float(int8_t(r_.w[r][0] >> (8 * c))) * sc[c]);
        else pair[r] = __builtin_bit_cast(f16, uint16_t(r_.w[r][c >> 1] >> (16 * (c & 1))));
      }
      *reinterpret_cast<half2_t*>(&Bs[s][w_c4 + c][w_kr]) = pair;
    }
  };

  // The epilogue gives thread t columns n0 + 4 (t % 16) .. + 3: their bias now.
  float bias[4];
  load_bias4(p.epi, n0 + 4 * (tid % (TBN / 4)), p.n, p.a, bias);
  float4_t acc[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int c = 0; c < 2; ++c) acc[t][c] = float4_t{0.f, 0.f, 0.f, 0.f};

  const int steps = (p.k + TBK - 1) / TBK;
  const int split = int(blockIdx.z);
  const int st0 = split * p.steps_per_split, nst = min(steps, st0 + p.steps_per_split) - st0;
  // Local step i's data lives in register set i % 3: steps i + 1 .. i + 3 are
  // in flight while step i computes from LDS buffer i & 1.
  Staged s0, s1, s2;
  load_global(s0, st0 * TBK);
  if (nst > 1) load_global(s1, (st0 + 1) * TBK);
  if (nst > 2) load_global(s2, (st0 + 2) * TBK);
  store_lds(s0, 0);
  __syncthreads();
  if (nst > 3) load_global(s0, (st0 + 3) * TBK);
  auto step = [&](int i, Staged& nxt) {
    const int cur = i & 1;
    half8_t af[2], bf[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) af[t] = *reinterpret_cast<const half8_t*>(&As[cur][wm * 32 + 16 * t + j][8 * g]);
#pragma unroll
    for (int c = 0; c < 2; ++c) bf[c] = *reinterpret_cast<const half8_t*>(&Bs[cur][wn * 32 + 16 * c + j][8 * g]);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int c = 0; c < 2; ++c) acc[t][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t], bf[c], acc[t][c], 0, 0, 0);
    if (i + 1 < nst) {
      store_lds(nxt, cur ^ 1);
      __syncthreads();
    }
    if (i + 4 < nst) load_global(nxt, (st0 + i + 4) * TBK);
  };
  for (int i = 0; i < nst; i += 3) {
    step(i, s1);
    if (i + 1 < nst) step(i + 1, s2);
    if (i + 2 < nst) step(i + 2, s0);
  }
  // Every wave is past its last LDS read before the tile overwrites the stages.
  __syncthreads();
  float* ctile = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        ctile[(wm * 32 + 16 * t + 4 * g + v) * tile_pitch(TBN) + wn * 32 + 16 * c + j] = acc[t][c][v];
  __syncthreads();
  if (POOL && gridDim.z > 1) {
    if (tile_split_finish<TBM, TBN, 256>(ctile, split, int(gridDim.z), int(blockIdx.x + gridDim.x * blockIdx.y)))
      tile_epilogue<TBM, TBN, 256>(p.epi, ctile, m0, n0, p.m, p.n, bias, nullptr, split);
    return;
  }
  tile_epilogue<TBM, TBN, 256>(p.epi, ctile, m0, n0, p.m, p.n, bias, gridDim.z > 1 ? p.partials : nullptr, split);
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

// The three FP32 GEMM variants of the legacy ABI's benchmark hook (the
// reference's naive / shared-memory tiled / register-tiled kernels,
// kernels/src/cuda/matmul.cu:7-80, chosen by bench_api.cu:43-51's variant).
// Every variant sums k in increasing order for each output.
// Variant 0: one thread per output, operands straight from global memory.
__global__ __launch_bounds__(256) void legacy_f32_naive_kernel(const float* a, const float* b, float* c, int m,
                                                               int n, int k) {
  const int64_t col = int64_t(blockIdx.x) * 16 + (threadIdx.x & 15);
  const int64_t row = int64_t(blockIdx.y) * 16 + (threadIdx.x >> 4);
  if (row >= m || col >= n) return;
  float acc = 0.f;
  for (int64_t kk = 0; kk < k; ++kk) acc += a[row * k + kk] * b[kk * n + col];
  c[row * n + col] = acc;
}

// Variant 1: 16x16 output tile per 256-thread block, one output per thread,
// A and B staged through LDS in 16-wide K slabs.
__global__ __launch_bounds__(256) void legacy_f32_tiled_kernel(const float* a, const float* b, float* c, int m,
                                                               int n, int k) {
  __shared__ float As[16][17];
  __shared__ float Bs[16][17];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t row = int64_t(blockIdx.y) * 16 + ty, col = int64_t(blockIdx.x) * 16 + tx;
  float acc = 0.f;
  for (int64_t k0 = 0; k0 < k; k0 += 16) {
    As[ty][tx] = (row < m && k0 + tx < k) ? a[row * k + k0 + tx] : 0.f;
    Bs[ty][tx] = (k0 + ty < k && col < n) ? b[(k0 + ty) * n + col] : 0.f;
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) acc += As[ty][kk] * Bs[kk][tx];
    __syncthreads();
  }
  if (row < m && col < n) c[row * n + col] = acc;
}

// Variant 2 (ti_cuda_gemm, ti_v2_legacy_gemm_f32): 64x64 output tile per
// 256-thread block, 4x4 outputs per thread, K in 16-wide LDS slabs.
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
// Number of K splits of the row-major M <= 32 kernel: aim for ~2 workgroups
// per CU (a 2.4 MB GEMV is latency-bound, so every CU should have loads in
// flight), with the fp32 partials (splits * M * N * 4 bytes, L2/MALL traffic)
// at most twice the weight bytes and within `capacity` floats (0: no scratch,
// one split).  Returns the split count after rounding to whole step ranges.
int skinny_splits(int m, int n, int k, size_t capacity) {
  const int ntile = (n + 63) / 64, steps = (k + 31) / 32;
  int splits = 1;
  if (capacity > 0) {
    const int target = (2 * 256 + ntile - 1) / ntile;
    const int max_by_traffic = std::max(1, k / (2 * std::max(1, m)));
    splits = std::max(1, std::min(target, std::min(steps, max_by_traffic)));
    while (splits > 1 && size_t(splits) * m * n > capacity) --splits;
  }
  const int spb = (steps + splits - 1) / splits;
  return (steps + spb - 1) / spb;
}

// Plan of rowgemv_kernel: about 192 workgroups (a 2.4 MB GEMV is latency-bound:
// one round of loads per wave over most CUs, each workgroup reading a few
// hundred weight rows), K split into equal whole-step ranges of at most
// 4 x 16 steps; 8 waves when a split has at most 8 steps, else 16.  Depends
// on N and K only.  hipErrorNotSupported when the shape does not fit (more
// than kRowSplits splits, or partials beyond the pool): the caller then takes
// the skinny kernel.
constexpr int kRowTargetBlocks = 192;
template <int W, int S>
hipError_t launch_rowgemv_ws(const SkinnyParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((rowgemv_kernel<W, S>), dim3(unsigned(p.ntile) * unsigned(p.splits)), dim3(W * 64), 0, stream, p);
  return hipGetLastError();
}
hipError_t launch_rowgemv(const GemmArgs& g, hipStream_t stream) {
  SkinnyParams p{};
  p.a = g.a; p.lda = g.lda; p.w = g.w; p.scales = g.scales;
  p.m = g.m; p.n = g.n; p.k = g.k; p.epi = g.epi;
  p.ldw = g.ldw > 0 ? g.ldw : g.n;
  p.ntile = (g.n + 63) / 64;
  p.steps = (g.k + 31) / 32;
  int splits = std::clamp((kRowTargetBlocks + p.ntile / 2) / p.ntile, 1, kRowSplits);
  splits = std::max(splits, (p.steps + 63) / 64);
  if (splits > kRowSplits) return hipErrorNotSupported;
  const int spb = (p.steps + splits - 1) / splits;
  splits = (p.steps + spb - 1) / spb;
  if (splits > 1 && (p.ntile > kPoolTiles || int64_t(p.ntile) * splits * 1024 > int64_t(kPoolFloats)))
    return hipErrorNotSupported;
  p.steps_per_block = spb;
  p.splits = splits;
  p.pool = splits > 1;
  if (spb <= 8) return launch_rowgemv_ws<8, 1>(p, stream);
  if (spb <= 16) return launch_rowgemv_ws<16, 1>(p, stream);
  if (spb <= 32) return launch_rowgemv_ws<16, 2>(p, stream);
  return launch_rowgemv_ws<16, 4>(p, stream);
}

// Plan of rowgemm_kernel (16 < M <= kRowMaxM): rows in blocks of 16 up to
// M = 64, then 32 (timed, configs[1] row-major shapes: M = 40 / 64 768->3072
// 7.7 / 7.8 us in 16-row blocks against 8.5 / 8.8 in 32-row ones, M = 512
// 24.4 against 16.2 us; 64-row blocks, four waves, lost everywhere: M = 64
// 14.3, M = 512 18.5 us); about 192 workgroups as above, K split within the
// finisher's one round of loads and the pool slot; 8 waves, 16 once a split
// of 16-row blocks has more than 8 steps; S steps a round, rounds repeated
// over longer splits.
constexpr int kRowMaxM = 1024;
template <int MT, int W, int S>
hipError_t launch_rowgemm_ws(const SkinnyParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((rowgemm_kernel<MT, W, S>), dim3(unsigned(p.ntile * p.rblocks * p.splits)), dim3(W * 64), 0,
                     stream, p);
  return hipGetLastError();
}
hipError_t launch_rowgemm(const GemmArgs& g, hipStream_t stream) {
  SkinnyParams p{};
  p.a = g.a; p.lda = g.lda; p.w = g.w; p.scales = g.scales;
  p.m = g.m; p.n = g.n; p.k = g.k; p.epi = g.epi;
  p.ldw = g.ldw > 0 ? g.ldw : g.n;
  p.ntile = (g.n + 63) / 64;
  p.steps = (g.k + 31) / 32;
  const int mt = g.m <= 64 ? 1 : 2;
  p.rblocks = (g.m + 16 * mt - 1) / (16 * mt);
  const int64_t units = int64_t(p.ntile) * p.rblocks;
  int splits = int(std::clamp<int64_t>((kRowTargetBlocks + units / 2) / units, 1, rowgemm_max_splits(mt, 8)));
  while (splits > 1 && units * splits * 16 * mt * 64 > int64_t(kPoolFloats)) --splits;
  if (splits > 1 && units > kPoolTiles) splits = 1;
  const int spb = (p.steps + splits - 1) / splits;
  splits = (p.steps + spb - 1) / spb;
  if (units * splits > INT_MAX / 2) return hipErrorNotSupported;
  p.steps_per_block = spb;
  p.splits = splits;
  p.pool = splits > 1;
  if (mt == 1) {
    if (spb <= 8) return launch_rowgemm_ws<1, 8, 1>(p, stream);
    if (spb <= 16) return launch_rowgemm_ws<1, 16, 1>(p, stream);
    if (spb <= 32) return launch_rowgemm_ws<1, 16, 2>(p, stream);
    return launch_rowgemm_ws<1, 16, 4>(p, stream);
  }
  if (spb <= 8) return launch_rowgemm_ws<2, 8, 1>(p, stream);
  if (spb <= 16) return launch_rowgemm_ws<2, 8, 2>(p, stream);
  return launch_rowgemm_ws<2, 8, 4>(p, stream);
}


// The skinny finisher spreads a tile's splits over its idle threads: rows
// below M of each 16-row pass take 16 threads each, and the 256 threads form
// skinny_groups(M) such groups, each summing a run of at most
// pool_max_splits(MT) splits.
int skinny_groups(int m) { return std::max(1, kSkinnyThreads / (16 * std::min(m, 16))); }
int skinny_pool_max_splits(int m, int mt) { return skinny_groups(m) * pool_max_splits(mt); }

template <bool INT8, int MT>
hipError_t launch_skinny(const GemmArgs& g, bool wvec, bool avec, const Scratch* s,
                         hipStream_t stream, int* deferred) {
  SkinnyParams p{};
  p.a = g.a; p.lda = g.lda; p.w = g.w; p.scales = g.scales;
  p.m = g.m; p.n = g.n; p.k = g.k; p.epi = g.epi;
  p.ldw = g.ldw > 0 ? g.ldw : g.n;
  p.ntile = (g.n + 63) / 64;
  p.steps = (g.k + 31) / 32;
  const bool pool = s && s->queue_pool && !deferred && p.ntile <= kPoolTiles;
  int splits = skinny_splits(g.m, g.n, g.k, pool ? kPoolFloats : (s && s->partials) ? s->partial_floats : 0);
  if (pool) splits = pool_splits(splits, p.ntile, int64_t(MT) * kSkinnyThreads * 4, skinny_pool_max_splits(g.m, MT), p.steps);
  const int spb = (p.steps + splits - 1) / splits;
  p.steps_per_block = spb;
  p.splits = splits;
  p.defer = deferred != nullptr;
  p.pool = pool;
  p.partials = s ? s->partials : nullptr;
  if (p.defer && (!p.partials || size_t(splits) * g.m * g.n > s->partial_floats)) return hipErrorInvalidValue;
  const dim3 grid(unsigned(p.ntile) * unsigned(splits));
#define TIA_SKINNY(WV, AV)                                                                                 \
  do {                                                                                                     \
    if (pool && splits > 1)                                                                                \
      hipLaunchKernelGGL((skinny_kernel<INT8, MT, WV, AV, true>), grid, dim3(kSkinnyThreads), 0, stream, p); \
    else                                                                                                   \
      hipLaunchKernelGGL((skinny_kernel<INT8, MT, WV, AV>), grid, dim3(kSkinnyThreads), 0, stream, p);       \
  } while (0)
  if (wvec && avec) TIA_SKINNY(true, true);
  else if (wvec) TIA_SKINNY(true, false);
  else if (avec) TIA_SKINNY(false, true);
  else TIA_SKINNY(false, false);
#undef TIA_SKINNY
  if (p.defer) {
    *deferred = splits;
    return hipGetLastError();
  }
  if (splits > 1 && !pool) {
    const int64_t total = int64_t(g.m) * g.n;
    const unsigned blocks = unsigned(std::min<int64_t>((total + 63) / 64, 8192));
    hipLaunchKernelGGL(splitk_epilogue_kernel, dim3(blocks), dim3(256), 0, stream, p.partials, splits, g.m,
                       g.n, g.epi);
  }
  return hipGetLastError();
}

// Launch shape of the packed GEMV (timed on MI355X over the GPT-2 small and XL
// decode shapes, M = 1 and 32, K = 768 .. 6400, N = 768 .. 50257):
//  * W waves x CPW chunks per wave cover a split's K range with the fewest dead
//    slots (a dead slot re-reads a chunk): 12 chunks -> 4 x 3, 16 -> 4 x 4,
//    24 -> 8 x 3, 32 -> 8 x 4, 48 -> 16 x 3, more -> rounds of 16 x 4;
//  * W x CPW follows the chunk count only, the same for 16- and 32-row
//    launches: wave w sums chunks w, w + W, ... in order and the waves are
//    added in wave order, so a row's sums do not depend on the batch size
//    (decode batches of 1..32 give a request the same bits; 32-row-only shapes
//    measured 2-5 % faster per launch: 3072 -> 768 as 12 x 4 6.0 against
//    6.3 us, 1600 -> 6400 as 16 x 2 with block pairs 6.5 against 7.7 us);
//  * at M > 16 two column blocks share each A fragment (CBG = 2: the same
//    per-column order) over >= 200 column blocks at 8 waves, and when that
//    still leaves >= 512 workgroups at 4 waves (the LM head);
//  * a deferred launch splits K to reach ~192 workgroups, keeping >= 4 chunks
//    per split and the partials within the scratch (the split count follows
//    the shape only); otherwise one split and the epilogue runs in the kernel;
//  * a LayerNorm-prologue launch is one split covered by one round.
struct GemvShape {
  int w, cpw, cbg;
};

GemvShape gemv_shape(int mt, int chunks, bool one_round, int nb) {
  GemvShape s{16, 4, 1};
  if (chunks <= 12) s = {4, 3, 1};
  else if (chunks <= 16) s = {4, 4, 1};
  else if (chunks <= 24) s = {8, 3, 1};
  else if (chunks <= 32) s = {8, 4, 1};
  else if (chunks <= 48) s = {16, 3, 1};
  if (mt == 2 && !one_round && s.w == 8 && nb >= 200) s.cbg = 2;
  return s;
}

template <int MT, bool LNA, bool PA, bool CW = false, bool POOL = false, bool RB = false>
hipError_t launch_gemv_shape(const PackedParams& p, GemvShape sh, int grid, hipStream_t st) {
#define TIA_GEMV(W_, C_, B_)                                                                            \
  if (sh.w == W_ && sh.cpw == C_ && sh.cbg == B_) {                                                     \
    hipLaunchKernelGGL((gemv_packed_kernel<MT, W_, C_, B_, LNA, PA, CW, POOL, RB>), dim3(unsigned(grid)), dim3(W_ * 64), 0, st, p); \
    return hipGetLastError();                                                                           \
  }
  TIA_GEMV(4, 3, 1)
  TIA_GEMV(4, 4, 1)
  TIA_GEMV(8, 3, 1)
  TIA_GEMV(8, 4, 1)
  if constexpr (MT == 2) {
    TIA_GEMV(4, 3, 2)
    TIA_GEMV(4, 4, 2)
  }
  if constexpr (!LNA) {
    TIA_GEMV(16, 3, 1)
    TIA_GEMV(16, 4, 1)
  }
  if constexpr (MT == 2 && !LNA) {
    TIA_GEMV(8, 3, 2)
    TIA_GEMV(8, 4, 2)
  }
#undef TIA_GEMV
  return hipErrorInvalidValue;
}

// M = 1 over packed weights with at most 128 column blocks (N <= 2048), or
// any N from K = 1536: the part-block kernel, 8 columns per workgroup.  W x LPW
// covers the record pairs in one round up to K = 3072 (timed on GPT-2 small /
// XL shapes: 768 -> 768 3.07 -> 2.73 us, 3072 -> 768 4.37 -> 3.30 us, 1600 ->
// 1600 3.95 -> 3.07 us; wider, it wins from K = 1536 on: 1600 -> 3072 4.17 ->
// 3.76 us, 3072 -> 3072 5.11 -> 4.51 us, 1600 -> 6400 5.66 -> 5.35 us, 1600 ->
// 50257 26.4 -> 24.0 us, and ties or loses below: 768 -> 3072 3.24 either way,
// 1024 -> 3072 3.45 against 3.58 us).  Not for a
// batching caller's decode (GemmArgs::decode_batches): there one kernel family
// serves every M up to 16, so a row's sums do not depend on the batch; the
// part-block kernel with several rows per workgroup measured slower than the
// MFMA GEMV from two rows up (b = 8 decode 25.8 K against 26.6 K tok/s, b = 16
// 44 K against 51 K).
bool part_gemv_preferred(const GemmArgs& g) {
  // (A caller that wants argmax partials keeps the MFMA GEMV, which writes them.)
  return g.m == 1 && !g.a_p32 && !g.ln_gamma && !g.decode_batches && !g.amax_groups &&
         ((g.n + 15) / 16 <= 128 || g.k >= 1536);
}

hipError_t launch_part(const GemmArgs& g, const Scratch* s, hipStream_t stream, int* deferred) {
  PackedParams p{};
  p.a = g.a; p.lda = g.lda; p.w = static_cast<const u32x4_t*>(g.w_packed); p.scales = g.scales;
  p.m = 1; p.n = g.n; p.k = g.k; p.epi = g.epi;
  p.nb = (g.n + 15) / 16;
  p.kc = g.k / 64;
  p.chunks_per_split = p.kc;
  p.splits = 1;
  p.defer = deferred != nullptr;
  p.partials = s ? s->partials : nullptr;
  if (p.defer && (!p.partials || size_t(g.n) > s->partial_floats)) return hipErrorInvalidValue;
  if (deferred) *deferred = 1;
  const int steps = (p.kc + 1) / 2;
  const dim3 grid(unsigned(2 * p.nb));
  if (steps <= 6) hipLaunchKernelGGL((gemv_part_kernel<3, 2, 8>), grid, dim3(192), 0, stream, p);
  else if (steps <= 16) hipLaunchKernelGGL((gemv_part_kernel<8, 2, 8>), grid, dim3(512), 0, stream, p);
  else hipLaunchKernelGGL((gemv_part_kernel<8, 3, 8>), grid, dim3(512), 0, stream, p);
  return hipGetLastError();
}

// Compute units of the current device (cached per device; 256 on MI355X).
int device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
  cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

template <int MT>
hipError_t launch_packed(const GemmArgs& g, const Scratch* s, hipStream_t stream, int* deferred) {
  PackedParams p{};
  p.a = g.a; p.lda = g.lda; p.w = static_cast<const u32x4_t*>(g.w_packed); p.scales = g.scales;
  p.m = g.m; p.n = g.n; p.k = g.k; p.epi = g.epi;
  p.nb = (g.n + 15) / 16;
  p.kc = g.k / 64;
  p.partials = s ? s->partials : nullptr;
  p.defer = deferred != nullptr;
  const bool ln = g.ln_gamma != nullptr;
  if (ln) {
    p.ln_gamma = g.ln_gamma; p.ln_beta = g.ln_beta; p.ln_eps = g.ln_eps;
  }
  // Wide N (the LM head shape, >= 1024 column blocks) at 17..32 rows: whole
  // column blocks per wave over an LDS copy of A, no cross-wave reduction and
  // A read once per workgroup instead of once per column block pair.  The
  // runtime's decode head (P32 A, fp32 logits) and the ABI's row-major calls
  // take it (768 -> 50257 at M = 32 through the ABI: 18.9 against 20.8 us for
  // the packed GEMV; at M = 1 the packed GEMV is faster, 10.0 against 11.6 us);
  // 16 column blocks per workgroup of 8 waves (two per wave): timed against
  // 8 / 16 / 32 blocks and 4 / 8 / 16 waves on the GPT-2 head.
  const bool wide_epi = p.epi.kind == EPI_F32 || ((p.epi.kind == EPI_F16 || p.epi.kind == EPI_GELU ||
                                                    p.epi.kind == EPI_RESIDUAL) && !p.epi.p32);
  if (MT == 2 && !ln && !deferred && p.nb >= 1024 && (p.kc == 12 || p.kc == 16) && wide_epi &&
      (!g.a_p32 || p.epi.kind == EPI_F32)) {
    WideParams wp{};
    wp.a = g.a; wp.lda = g.lda; wp.w = p.w; wp.scales = p.scales; wp.m = p.m; wp.n = p.n; wp.nb = p.nb;
    wp.epi = p.epi;
    const int cus = device_cus();
    wp.per = std::max(kWideMinWaves, std::min(kWideWaves, (p.nb + 2 * cus - 1) / (2 * cus)));
    const int grid = (p.nb + wp.per - 1) / wp.per;
    if (p.epi.kind == EPI_F32 && g.amax_v && g.amax_i && g.amax_groups && size_t(grid) * 32 <= g.amax_capacity) {
      wp.amax_v = g.amax_v;
      wp.amax_i = g.amax_i;
      *g.amax_groups = grid;
    }
    const dim3 gd{unsigned(grid)}, bd{unsigned(wp.per * 64)};
    if constexpr (MT == 2) {
      auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, gd, bd, 0, stream, wp); };
      if (g.a_p32) {
        if (p.kc == 12) go(gemv_wide_kernel<2, 12, EPI_F32, true>);
        else go(gemv_wide_kernel<2, 16, EPI_F32, true>);
      } else {
        const bool k12 = p.kc == 12;
        switch (p.epi.kind) {
          case EPI_F32: k12 ? go(gemv_wide_kernel<2, 12, EPI_F32, false>) : go(gemv_wide_kernel<2, 16, EPI_F32, false>); break;
          case EPI_GELU: k12 ? go(gemv_wide_kernel<2, 12, EPI_GELU, false>) : go(gemv_wide_kernel<2, 16, EPI_GELU, false>); break;
          case EPI_RESIDUAL:
            k12 ? go(gemv_wide_kernel<2, 12, EPI_RESIDUAL, false>) : go(gemv_wide_kernel<2, 16, EPI_RESIDUAL, false>);
            break;
          default: k12 ? go(gemv_wide_kernel<2, 12, EPI_F16, false>) : go(gemv_wide_kernel<2, 16, EPI_F16, false>); break;
        }
      }
    }
    return hipGetLastError();
  }
  int splits = 1;
  // A C-ABI call over few column blocks and a long K splits K and finishes in
  // the launch (queue pool): >= 12 chunks per split, ~192 workgroups.  The
  // finish costs about a microsecond, so only where the unsplit launch is long
  // (timed, unsplit -> split: 3072 -> 768 at M = 16 6.05 -> 5.27 us, M = 32
  // 8.54 -> 6.41, 6400 -> 1600 at M = 8 8.81 -> 7.77; but M = 8 3072 -> 768
  // 5.09 -> 5.11, 1600 -> 1600 4.42 -> 5.26, 2048 -> 1000 4.41 -> 5.21, and
  // M = 32 1600 -> 1600 6.62 -> 6.71).
  const bool pool = s && s->queue_pool && !deferred && !ln && !g.a_p32 &&
                    ((g.m > 8 && p.kc >= 48) || p.kc >= 64);
  if (deferred && !ln && s && s->partials) {
    const int groups = p.nb;
    const int target = std::max(1, g.defer_workgroups);
    splits = std::max(1, std::min((target + groups - 1) / groups, p.kc / 4));
    while (splits > 1 && size_t(splits) * g.m * g.n > s->partial_floats) --splits;
  } else if (pool && p.nb < 128 && p.kc >= 24) {
    splits = std::max(1, std::min({kPoolGemvSplits, (192 + p.nb - 1) / p.nb, p.kc / 12}));
  }
  p.chunks_per_split = (p.kc + splits - 1) / splits;
  splits = (p.kc + p.chunks_per_split - 1) / p.chunks_per_split;
  p.splits = splits;
  if (p.defer && (!p.partials || size_t(splits) * g.m * g.n > s->partial_floats)) return hipErrorInvalidValue;
  GemvShape sh = gemv_shape(MT, p.chunks_per_split, ln, p.nb);
  if (ln && sh.w * sh.cpw < p.kc) return hipErrorInvalidValue;
  if (MT == 2 && !p.defer && sh.w == 4 && (p.nb + 1) / 2 >= 512) sh.cbg = 2;
  const int grid = (p.nb + sh.cbg - 1) / sh.cbg * splits;
  if (deferred) *deferred = splits;
  if (MT == 1 && splits == 1 && !p.defer && p.epi.kind == EPI_F32 && g.amax_v && g.amax_i && g.amax_groups &&
      size_t(grid) * 32 <= g.amax_capacity) {
    p.amax_v = g.amax_v;
    p.amax_i = g.amax_i;
    *g.amax_groups = grid;
  }
  if (pool && splits > 1) {
    // The finisher holds every split of its outputs in registers.
    const int out_iters = (sh.cbg * MT * 256 + sh.w * 64 - 1) / (sh.w * 64);
    if (splits > kPoolLoads / out_iters || int64_t(grid / splits) > kPoolTiles ||
        int64_t(grid) * sh.cbg * MT * 256 > int64_t(kPoolFloats))
      return hipErrorInvalidValue;
    return launch_gemv_shape<MT, false, false, false, true>(p, sh, grid, stream);
  }
  if (g.a_p32) {
    if constexpr (MT == 1) {
      if (g.weights_shared)
        return ln ? launch_gemv_shape<MT, true, true, true>(p, sh, grid, stream)
                  : launch_gemv_shape<MT, false, true, true>(p, sh, grid, stream);
    }
    return ln ? launch_gemv_shape<MT, true, true>(p, sh, grid, stream)
              : launch_gemv_shape<MT, false, true>(p, sh, grid, stream);
  }
  if constexpr (MT == 1) {
    if (g.weights_shared)
      return ln ? launch_gemv_shape<MT, true, false, true>(p, sh, grid, stream)
                : launch_gemv_shape<MT, false, false, true>(p, sh, grid, stream);
  }
  return ln ? launch_gemv_shape<MT, true, false>(p, sh, grid, stream)
            : launch_gemv_shape<MT, false, false>(p, sh, grid, stream);
}

// 33..128 rows through the C ABI over at most 192 column blocks and K <= 3072:
// the single-tile (MT = 1) GEMV over row blocks of 16 up to 64 rows, the
// two-tile one over row blocks of 32 above, in one launch, no K split: a
// column block's row blocks read its records through one XCD's L2 (cached
// loads), and each workgroup does a 16- or 32-row GEMV's work (timed: M = 64
// 768->3072 6.3 -> 5.45 us, 3072->768 8.2 -> 6.4 us against four 16-row MFMA
// tiles per wave with 4 K splits finished in the launch; M = 40 3072->768
// 7.1 -> 6.3 us; M = 128 against the panel GEMM 8.9 -> 7.6 us and 10.3 ->
// 9.2 us; at 17..32 rows the two-tile GEMV stays faster, M = 32 4.4 / 5.9
// against 4.6 / 6.4 us; from M = 256 the panel GEMM, 9.1 / 11.8 against 12.0 /
// 14.8 us, and wider or longer shapes keep it too).
hipError_t launch_packed_rb(const GemmArgs& g, hipStream_t stream) {
  PackedParams p{};
  p.a = g.a; p.lda = g.lda; p.w = static_cast<const u32x4_t*>(g.w_packed); p.scales = g.scales;
  p.m = g.m; p.n = g.n; p.k = g.k; p.epi = g.epi;
  p.nb = (g.n + 15) / 16;
  p.kc = g.k / 64;
  p.chunks_per_split = p.kc;
  p.splits = 1;
  const int mt = g.m <= 64 ? 1 : 2;
  p.rblocks = (g.m + 16 * mt - 1) / (16 * mt);
  if (int64_t(p.nb) * p.rblocks > INT_MAX / 2) return hipErrorNotSupported;
  GemvShape sh = gemv_shape(mt, p.kc, false, p.nb);
  sh.cbg = 1;
  if (mt == 1) return launch_gemv_shape<1, false, false, true, false, true>(p, sh, p.nb * p.rblocks, stream);
  sh.w = std::min(sh.w, 8);  // two A tiles per chunk: at most 8 waves, K in rounds
  return launch_gemv_shape<2, false, false, true, false, true>(p, sh, p.nb * p.rblocks, stream);
}


// 64x64 tiles, S = 4 stages of 12 KiB (48 KiB of LDS: three workgroups per CU,
// three chunks in flight each; six stages measured slower, since occupancy
// matters more than depth here).  Fewer tiles than ~one per CU split K (at
// least S - 1 chunks per split) when the caller lets partials go to scratch; a
// split launch is finished by splitk_epilogue_kernel unless the caller defers it.
template <int WM, int WN, int MT, int R, int S>
hipError_t launch_panel_cfg(const GemmArgs& g, const Scratch* s, hipStream_t stream, int* deferred) {
  const bool may_split = !g.canonical;
  constexpr int BM = WM * MT * 16, BN = WN * R * 16;
  constexpr int NL = (BM / 16) * 2 + BN / 16;
  constexpr size_t kLds = size_t(S) * NL * 1024 + BN * 4;
  static hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&panel_gemm_kernel<WM, WN, MT, R, S>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, int(kLds));
  static hipError_t attr_pool = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&panel_gemm_kernel<WM, WN, MT, R, S, true>),
      hipFuncAttributeMaxDynamicSharedMemorySize, int(kLds));
  if (attr != hipSuccess) return attr;
  if (attr_pool != hipSuccess) return attr_pool;
  PanelParams p{};
  p.a = g.a; p.lda = g.lda; p.w = static_cast<const u32x4_t*>(g.w_packed); p.scales = g.scales;
  p.m = g.m; p.n = g.n; p.k = g.k; p.epi = g.epi;
  p.nb = (g.n + 15) / 16;
  p.kc = g.k / 64;
  p.tiles_n = (g.n + BN - 1) / BN;
  p.group_m = 8;  // M = 8192, 1600->6400: 356 us against 379 in row-major tile order
  const int64_t tiles = int64_t(p.tiles_n) * ((g.m + BM - 1) / BM);
  if (tiles > (int64_t(1) << 28)) return hipErrorInvalidValue;
  p.tiles = int(tiles);
  int splits = 1;
  const bool pool = s && s->queue_pool && !deferred && tiles <= kPoolTiles;
  const size_t capacity = pool ? kPoolFloats : (s && s->partials) ? s->partial_floats : 0;
  // Split K below ~one tile per CU; a pool plan also below two per CU (M =
  // 512, 3072 -> 768 as 32 x 64 tiles in two K halves: 18.6 -> 14.5 us, the
  // finisher re-reading 16 KB per tile).
  if (may_split && capacity > 0 && tiles < (pool ? 384 : 192)) {
    splits = int(std::min<int64_t>((256 + tiles - 1) / tiles, std::max(1, p.kc / (S - 1))));
    while (splits > 1 && size_t(splits) * g.m * g.n > capacity) --splits;
    if (pool) splits = pool_splits(splits, tiles, BM * BN, kTileRounds * pool_max_splits(BM / (256 / (BN / 4))), p.kc);
  }
  p.chunks_per_split = (p.kc + splits - 1) / splits;
  splits = (p.kc + p.chunks_per_split - 1) / p.chunks_per_split;
  p.splits = splits;
  p.defer = deferred != nullptr && splits > 1;
  p.pool = pool;
  p.partials = s ? s->partials : nullptr;
  if (pool && splits > 1)
    hipLaunchKernelGGL((panel_gemm_kernel<WM, WN, MT, R, S, true>), dim3(unsigned(tiles * splits)), dim3(256), kLds,
                       stream, p);
  else
    hipLaunchKernelGGL((panel_gemm_kernel<WM, WN, MT, R, S>), dim3(unsigned(tiles * splits)), dim3(256), kLds,
                       stream, p);
  if (p.defer) {
    *deferred = splits;
    return hipGetLastError();
  }
  if (splits > 1 && !pool) {
    const int64_t total = int64_t(g.m) * g.n;
    const unsigned blocks = unsigned(std::min<int64_t>((total + 63) / 64, 8192));
    hipLaunchKernelGGL(splitk_epilogue_kernel, dim3(blocks), dim3(256), 0, stream, p.partials, splits, g.m, g.n,
                       g.epi);
  }
  return hipGetLastError();
}

// (Tiles of 128 x 64 and 128 x 128 halve the LDS bytes and dequant work per
// MFMA, but hold one or two 4-wave workgroups per CU and measured 1.3-2x slower
// from M = 512 to 8192; the 64 x 64 tile keeps three per CU.  A 3-stage ring
// (two chunks in flight, 36 KiB, four workgroups per CU) times as fast as or
// faster than 4 stages: M = 512 768->3072 13.2 against 13.7 us, M = 2048
// 768->2304 24.6 against 25.7 us; 6 stages 15.0 / 32.5 us.)
// 64 x 64 tiles; a shape that would split K over fewer than 192 of them but
// has 192 tiles of 32 x 64 takes those unsplit instead (no fp32 partials:
// M = 512, 3072 -> 768 moved 2.85x its algorithmic bytes as three K splits;
// 23.5 -> 21.2 us).  The canonical (batch-invariant) route keeps 64-row tiles.
hipError_t launch_panel(const GemmArgs& g, const Scratch* s, hipStream_t stream, int* deferred) {
  const int64_t tiles64 = int64_t((g.m + 63) / 64) * ((g.n + 63) / 64);
  const int64_t tiles32 = int64_t((g.m + 31) / 32) * ((g.n + 63) / 64);
  // Pool plans finish each tile in one workgroup with a bounded split count
  // (4 for 64 x 64 tiles, 8 for 32 x 64), so a grid short of tiles takes the
  // 32-row tiles there too.
  const bool pool = s && s->queue_pool && !deferred;
  if (!g.canonical && tiles64 < 192 && (tiles32 >= 192 || pool))
    return launch_panel_cfg<1, 4, 2, 1, 4>(g, s, stream, deferred);
  return launch_panel_cfg<1, 4, 4, 1, 3>(g, s, stream, deferred);
}

// ---------------------------------------------------------------------------
// Prefill GEMM over pre-dequantised fp16 weights (M > 32)
// ---------------------------------------------------------------------------
// With the weights dequantised once at load (fp16_rn(float(q) * scale), the
// same values the int8 kernels compute on the fly) the prefill GEMM is a plain
// fp16 MFMA GEMM: no dequantisation VALU per row tile, so each wave can own a
// 64 x 64 output tile (16 accumulators of v_mfma_f32_16x16x32_f16), which cuts
// the LDS bytes per MFMA to a quarter of the int8 panel kernel's.  fp16 B
// records: (column block cb, K group kk of 32) is 1 KiB at (cb * KK + kk) *
// 1024 bytes, lane l holding column cb * 16 + (l & 15), rows kk * 32 + 8 (l >> 4)
// + 0..7 (the MFMA B operand); zero past K and N.
struct F16GemmParams {
  const uint16_t* a;
  int64_t lda;
  const u32x4_t* w;  // fp16 B records
  int m, n, k;
  int kk;            // K groups of 32
  int tiles_n, tiles;
  int group_m;       // tile rows per group of the tile order
  int chunks_per_split, splits;
  bool defer;
  bool pool;         // splits > 1 finish in this launch through the queue pool (EP == 1 only)
  Epilogue epi;
  float* partials;
};

__global__ void pack_w16_kernel(const int8_t* q, int64_t ldq, const float* scales, int k, int n, int kk,
                                int64_t records, u32x4_t* out) {
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= records * 64) return;
  const int64_t rec = t >> 6;
  const int lane = int(t & 63);
  const int cb = int(rec / kk), g = int(rec % kk);
  const int col = cb * 16 + (lane & 15), r0 = g * 32 + 8 * (lane >> 4);
  half8_t v;
  const float sc = col < n ? scales[col] : 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int row = r0 + e;
    v[e] = (row < k && col < n) ? f16r(float(q[int64_t(row) * ldq + col]) * sc) : f16(0.f);
  }
  out[t] = __builtin_bit_cast(u32x4_t, v);
}

// Tile (WM * MT * 16) x (WN * R * 16), WM x WN waves, each MT x R MFMA blocks;
// K in chunks of 32 moved HBM/L2 -> LDS by global_load_lds_dwordx4 (A
// fragments of 16 rows x 32 K in MFMA A order, B records as stored), S stages
// as in the int8 panel kernel.  The epilogue runs from the accumulators.
template <int WM, int WN, int MT, int R, int S, int EP = 1, int OCC = 2, bool POOL = false>
__global__ __launch_bounds__(WM * WN * 64, OCC) void f16_gemm_kernel(F16GemmParams p) {
  constexpr int W = WM * WN, NT = W * 64;
  constexpr int BM = WM * MT * 16, BN = WN * R * 16;
  constexpr int NA = BM / 16, NB = BN / 16, NL = NA + NB;
  static_assert(NL % W == 0, "loads must split evenly over the waves");
  constexpr int LPW = NL / W;
  constexpr int STAGE = NL * 1024;
  static_assert(S >= 3 && (S - 2) * LPW < 64, "in-flight loads within vmcnt");
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];  // max(S * STAGE, epilogue tile)

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int wm = wave / WN, wn = wave % WN;
  int split, tm, tn;
  tile_of_block(p.group_m, p.tiles_n, p.tiles, split, tm, tn);
  const int m0 = tm * BM, cb0 = tn * NB;
  const int nbt = (p.n + 15) / 16;
  const int c_begin = split * p.chunks_per_split;
  const int kc = min(p.kk - c_begin, p.chunks_per_split);  // chunks of this split (>= 1)

  // Load id < NA: A fragment t (rows m0 + 16t .. +15, clamped), lane (j, g) at
  // k = 32c + 8g; otherwise B record cb0 + id - NA (clamped).
  const char* src[LPW];
  int stride[LPW];
#pragma unroll
  for (int l = 0; l < LPW; ++l) {
    const int id = wave * LPW + l;
    if (id < NA) {
      const int row = min(m0 + 16 * id + j, p.m - 1);
      src[l] = reinterpret_cast<const char*>(p.a + int64_t(row) * p.lda + 32 * c_begin + 8 * g);
      stride[l] = 64;
    } else {
      const int cb = min(cb0 + id - NA, nbt - 1);
      src[l] = reinterpret_cast<const char*>(p.w + (int64_t(cb) * p.kk + c_begin) * 64 + lane);
      stride[l] = 1024;
    }
  }
  auto issue = [&](int chunk, int stage) {
#pragma unroll
    for (int l = 0; l < LPW; ++l)
      __builtin_amdgcn_global_load_lds((global_ptr)(src[l] + int64_t(chunk) * stride[l]),
                                       (lds_ptr)(lds + stage * STAGE + (wave * LPW + l) * 1024), 16, 0, 0);
  };
  // The epilogue gives thread t columns 4 (t % (BN / 4)) .. + 3 of the tile:
  // their bias is loaded now and used after the loop.
  const bool epi_now = p.splits == 1 && !p.defer;
  float bias[4];
  load_bias4(p.epi, cb0 * 16 + 4 * int(threadIdx.x % (BN / 4)), p.n, p.a, bias);

  float4_t acc[MT][R];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[t][r] = float4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int c = 0; c < S - 1; ++c) issue(min(c, kc - 1), c);
  for (int c = 0; c < kc; ++c) {
    wait_chunk<LPW, 0, S - 2>(min(c + S - 2, kc - 1) - c);
    __builtin_amdgcn_s_barrier();
    if (c + S - 1 < kc) issue(c + S - 1, (c + S - 1) % S);
    const uint8_t* st = lds + (c % S) * STAGE;
    half8_t bf[R];
#pragma unroll
    for (int r = 0; r < R; ++r) bf[r] = *reinterpret_cast<const half8_t*>(st + (NA + wn * R + r) * 1024 + lane * 16);
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const half8_t af = *reinterpret_cast<const half8_t*>(st + (wm * MT + t) * 1024 + lane * 16);
#pragma unroll
      for (int r = 0; r < R; ++r) acc[t][r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[r], acc[t][r], 0, 0, 0);
    }
  }
  wait_vmcnt<0>();

  // Epilogue through an LDS fp32 tile of BM / EP rows x BN, EP passes (the
  // accumulators never meet the epilogue's registers; EP > 1 cuts the LDS the
  // kernel needs), each finished 4 columns per thread by tile_epilogue.
  constexpr int PR = BM / EP;  // rows per pass
  static_assert(BM % EP == 0 && PR % 16 == 0, "whole 16-row blocks per pass");
  float* ctile = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int pass = 0; pass < EP; ++pass) {
    __syncthreads();
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int rb = (wm * MT + t) * 16 - pass * PR;  // block row inside this pass
      if (rb < 0 || rb >= PR) continue;
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          ctile[(rb + 4 * g + v) * tile_pitch(BN) + (wn * R + r) * 16 + j] = acc[t][r][v];
    }
    __syncthreads();
    if constexpr (EP == 1 && POOL) {
      if (p.splits > 1) {
        if (tile_split_finish<PR, BN, NT>(ctile, split, p.splits, tm * p.tiles_n + tn))
          tile_epilogue<PR, BN, NT>(p.epi, ctile, m0, cb0 * 16, p.m, p.n, bias, nullptr, split);
        return;
      }
    }
    tile_epilogue<PR, BN, NT>(p.epi, ctile, m0 + pass * PR, cb0 * 16, p.m, p.n, bias,
                              epi_now ? nullptr : p.partials, split);
  }
}

template <int WM, int WN, int MT, int R, int S, int EP = 1, int OCC = 2>
hipError_t launch_f16_cfg(const GemmArgs& g, const Scratch* s, hipStream_t stream, int* deferred) {
  constexpr int BM = WM * MT * 16, BN = WN * R * 16;
  constexpr int NL = BM / 16 + BN / 16;
  constexpr size_t kLds = std::max(size_t(S) * NL * 1024, size_t(BM / EP) * tile_pitch(BN) * 4);
  static hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&f16_gemm_kernel<WM, WN, MT, R, S, EP, OCC>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, int(kLds));
  if (attr != hipSuccess) return attr;
  static hipError_t attr_pool =
      EP == 1 ? hipFuncSetAttribute(reinterpret_cast<const void*>(&f16_gemm_kernel<WM, WN, MT, R, S, EP, OCC, EP == 1>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, int(kLds))
              : hipSuccess;
  if (attr_pool != hipSuccess) return attr_pool;
  F16GemmParams p{};
  p.a = g.a; p.lda = g.lda; p.w = static_cast<const u32x4_t*>(g.w_f16p);
  p.m = g.m; p.n = g.n; p.k = g.k; p.epi = g.epi;
  p.kk = (g.k + 31) / 32;
  p.tiles_n = (g.n + BN - 1) / BN;
  p.group_m = 2;  // M = 8192, 1600->6400: 315 us; row-major order 321, groups of 8 rows 327
  const int64_t tiles = int64_t(p.tiles_n) * ((g.m + BM - 1) / BM);
  if (tiles > (int64_t(1) << 28)) return hipErrorInvalidValue;
  p.tiles = int(tiles);
  int splits = 1;
  const bool pool = s && s->queue_pool && !deferred;
  const size_t capacity = !pool ? ((s && s->partials) ? s->partial_floats : 0)
                                : (EP == 1 && tiles <= kPoolTiles) ? kPoolFloats : 0;
  if (!g.canonical && capacity > 0 && tiles < 192) {
    splits = int(std::min<int64_t>((256 + tiles - 1) / tiles, std::max(1, p.kk / (S - 1))));
    while (splits > 1 && size_t(splits) * g.m * g.n > capacity) --splits;
    if (pool)
      splits = pool_splits(splits, tiles, BM * BN,
                           kTileRounds * pool_max_splits(std::max(1, BM / (WM * WN * 64 / (BN / 4)))), p.kk);
  }
  p.chunks_per_split = (p.kk + splits - 1) / splits;
  splits = (p.kk + p.chunks_per_split - 1) / p.chunks_per_split;
  p.splits = splits;
  p.defer = deferred != nullptr && splits > 1;
  p.pool = pool;
  p.partials = s ? s->partials : nullptr;
  if (pool && splits > 1)
    hipLaunchKernelGGL((f16_gemm_kernel<WM, WN, MT, R, S, EP, OCC, EP == 1>), dim3(unsigned(tiles * splits)),
                       dim3(WM * WN * 64), kLds, stream, p);
  else
    hipLaunchKernelGGL((f16_gemm_kernel<WM, WN, MT, R, S, EP, OCC>), dim3(unsigned(tiles * splits)), dim3(WM * WN * 64),
                       kLds, stream, p);
  if (p.defer) {
    *deferred = splits;
    return hipGetLastError();
  }
  if (splits > 1 && !pool) {
    const int64_t total = int64_t(g.m) * g.n;
    const unsigned blocks = unsigned(std::min<int64_t>((total + 63) / 64, 8192));
    hipLaunchKernelGGL(splitk_epilogue_kernel, dim3(blocks), dim3(256), 0, stream, p.partials, splits, g.m, g.n,
                       g.epi);
  }
  return hipGetLastError();
}

// Tile choice over the fp16 records, and when they beat the int8 panel
// kernel, from timings on MI355X (graph replays over rotating weights):
// * 128 x 128 tiles on 8 waves (each 64 x 32, 3 stages, the epilogue in 4
//   passes of 32 rows so three workgroups fit a CU) once the grid holds >= 384
//   of them, or >= 192 at K >= 1536: M = 8192 1600->6400 247 us (679 TF/s;
//   4 waves of 64 x 64: 309 us), 768->2304 65 us (64 x 64 tiles: 76),
//   3072->768 71 us (81); M = 4096 1600->4800 107 us (138); M = 2048
//   1600->1600 35 us (41);
// * below that, 64 x 64 tiles on 8 waves (each 32 x 16): M = 2048 768->2304
//   27.5 us (4 waves: 29.3), 3072->768 37 us (40);
// * the int8 panels stay for M < 2048 at K < 1536, where the two time the same;
// * at K >= 1536 the 64 x 64 tiles keep a 4-stage ring (two chunks of 32 in
//   flight): M = 1024 3072->768 25.3 us against 31.5 with 3 stages, which time
//   the same or better at K = 768 (6 stages: slower everywhere).
bool f16_gemm_large(int m, int n, int k) {
  const int64_t tiles = int64_t((m + 127) / 128) * ((n + 127) / 128);
  return tiles >= 384 || (k >= 1536 && tiles >= 192);
}
bool f16_gemm_preferred(int m, int n, int k) { return f16_gemm_large(m, n, k) || (m >= 2048 && k < 1536); }

// Larger tiles halve the LDS bytes per MFMA (a wave's 128 x 64 or 128 x 32
// block reads 12 / 10 KiB per 32 / 16 MFMAs, against 6 KiB per 8 for 64 x 32)
// but hold one (256 x 256: 96 KiB, 202 registers) or two (256 x 128) 8-wave
// workgroups per CU, so they win only where the grid fills whole rounds of
// them (timed on MI355X, XL shapes, graph replays):
// * 256 x 256 at K >= 4096 when the tiles make one nearly full round:
//   M = 8192 6400->1600 (224 tiles) 199 us against 256; at 112 tiles 188
//   against 143, at 294 (two rounds) 388 against 328;
// * 256 x 128 from four rounds of two per CU at K < 4096: M = 8192
//   1600->4800 180 against 194 us, 1600->6400 244 against 257, M = 10752
//   1600->4800 238 against 250, 1600->6400 310 against 326; at 1.2-2 rounds
//   slower (M = 4096 1600->4800 121 against 110 us).  Its occupancy (two
//   8-wave workgroups per CU) needs <= 128 registers, held by the launch
//   bound (a few epilogue values spill).
hipError_t launch_f16(const GemmArgs& g, const Scratch* s, hipStream_t stream, int* deferred) {
  if (f16_gemm_large(g.m, g.n, g.k)) {
    const int64_t cus = device_cus(), rows256 = (g.m + 255) / 256;
    const int64_t t256 = rows256 * ((g.n + 255) / 256), t256x128 = rows256 * ((g.n + 127) / 128);
    if (g.k >= 4096 && 4 * t256 >= 3 * cus && t256 <= cus) return launch_f16_cfg<2, 4, 8, 4, 3, 8, 2>(g, s, stream, deferred);
    if (g.k < 4096 && t256x128 >= 4 * cus) return launch_f16_cfg<2, 4, 8, 2, 3, 8, 4>(g, s, stream, deferred);
    return launch_f16_cfg<2, 4, 4, 2, 3, 4, 3>(g, s, stream, deferred);
  }
  if (g.k >= 1536) return launch_f16_cfg<2, 4, 2, 1, 4, 1, 3>(g, s, stream, deferred);
  return launch_f16_cfg<2, 4, 2, 1, 3, 1, 3>(g, s, stream, deferred);
}

// Row-major W (the reference ABI's [K, N]).  Each K step of a workgroup waits
// for one global round trip, so a grid of few tiles (M = 64, 3072 -> 768: 12
// tiles x 96 steps, 138 us) splits K until >= 256 workgroups run (at least 4
// steps each); the splits are summed in a fixed order and the epilogue applied
// by the last workgroup of each tile (queue pool, capped split count) or by
// splitk_epilogue_kernel over caller scratch.  Canonical (batch-invariant)
// calls stay unsplit: their K order must not depend on M.
// Split count of the row-major M > 32 kernel (0 capacity or a canonical call:
// one split), after rounding to whole step ranges.
int tiled_splits(int m, int n, int k, bool canonical, size_t capacity) {
  const int steps = (k + TBK - 1) / TBK;
  const int64_t tiles = int64_t((n + TBN - 1) / TBN) * ((m + TBM - 1) / TBM);
  int splits = 1;
  if (!canonical && capacity > 0 && tiles < 256) {
    splits = int(std::min<int64_t>((256 + tiles - 1) / tiles, std::max(1, steps / 4)));
    while (splits > 1 && size_t(splits) * m * n > capacity) --splits;
  }
  const int per = (steps + splits - 1) / splits;
  return (steps + per - 1) / per;
}

template <bool INT8>
hipError_t launch_tiled(const GemmArgs& g, bool wvec, bool avec, const Scratch* s, hipStream_t stream) {
  TiledParams p{};
  p.a = g.a; p.lda = g.lda; p.w = g.w; p.scales = g.scales;
  p.m = g.m; p.n = g.n; p.k = g.k; p.epi = g.epi;
  p.ldw = g.ldw > 0 ? g.ldw : g.n;
  const int steps = (g.k + TBK - 1) / TBK;
  const int64_t tiles = int64_t((g.n + TBN - 1) / TBN) * ((g.m + TBM - 1) / TBM);
  const bool pool = s && s->queue_pool && tiles <= kPoolTiles;
  int splits = tiled_splits(g.m, g.n, g.k, g.canonical,
                            pool ? kPoolFloats : (s && s->partials) ? s->partial_floats : 0);
  if (pool) splits = pool_splits(splits, tiles, TBM * TBN, kTileRounds * pool_max_splits(TBM / (256 / (TBN / 4))), steps);
  p.steps_per_split = (steps + splits - 1) / splits;
  p.partials = splits > 1 && !pool ? s->partials : nullptr;
  p.pool = pool;
  const dim3 grid(unsigned((g.n + TBN - 1) / TBN), unsigned((g.m + TBM - 1) / TBM), unsigned(splits));
#define TIA_TILED(WV, AV)                                                                 \
  do {                                                                                     \
    if (pool && splits > 1)                                                                \
      hipLaunchKernelGGL((tiled_kernel<INT8, WV, AV, true>), grid, dim3(256), 0, stream, p); \
    else                                                                                   \
      hipLaunchKernelGGL((tiled_kernel<INT8, WV, AV>), grid, dim3(256), 0, stream, p);       \
  } while (0)
  if (wvec && avec) TIA_TILED(true, true);
  else if (wvec) TIA_TILED(true, false);
  else if (avec) TIA_TILED(false, true);
  else TIA_TILED(false, false);
#undef TIA_TILED
  if (splits > 1 && !pool) {
    const int64_t total = int64_t(g.m) * g.n;
    const unsigned blocks = unsigned(std::min<int64_t>((total + 63) / 64, 8192));
    hipLaunchKernelGGL(splitk_epilogue_kernel, dim3(blocks), dim3(256), 0, stream, p.partials, splits, g.m, g.n,
                       g.epi);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t gemm(const GemmArgs& g, const Scratch* s, hipStream_t stream, int* deferred) {
  if (deferred) *deferred = 0;
  if (g.amax_groups) *g.amax_groups = 0;
  if (g.m <= 0 || g.n <= 0 || g.k <= 0) return hipErrorInvalidValue;
  const uintptr_t wp = reinterpret_cast<uintptr_t>(g.w), ap = reinterpret_cast<uintptr_t>(g.a);
  // Whole 4-column groups may be loaded when rows are 4-aligned and the row
  // pitch covers n rounded up to 4 (columns past n are padding, never stored).
  const int64_t ldw = g.ldw > 0 ? g.ldw : g.n;
  const bool wvec = ldw % 4 == 0 && ldw >= (int64_t(g.n) + 3) / 4 * 4 &&
                    (g.w_int8 ? wp % 4 == 0 : wp % 8 == 0);
  const bool avec = ((g.lda % 8 == 0) || g.a_p32) && (ap % 16 == 0);
  if (g.a_p32 || g.epi.p32) {
    // P32 operands exist only for the packed-weight decode GEMV.
    const bool epi_ok = !g.epi.p32 || ((g.epi.kind == EPI_F16 || g.epi.kind == EPI_GELU ||
                                        g.epi.kind == EPI_RESIDUAL) && g.n % 64 == 0 && !deferred);
    if (g.m > 32 || g.k % 64 != 0 || !g.w_int8 || !g.w_packed || !epi_ok ||
        reinterpret_cast<uintptr_t>(g.a) % 16 != 0 || reinterpret_cast<uintptr_t>(g.w_packed) % 16 != 0)
      return hipErrorInvalidValue;
  }
  if (g.ln_gamma) {
    if (!gemm_ln_supported(g.m, g.k, g.n) || !g.w_int8 || !g.w_packed || !g.ln_beta || !avec ||
        reinterpret_cast<uintptr_t>(g.w_packed) % 16 != 0 || reinterpret_cast<uintptr_t>(g.ln_gamma) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(g.ln_beta) % 16 != 0)
      return hipErrorInvalidValue;
  }
  // (K % 32 == 0: an A fragment never reads past its row.)  With int8 packed
  // weights also present, the fp16 copy serves only the shapes where it wins.
  if (g.w_f16p && g.m > 32 && !g.ln_gamma && !g.a_p32 && !g.epi.p32 && g.k % 32 == 0 && avec &&
      reinterpret_cast<uintptr_t>(g.w_f16p) % 16 == 0 && (!g.w_packed || f16_gemm_preferred(g.m, g.n, g.k)))
    return launch_f16(g, s, stream, deferred);
  if (g.canonical && g.w_int8 && g.w_packed && g.k % 64 == 0 && avec && !g.a_p32 && !g.ln_gamma &&
      reinterpret_cast<uintptr_t>(g.w_packed) % 16 == 0) {
    // Batch-invariant rows: the fp16-record or the int8 panel kernel (same MFMA
    // sequence, same values) at every M, unsplit, each where it times faster:
    // the panels below f16_gemm_preferred's shapes (M = 1024 768->2304 17.5
    // against 18.3 us, 3072->768 24.7 against 25.3 us), the fp16 records at
    // the large-tile shapes and M >= 2048 at K < 1536, and at M <= 64
    // (M = 32 768->768: 7.4 against 9.1 us).
    if (g.w_f16p && reinterpret_cast<uintptr_t>(g.w_f16p) % 16 == 0 && (g.m <= 64 || f16_gemm_preferred(g.m, g.n, g.k)))
      return launch_f16(g, s, stream, deferred);
    return launch_panel(g, s, stream, deferred);
  }
  if (g.w_int8 && g.w_packed && g.k % 64 == 0 && avec && reinterpret_cast<uintptr_t>(g.w_packed) % 16 == 0) {
    if (part_gemv_preferred(g)) return launch_part(g, s, stream, deferred);
    if (g.m <= 16) return launch_packed<1>(g, s, stream, deferred);
    if (g.m <= 32) return launch_packed<2>(g, s, stream, deferred);
    if (g.m <= 128 && s && s->queue_pool && !deferred && !g.ln_gamma && !g.a_p32 && !g.amax_groups &&
        (g.n + 15) / 16 <= 192 && g.k <= 3072) {
      const hipError_t e = launch_packed_rb(g, stream);
      if (e != hipErrorNotSupported) return e;
    }
    return launch_panel(g, s, stream, deferred);
  }
  if (g.m <= kRowMaxM && g.w_int8 && wvec && avec && s && s->queue_pool && !deferred) {
    const hipError_t e = g.m <= 16 ? launch_rowgemv(g, stream) : launch_rowgemm(g, stream);
    if (e != hipErrorNotSupported) return e;
  }
  if (g.m <= 16) return g.w_int8 ? launch_skinny<true, 1>(g, wvec, avec, s, stream, deferred)
                                 : launch_skinny<false, 1>(g, wvec, avec, s, stream, deferred);
  if (g.m <= 32) return g.w_int8 ? launch_skinny<true, 2>(g, wvec, avec, s, stream, deferred)
                                 : launch_skinny<false, 2>(g, wvec, avec, s, stream, deferred);
  return g.w_int8 ? launch_tiled<true>(g, wvec, avec, s, stream) : launch_tiled<false>(g, wvec, avec, s, stream);
}

hipError_t argmax_partials(const float* vals, const int32_t* idx, int groups, int rows, int32_t* out,
                           hipStream_t stream) {
  if (rows < 1 || rows > 32 || groups < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(argmax_partials_kernel, dim3(unsigned(rows)), dim3(64), 0, stream, vals, idx, groups, out);
  return hipGetLastError();
}

bool gemm_ln_supported(int m, int k, int n) {
  return m >= 1 && m <= 32 && n >= 1 && k >= 64 && k % 64 == 0 && k / 64 <= kLnMaxChunks;
}

size_t packed_w16_bytes(int k, int n) {
  if (k <= 0 || n <= 0) return 0;
  return size_t((n + 15) / 16) * size_t((k + 31) / 32) * 1024;
}

hipError_t pack_w16(const int8_t* q, int64_t ldq, const float* scales, int k, int n, void* out,
                    hipStream_t stream) {
  if (k <= 0 || n <= 0 || !q || !scales || !out || ldq < n) return hipErrorInvalidValue;
  const int kk = (k + 31) / 32;
  const int64_t records = int64_t((n + 15) / 16) * kk;
  const int64_t threads = records * 64;
  hipLaunchKernelGGL(pack_w16_kernel, dim3(unsigned((threads + 255) / 256)), dim3(256), 0, stream, q, ldq, scales, k,
                     n, kk, records, static_cast<u32x4_t*>(out));
  return hipGetLastError();
}

size_t packed_w8_bytes(int k, int n) {
  if (k <= 0 || n <= 0) return 0;
  return size_t((n + 15) / 16) * size_t((k + 63) / 64) * 1024;
}

hipError_t pack_w8(const int8_t* q, int64_t ldq, int k, int n, void* out, hipStream_t stream) {
  if (k <= 0 || n <= 0 || ldq < n) return hipErrorInvalidValue;
  const int kc = (k + 63) / 64;
  const int64_t total16 = int64_t(packed_w8_bytes(k, n) / 16);
  const unsigned blocks = unsigned(std::min<int64_t>((total16 + 255) / 256, 16384));
  hipLaunchKernelGGL(pack_w8_kernel, dim3(blocks), dim3(256), 0, stream, q, ldq, k, n, kc, total16,
                     static_cast<u32x4_t*>(out));
  return hipGetLastError();
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
  return legacy_gemm_f32_variant(2, a, b, c, m, n, k, stream);
}

hipError_t legacy_gemm_f32_variant(int variant, const float* a, const float* b, float* c, int m, int n, int k,
                                   hipStream_t stream) {
  if (m <= 0 || n <= 0 || k <= 0) return hipErrorInvalidValue;
  if (variant == 2) {
    if ((m + 63) / 64 > 65535) return hipErrorInvalidValue;
    hipLaunchKernelGGL(legacy_f32_kernel, dim3(unsigned((n + 63) / 64), unsigned((m + 63) / 64)), dim3(256), 0,
                       stream, a, b, c, m, n, k);
  } else if (variant == 0 || variant == 1) {
    if ((m + 15) / 16 > 65535) return hipErrorInvalidValue;
    const dim3 grid(unsigned((n + 15) / 16), unsigned((m + 15) / 16));
    if (variant == 0) hipLaunchKernelGGL(legacy_f32_naive_kernel, grid, dim3(256), 0, stream, a, b, c, m, n, k);
    else hipLaunchKernelGGL(legacy_f32_tiled_kernel, grid, dim3(256), 0, stream, a, b, c, m, n, k);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace tia
