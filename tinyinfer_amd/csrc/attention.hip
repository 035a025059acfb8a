// Attention for gfx950: fused QK^T, online softmax and PV with fp32 state.
//
// Lane layout inside a wave (head_dim D, LPK = D/8 lanes per key):
//   lane = key_group * LPK + dim_segment; each lane holds 8 consecutive dims
//   (16 bytes) of one key, so a wave-wide load covers 64/LPK whole keys (128 or
//   256 contiguous bytes each) and both K and V are read exactly once, fully
//   coalesced, from either the packed [B,H,K,D] ABI layout or the runtime's
//   [slot][layer][head][pos][64] cache.  The q.k dot finishes with a
//   butterfly over the LPK lanes of a key group; probabilities never leave the
//   lane that owns the key, so PV needs no broadcast.
// A workgroup serves QW queries with KW waves each: KW > 1 splits the keys of a
// query across waves (decode, where one (b, h) row otherwise gives only
// B*H waves) and merges their (m, l, acc) states through LDS.
// Semantics follow reference kernels/src/cuda/tc/attention.cu:29-56: scores
// are dot(q,k) * D^-1/2, keys j < kv_valid (and j <= offset + qi when causal),
// rows with no visible key (or padded queries) are exactly zero.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace tia {
namespace {

constexpr float kNegInf = -__builtin_huge_valf();

struct AttnParams {
  AttnArgs a;
  float scale;
  bool vec;  // every pointer and stride allows 16-byte accesses
};

template <bool VEC>
__device__ __forceinline__ half8_t load8(const uint16_t* p) {
  if constexpr (VEC) return *reinterpret_cast<const half8_t*>(p);
  half8_t out;
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = __builtin_bit_cast(f16, p[i]);
  return out;
}

// K and V fragments of one tile: NI wave-wide loads each of 64/LPK whole keys.
template <int NI>
struct KVTile {
  half8_t k[NI], v[NI];
};

template <int D, int QW, int KW, bool VEC, bool FUSEDQKV = false>
__global__ __launch_bounds__(QW * KW * 64) void attention_kernel(AttnParams p) {
  // A tile is NI wave-wide loads: D=64 -> 32 keys, D=128 -> 16 keys.  Two tiles
  // are kept in registers so the next tile's K and V are in flight while the
  // current one is scored (one memory round trip per wave, not per tile).
  constexpr int LPK = D / 8, KPI = 64 / LPK, NI = 4, TK = NI * KPI;
  const AttnArgs& a = p.a;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kg = lane / LPK, ds = lane % LPK;
  const int qslot = wave / KW, kw = wave % KW;
  const int qi = blockIdx.x * QW + qslot, h = blockIdx.y, b = blockIdx.z;

  const int q_valid = max(0, min(a.q_len, a.q_lengths[b]));
  int end = 0;
  if (qi < q_valid) {
    const int64_t off = a.offsets ? int64_t(a.offsets[b]) : 0;
    const int64_t kvv = a.kv_from_offsets ? off + q_valid
                                          : int64_t(max(0, min(a.kv_len, a.kv_lengths[b])));
    const int64_t bound = a.causal ? off + qi + 1 : kvv;
    end = int(max<int64_t>(0, min<int64_t>(bound, kvv)));
  }
  const int64_t slot = a.kv_slot ? int64_t(a.kv_slot[b]) : int64_t(b);
  const uint16_t* kb = a.k + slot * a.kv_sb + int64_t(h) * a.kv_sh + 8 * ds;
  const uint16_t* vb = a.v + slot * a.kv_sb + int64_t(h) * a.kv_sh + 8 * ds;

  half8_t qf = {};
  if constexpr (FUSEDQKV) {
    // Wave 0 finishes the deferred QKV GEMM for this (b, h): lane d sums the
    // split-K partials of q, k and v (bias added, fp16 rounding as the QKV
    // output), stores k and v into the cache at the new position, and shares q
    // through LDS.  The barrier orders those stores before any tile load.
    static_assert(D == 64 && QW == 1, "fused QKV decode is for 64-dim heads, one query");
    __shared__ f16 sq[64];
    if (wave == 0 && q_valid > 0) {
      const int64_t plane = int64_t(a.batch) * 3 * a.hidden;
      const float* pp = a.qkv_partials + int64_t(b) * 3 * a.hidden + h * 64 + lane;
      const uint16_t* bq = a.qkv_bias + h * 64 + lane;
      const float bqv = h2f(bq[0]), bkv = h2f(bq[a.hidden]), bvv = h2f(bq[2 * a.hidden]);
      float sqv[4] = {0.f, 0.f, 0.f, 0.f}, skv[4] = {0.f, 0.f, 0.f, 0.f}, svv[4] = {0.f, 0.f, 0.f, 0.f};
      int sp = 0;
      for (; sp + 4 <= a.qkv_splits; sp += 4) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float* ps = pp + int64_t(sp + u) * plane;
          sqv[u] += ps[0];
          skv[u] += ps[a.hidden];
          svv[u] += ps[2 * a.hidden];
        }
      }
      for (; sp < a.qkv_splits; ++sp) {
        const float* ps = pp + int64_t(sp) * plane;
        sqv[0] += ps[0];
        skv[0] += ps[a.hidden];
        svv[0] += ps[2 * a.hidden];
      }
      sq[lane] = f16(((sqv[0] + sqv[1]) + (sqv[2] + sqv[3])) + bqv);
      const int64_t pos = a.offsets[b];
      const int64_t at = slot * a.kv_sb + int64_t(h) * a.kv_sh + pos * D + lane;
      const_cast<uint16_t*>(a.k)[at] = f2h(((skv[0] + skv[1]) + (skv[2] + skv[3])) + bkv);
      const_cast<uint16_t*>(a.v)[at] = f2h(((svv[0] + svv[1]) + (svv[2] + svv[3])) + bvv);
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 8; ++e) qf[e] = sq[8 * ds + e];
  } else {
    if (qi < q_valid) qf = load8<VEC>(a.q + int64_t(b) * a.q_sb + int64_t(h) * a.q_sh + int64_t(qi) * a.q_sq + 8 * ds);
  }

  float m = kNegInf, l = 0.f;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};

  // Keys at or past `end` re-read key end-1 (valid, written data) instead of
  // branching, so every load of a tile is unconditional and the compiler can
  // wait for one tile while the next is still in flight; their scores are -inf
  // and their probabilities 0 in `process`.
  auto load_tile = [&](KVTile<NI>& t, int k0) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int key = min(k0 + kg + KPI * i, end - 1);
      t.k[i] = load8<VEC>(kb + int64_t(key) * D);
      t.v[i] = load8<VEC>(vb + int64_t(key) * D);
    }
  };
  // Online-softmax update with one tile (its first key k0 < end is visible, so
  // the running maximum is finite afterwards).
  auto process = [&](const KVTile<NI>& t, int k0) {
    float s[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int key = k0 + kg + KPI * i;
      float part = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) part += float(qf[e]) * float(t.k[i][e]);
#pragma unroll
      for (int o = LPK / 2; o > 0; o >>= 1) part += __shfl_xor(part, o, 64);
      s[i] = key < end ? part * p.scale : kNegInf;
    }
    float tmax = s[0];
#pragma unroll
    for (int i = 1; i < NI; ++i) tmax = fmaxf(tmax, s[i]);
#pragma unroll
    for (int o = LPK; o < 64; o <<= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, o, 64));
    const float nm = fmaxf(m, tmax);
    const float alpha = l == 0.f ? 0.f : __expf(m - nm);
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= alpha;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int key = k0 + kg + KPI * i;
      const float pr = key < end ? __expf(s[i] - nm) : 0.f;
      psum += pr;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += pr * float(t.v[i][e]);
    }
#pragma unroll
    for (int o = LPK; o < 64; o <<= 1) psum += __shfl_xor(psum, o, 64);
    l = l * alpha + psum;
    m = nm;
  };

  // Wave kw takes tiles kw, kw + KW, ...; tile loads for the next tile are
  // issued before the current tile is processed (keys past `end` load nothing).
  // The scheduling barriers keep the compiler from sinking the prefetch loads
  // next to their uses (which would serialize them again).
  constexpr int STEP = TK * KW;
  int k0 = kw * TK;
  if (k0 < end) {
    KVTile<NI> ta, tb;
    load_tile(ta, k0);
    for (;;) {
      load_tile(tb, k0 + STEP);
      __builtin_amdgcn_sched_barrier(0);
      process(ta, k0);
      k0 += STEP;
      if (k0 >= end) break;
      load_tile(ta, k0 + STEP);
      __builtin_amdgcn_sched_barrier(0);
      process(tb, k0);
      k0 += STEP;
      if (k0 >= end) break;
    }
  }
  // Sum the per-key-group partial accumulators: lanes with the same dim segment.
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int o = LPK; o < 64; o <<= 1) acc[e] += __shfl_xor(acc[e], o, 64);

  if constexpr (KW > 1) {
    __shared__ float sm[QW][KW], sl[QW][KW];
    __shared__ float sacc[QW][KW][D];
    if (lane == 0) {
      sm[qslot][kw] = m;
      sl[qslot][kw] = l;
    }
    if (kg == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sacc[qslot][kw][8 * ds + e] = acc[e];
    }
    __syncthreads();
    if (kw != 0) return;
    float gm = kNegInf;
#pragma unroll
    for (int w = 0; w < KW; ++w)
      if (sl[qslot][w] > 0.f) gm = fmaxf(gm, sm[qslot][w]);
    float tl = 0.f;
    float tacc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < KW; ++w) {
      if (sl[qslot][w] > 0.f) {
        const float f = __expf(sm[qslot][w] - gm);
        tl += sl[qslot][w] * f;
#pragma unroll
        for (int e = 0; e < 8; ++e) tacc[e] += sacc[qslot][w][8 * ds + e] * f;
      }
    }
    l = tl;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = tacc[e];
  }
  if (qi >= a.q_len || kg != 0) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  uint16_t* op = a.out + int64_t(b) * a.o_sb + int64_t(h) * a.o_sh + int64_t(qi) * a.o_sq + 8 * ds;
  half8_t o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = f16(l > 0.f ? acc[e] * inv : 0.f);
  if constexpr (VEC) *reinterpret_cast<half8_t*>(op) = o;
  else {
#pragma unroll
    for (int e = 0; e < 8; ++e) op[e] = __builtin_bit_cast(uint16_t, o[e]);
  }
}

template <int D, bool VEC>
hipError_t launch(const AttnParams& p, hipStream_t stream) {
  const AttnArgs& a = p.a;
  const dim3 blocks_per(1, unsigned(a.heads), unsigned(a.batch));
  if (a.q_len == 1) {
    // Decode: one workgroup per (b, h) whose KW waves split the keys.  Aim for
    // ~2048 waves in total (every workgroup resident at once: 4-wave groups fit
    // three per CU), never more waves than 32/16-key tiles.
    const int tile_keys = D == 64 ? 32 : 16;
    const int tiles = (a.kv_len + tile_keys - 1) / tile_keys;
    const int64_t groups = int64_t(a.batch) * a.heads;
    int kw = 1;
    while (kw < 16 && kw * 2 <= tiles && groups * kw * 2 <= 2048) kw *= 2;
    dim3 grid = blocks_per;
    grid.x = 1;
    if (a.qkv_partials) {
      if constexpr (D == 64 && VEC) {
        if (kw >= 16) hipLaunchKernelGGL((attention_kernel<64, 1, 16, true, true>), grid, dim3(1024), 0, stream, p);
        else if (kw == 8) hipLaunchKernelGGL((attention_kernel<64, 1, 8, true, true>), grid, dim3(512), 0, stream, p);
        else if (kw == 4) hipLaunchKernelGGL((attention_kernel<64, 1, 4, true, true>), grid, dim3(256), 0, stream, p);
        else if (kw == 2) hipLaunchKernelGGL((attention_kernel<64, 1, 2, true, true>), grid, dim3(128), 0, stream, p);
        else hipLaunchKernelGGL((attention_kernel<64, 1, 1, true, true>), grid, dim3(64), 0, stream, p);
        return hipGetLastError();
      }
      return hipErrorInvalidValue;
    }
    if (kw >= 16) hipLaunchKernelGGL((attention_kernel<D, 1, 16, VEC>), grid, dim3(1024), 0, stream, p);
    else if (kw == 8) hipLaunchKernelGGL((attention_kernel<D, 1, 8, VEC>), grid, dim3(512), 0, stream, p);
    else if (kw == 4) hipLaunchKernelGGL((attention_kernel<D, 1, 4, VEC>), grid, dim3(256), 0, stream, p);
    else if (kw == 2) hipLaunchKernelGGL((attention_kernel<D, 1, 2, VEC>), grid, dim3(128), 0, stream, p);
    else hipLaunchKernelGGL((attention_kernel<D, 1, 1, VEC>), grid, dim3(64), 0, stream, p);
  } else {
    if (a.qkv_partials) return hipErrorInvalidValue;
    dim3 grid = blocks_per;
    grid.x = unsigned((a.q_len + 3) / 4);
    hipLaunchKernelGGL((attention_kernel<D, 4, 1, VEC>), grid, dim3(256), 0, stream, p);
  }
  return hipGetLastError();
}

bool al16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace

hipError_t attention(const AttnArgs& a, hipStream_t stream) {
  if (a.batch <= 0 || a.heads <= 0 || a.q_len <= 0) return hipSuccess;
  AttnParams p{};
  p.a = a;
  p.scale = float(1.0 / __builtin_sqrt(double(a.head_dim)));
  p.vec = al16(a.q) && al16(a.k) && al16(a.v) && al16(a.out) && a.q_sb % 8 == 0 && a.q_sh % 8 == 0 &&
          a.q_sq % 8 == 0 && a.kv_sb % 8 == 0 && a.kv_sh % 8 == 0 && a.o_sb % 8 == 0 &&
          a.o_sh % 8 == 0 && a.o_sq % 8 == 0;
  if (a.head_dim == 64) return p.vec ? launch<64, true>(p, stream) : launch<64, false>(p, stream);
  if (a.head_dim == 128) return p.vec ? launch<128, true>(p, stream) : launch<128, false>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace tia
