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

__device__ __forceinline__ half8_t load8(const uint16_t* p, bool vec) {
  if (vec) return *reinterpret_cast<const half8_t*>(p);
  half8_t out;
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = __builtin_bit_cast(f16, p[i]);
  return out;
}

template <int D, int QW, int KW>
__global__ __launch_bounds__(QW * KW * 64) void attention_kernel(AttnParams p) {
  constexpr int LPK = D / 8, KPI = 64 / LPK, NI = 64 / KPI;
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
  if (qi < q_valid) qf = load8(a.q + int64_t(b) * a.q_sb + int64_t(h) * a.q_sh + int64_t(qi) * a.q_sq + 8 * ds, p.vec);

  float m = kNegInf, l = 0.f;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int k0 = kw * 64; k0 < end; k0 += 64 * KW) {
    // K and V of the whole 64-key tile are requested before any use: one memory
    // round trip per tile.
    half8_t kfr[NI], vfr[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int key = k0 + kg + KPI * i;
      if (key < end) {
        kfr[i] = load8(kb + int64_t(key) * D, p.vec);
        vfr[i] = load8(vb + int64_t(key) * D, p.vec);
      } else {
        kfr[i] = half8_t{};
        vfr[i] = half8_t{};
      }
    }
    float s[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int key = k0 + kg + KPI * i;
      float part = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) part += float(qf[e]) * float(kfr[i][e]);
#pragma unroll
      for (int o = LPK / 2; o > 0; o >>= 1) part += __shfl_xor(part, o, 64);
      s[i] = key < end ? part * p.scale : kNegInf;
    }
    float tmax = s[0];
#pragma unroll
    for (int i = 1; i < NI; ++i) tmax = fmaxf(tmax, s[i]);
#pragma unroll
    for (int o = LPK; o < 64; o <<= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, o, 64));
    const float nm = fmaxf(m, tmax);  // finite: key k0 + 0 < end is always visible here
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
      for (int e = 0; e < 8; ++e) acc[e] += pr * float(vfr[i][e]);
    }
#pragma unroll
    for (int o = LPK; o < 64; o <<= 1) psum += __shfl_xor(psum, o, 64);
    l = l * alpha + psum;
    m = nm;
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
  if (p.vec) *reinterpret_cast<half8_t*>(op) = o;
  else {
#pragma unroll
    for (int e = 0; e < 8; ++e) op[e] = __builtin_bit_cast(uint16_t, o[e]);
  }
}

template <int D>
hipError_t launch(const AttnParams& p, hipStream_t stream) {
  const AttnArgs& a = p.a;
  const dim3 blocks_per(1, unsigned(a.heads), unsigned(a.batch));
  if (a.q_len == 1) {
    // Split keys across up to 16 waves so one (b, h) fills a CU.
    const int tiles = (a.kv_len + 63) / 64;
    dim3 grid = blocks_per;
    grid.x = 1;
    if (tiles >= 12) hipLaunchKernelGGL((attention_kernel<D, 1, 16>), grid, dim3(1024), 0, stream, p);
    else if (tiles >= 6) hipLaunchKernelGGL((attention_kernel<D, 1, 8>), grid, dim3(512), 0, stream, p);
    else if (tiles >= 3) hipLaunchKernelGGL((attention_kernel<D, 1, 4>), grid, dim3(256), 0, stream, p);
    else if (tiles == 2) hipLaunchKernelGGL((attention_kernel<D, 1, 2>), grid, dim3(128), 0, stream, p);
    else hipLaunchKernelGGL((attention_kernel<D, 1, 1>), grid, dim3(64), 0, stream, p);
  } else {
    dim3 grid = blocks_per;
    grid.x = unsigned((a.q_len + 3) / 4);
    hipLaunchKernelGGL((attention_kernel<D, 4, 1>), grid, dim3(256), 0, stream, p);
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
  if (a.head_dim == 64) return launch<64>(p, stream);
  if (a.head_dim == 128) return launch<128>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace tia
