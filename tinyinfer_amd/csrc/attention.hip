// Attention for gfx950: fused QK^T, online softmax and PV with fp32 state.
//
// Lane layout inside a wave (head_dim D, LPK = D/8 lanes per key):
//   lane = key_group * LPK + dim_segment; each lane holds 8 consecutive dims
//   (16 bytes) of one key, so a wave-wide load covers 64/LPK whole keys (128 or
//   256 contiguous bytes each) and both K and V are read exactly once, fully
//   coalesced, from either the packed [B,H,K,D] ABI layout or the runtime's
//   [slot][layer][head][pos][64] cache.  The q.k dot finishes with a DPP
//   butterfly inside the LPK lanes of a key group; each key group keeps its
//   own online-softmax state, so probabilities never leave the lanes that own
//   the key (PV needs no broadcast) and the groups merge once per wave.
// A workgroup serves QW queries with KW waves each: KW > 1 splits the keys of a
// query across waves (decode, where one (b, h) row otherwise gives only
// B*H waves) and merges their (m, l, acc) states through LDS.
// Semantics follow reference kernels/src/cuda/tc/attention.cu:29-56: scores
// are dot(q,k) * D^-1/2, keys j < kv_valid (and j <= offset + qi when causal),
// rows with no visible key (or padded queries) are exactly zero.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"
#include "queue_scratch.hpp"

namespace tia {
namespace {

constexpr float kNegInf = -__builtin_huge_valf();

// Split decode of the C ABI: per hardware queue, 2 MiB of chunk states (acc
// [B][H][chunks][D], then (m, l) [B][H][chunks]) and one arrival counter per
// (b, h) row (queue_scratch.hpp); a call beyond either runs the one-pass
// kernel.
constexpr size_t kAttnPoolFloats = size_t(1) << 19;
constexpr int kAttnPoolRows = 4096;
TIA_QUEUE_POOL(attn_pool, kAttnPoolFloats, kAttnPoolRows)

// Offset of query row qi of request b in q or out (batch stride sb, row stride
// sq): b * sb + qi * sq, or (q_row_start[b] + qi) * sq over compact rows.
__device__ __forceinline__ int64_t query_row(const AttnArgs& a, int b, int qi, int64_t sb, int64_t sq) {
  return a.q_row_start ? (int64_t(a.q_row_start[b]) + qi) * sq : int64_t(b) * sb + int64_t(qi) * sq;
}
// Queries of request b whose output rows are written: its q_len slots, or over
// compact rows (where the next request's rows follow) only its q_valid own.
__device__ __forceinline__ int written_queries(const AttnArgs& a, int q_valid) {
  return a.q_row_start ? q_valid : a.q_len;
}

struct AttnParams {
  AttnArgs a;
  float scale;
  bool vec;       // every pointer and stride allows 16-byte accesses
  bool split;     // split decode: key chunks of each (b, h) over workgroups, each
                  // chunk's (m, l, unnormalized acc) in the queue's pool slot,
                  // merged by the row's last chunk to finish
  int chunks;     // split decode: key chunks per (b, h)
};

template <bool VEC>
__device__ __forceinline__ half8_t load8(const uint16_t* p) {
  if constexpr (VEC) return __builtin_nontemporal_load(reinterpret_cast<const half8_t*>(p));
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

template <int D, int QW, int KW, bool VEC, bool FUSEDQKV = false, bool SPLIT = false>
__global__ __launch_bounds__(QW * KW * 64) void attention_kernel(AttnParams p) {
  // A tile is NI wave-wide loads: D=64 -> 32 keys, D=128 -> 16 keys; a wave
  // loads two tiles at a time.
  constexpr int LPK = D / 8, KPI = 64 / LPK, NI = 4, TK = NI * KPI;
  const AttnArgs& a = p.a;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kg = lane / LPK, ds = lane % LPK;
  const int qslot = wave / KW, kw = wave % KW;
  // Split decode: grid (heads, batch, key chunks of 2 * KW tiles), one query; the
  // chunk index varies slowest so every (b, h)'s first chunks are dispatched
  // before any trailing (often empty) ones.
  const int qi = SPLIT ? 0 : blockIdx.x * QW + qslot;
  const int h = SPLIT ? blockIdx.x : blockIdx.y, b = SPLIT ? blockIdx.y : blockIdx.z;
  const int chunk_id = SPLIT ? int(blockIdx.z) : 0;
  const int64_t slot = a.kv_slot ? int64_t(a.kv_slot[b]) : int64_t(b);
  const uint16_t* kb = a.k + slot * a.kv_sb + int64_t(h) * a.kv_sh + 8 * ds;
  const uint16_t* vb = a.v + slot * a.kv_sb + int64_t(h) * a.kv_sh + 8 * ds;
  constexpr int STEP = TK * KW;

  // Split decode, chunk 0: q and both tiles are loaded before the lengths
  // arrive, keys clamped to kv_len - 1 (inside the cache whatever the
  // lengths) instead of end - 1, so the chunk's bytes stream during the
  // lengths' round trip; keys past end are masked in `process`, their V by a
  // select (that memory may hold anything, NaN included).  configs[3]:
  // 14.8-14.9 -> 14.4-14.6 us per call.
  KVTile<NI> ea, eb;
  half8_t eq = {};
  if constexpr (SPLIT) {
    if (chunk_id == 0) {
      eq = load8<VEC>(a.q + query_row(a, b, 0, a.q_sb, a.q_sq) + int64_t(h) * a.q_sh + 8 * ds);
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int k1 = min(kw * TK + kg + KPI * i, a.kv_len - 1);
        const int k2 = min(kw * TK + STEP + kg + KPI * i, a.kv_len - 1);
        ea.k[i] = load8<VEC>(kb + int64_t(k1) * D);
        ea.v[i] = load8<VEC>(vb + int64_t(k1) * D);
        eb.k[i] = load8<VEC>(kb + int64_t(k2) * D);
        eb.v[i] = load8<VEC>(vb + int64_t(k2) * D);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // the loads ahead of the lengths' wait
  }

  const int q_valid = max(0, min(a.q_len, a.q_lengths[b]));
  int end = 0;
  if (qi < q_valid) {
    const int64_t off = a.offsets ? int64_t(a.offsets[b]) : 0;
    const int64_t kvv = a.kv_from_offsets ? off + q_valid
                                          : int64_t(max(0, min(a.kv_len, a.kv_lengths[b])));
    const int64_t bound = a.causal ? off + qi + 1 : kvv;
    end = int(max<int64_t>(0, min<int64_t>(bound, kvv)));
  }
  // Keys [kbeg, end) of this workgroup.
  constexpr int CHUNK = 2 * KW * TK;
  const int kbeg = chunk_id * CHUNK;
  // Split decode: the row's chunks that hold a visible key (at least chunk 0,
  // which writes a row with no visible key); the others do nothing.
  const int active = max(1, min(p.chunks, (end + CHUNK - 1) / CHUNK));
  if constexpr (SPLIT) {
    if (chunk_id >= active) return;
    end = min(end, kbeg + CHUNK);
  }

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
  const int k_first = kbeg + kw * TK;
  KVTile<NI> ta0, tb0;  // FUSEDQKV: the first pair, loaded before q, k, v are known
  half8_t kfresh = {}, vfresh = {};
  half8_t qf = {};
  if constexpr (FUSEDQKV) {
    // Wave 0 finishes the deferred QKV GEMM for this (b, h): lane d sums the
    // split-K partials of q, k and v (bias added, fp16 rounding as the QKV
    // output), stores k and v into the cache at the new position, and shares q
    // through LDS.  The barrier orders those stores before any tile load.
    static_assert(D == 64 && QW == 1, "fused QKV decode is for 64-dim heads, one query");
    __shared__ f16 sq[64], sk[64], sv[64];
    // The first pair of tiles is already in flight while the new token's q, k,
    // v are summed; its key end - 1 (the new token, not yet in the cache when
    // loaded) is taken from LDS when scored.
    if (k_first < end) {
      load_tile(ta0, k_first);
      load_tile(tb0, k_first + STEP);
    }
    __builtin_amdgcn_sched_barrier(0);
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
      sq[lane] = f16r(((sqv[0] + sqv[1]) + (sqv[2] + sqv[3])) + bqv);
      const f16 kn = f16r(((skv[0] + skv[1]) + (skv[2] + skv[3])) + bkv);
      const f16 vn = f16r(((svv[0] + svv[1]) + (svv[2] + svv[3])) + bvv);
      sk[lane] = kn;
      sv[lane] = vn;
      const int64_t pos = a.offsets[b];
      const int64_t at = slot * a.kv_sb + int64_t(h) * a.kv_sh + pos * D + lane;
      const_cast<uint16_t*>(a.k)[at] = __builtin_bit_cast(uint16_t, kn);
      const_cast<uint16_t*>(a.v)[at] = __builtin_bit_cast(uint16_t, vn);
    }
    // LDS only: this workgroup never reads the new cache entry back (later
    // kernels do, after the kernel boundary), and the tile loads stay in flight.
    lds_barrier();
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      qf[e] = sq[8 * ds + e];
      kfresh[e] = sk[8 * ds + e];
      vfresh[e] = sv[8 * ds + e];
    }
  }
  // Unfused: q is re-read with each pair of tiles (an L2 hit after the first)
  // rather than once up front, which would make the compiler wait for it
  // before issuing any K/V load.
  const uint16_t* qptr = a.q + query_row(a, b, qi, a.q_sb, a.q_sq) + int64_t(h) * a.q_sh + 8 * ds;

  float m = kNegInf, l = 0.f;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};

  // Online softmax per key group: the LPK lanes of a key group keep their own
  // (m, l, acc) over the keys they own, so a tile needs no cross-group
  // communication; the dot product of a key finishes with a DPP butterfly
  // inside its group (row_mirror for 16 lanes, row_half_mirror, then two
  // quad_perm steps: every lane of the group ends with the full sum).  The
  // groups merge once, after the last tile.
  auto dpp_add = [](float x, int ctrl_sel) {
    int v = __builtin_bit_cast(int, x);
    switch (ctrl_sel) {
      case 0: v = __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false); break;  // row_mirror
      case 1: v = __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false); break;  // row_half_mirror
      case 2: v = __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false); break;   // quad_perm [1,0,3,2]
      default: v = __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false); break;  // quad_perm [2,3,0,1]
    }
    return x + __builtin_bit_cast(float, v);
  };
  auto group_sum = [&](float x) {
    static_assert(LPK == 8 || LPK == 16, "key groups of 8 or 16 lanes");
    if constexpr (LPK == 16) x = dpp_add(x, 0);
    x = dpp_add(x, 1);
    x = dpp_add(x, 2);
    return dpp_add(x, 3);
  };
  // PLAIN: every key of the tile is visible and none is the new token (the
  // FUSEDQKV substitution), so the masks and selects below are no-ops and are
  // left out (the same values, ~40 % fewer VALU instructions per tile).
  auto process_t = [&](auto plain_c, const KVTile<NI>& t, int k0, const half8_t& qf, bool select_v) {
    constexpr bool PLAIN = decltype(plain_c)::value;
    float s[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int key = k0 + kg + KPI * i;
      float part = 0.f;
      const half8_t kv8 = !PLAIN && FUSEDQKV && key >= end - 1 ? kfresh : t.k[i];
#pragma unroll
      for (int e = 0; e < 8; ++e) part += float(qf[e]) * float(kv8[e]);
      part = group_sum(part);
      s[i] = PLAIN || key < end ? part * p.scale : kNegInf;
    }
    float tmax = s[0];
#pragma unroll
    for (int i = 1; i < NI; ++i) tmax = fmaxf(tmax, s[i]);
    const float nm = fmaxf(m, tmax);
    const float alpha = l == 0.f ? 0.f : __expf(m - nm);
    l *= alpha;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= alpha;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int key = k0 + kg + KPI * i;
      const float pr = PLAIN || key < end ? __expf(s[i] - nm) : 0.f;
      l += pr;
      const half8_t vv8 = !PLAIN && FUSEDQKV && key >= end - 1 ? vfresh : t.v[i];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += !PLAIN && select_v && key >= end ? 0.f : pr * float(vv8[e]);
    }
    m = nm;
  };
  // The tile test is uniform over the wave (k0 and end are), so it is a scalar
  // branch between the two forms.
  auto process = [&](const KVTile<NI>& t, int k0, const half8_t& qf, bool select_v = false) {
    const bool plain = FUSEDQKV ? k0 + TK < end : k0 + TK <= end;
    if (__builtin_amdgcn_readfirstlane(int(plain))) process_t(std::true_type{}, t, k0, qf, false);
    else process_t(std::false_type{}, t, k0, qf, select_v);
  };

  // Wave kw takes tiles kw, kw + KW, ... in pairs: both tiles' loads are issued
  // before the first is scored, so a pair costs one memory round trip.  (A
  // loop that issues the next tile while scoring the current one gets a full
  // vmcnt(0) at its header from the compiler, i.e. one round trip per tile.)
  int k0 = k_first;
  if constexpr (FUSEDQKV) {
    if (k0 < end) {
      process(ta0, k0, qf);
      if (k0 + STEP < end) process(tb0, k0 + STEP, qf);
    }
    k0 += 2 * STEP;
  }
  if constexpr (SPLIT) {
    if (chunk_id == 0) {
      // A tile wholly past end leaves (m, l, acc) as they were.
      process(ea, k0, eq, true);
      process(eb, k0 + STEP, eq, true);
      k0 = max(k0, end);
    }
  }
  for (; k0 < end; k0 += 2 * STEP) {
    half8_t qv = qf;
    if constexpr (!FUSEDQKV) qv = load8<VEC>(qptr);
    KVTile<NI> ta, tb;
    load_tile(ta, k0);
    load_tile(tb, k0 + STEP);
    __builtin_amdgcn_sched_barrier(0);  // every load of the pair ahead of the first use
    process(ta, k0, qv);
    if (k0 + STEP < end) process(tb, k0 + STEP, qv);
  }
  // Merge the key groups of this wave (lanes with the same dim segment): common
  // maximum over groups that saw a key, rescale, then sum l and acc.
  {
    float gm = l > 0.f ? m : kNegInf;
#pragma unroll
    for (int o = LPK; o < 64; o <<= 1) gm = fmaxf(gm, __shfl_xor(gm, o, 64));
    const float f = l > 0.f ? __expf(m - gm) : 0.f;
    l *= f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= f;
#pragma unroll
    for (int o = LPK; o < 64; o <<= 1) l += __shfl_xor(l, o, 64);
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int o = LPK; o < 64; o <<= 1) acc[e] += __shfl_xor(acc[e], o, 64);
    m = gm;
  }

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
    m = gm;  // the split pass stores (m, l, acc) as one state
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = tacc[e];
  }
  if constexpr (SPLIT) {
    if (active > 1) {
      // Store this chunk's state; the row's last chunk to arrive merges every
      // chunk's state (common maximum over chunks that saw a key, rescale, sum
      // in chunk order) and writes fp16_rn(acc / l), or 0 when no key was
      // visible.
      const int lane64 = int(threadIdx.x & 63);
      const unsigned long long key = lane64 < kQueueSlots ? attn_pool_keys[lane64] : 0ull;
      const int sl = queue_slot_resolve(attn_pool_keys, key);
      // Layout: acc [row][chunk][D] (a key group's lanes write it as 16-byte
      // pieces), then (m, l) [row][chunk].
      const int64_t row = int64_t(b) * a.heads + h;
      const int64_t states = int64_t(a.batch) * a.heads * p.chunks;
      float* base = attn_pool_data[sl] + row * p.chunks * D;
      float* mlb = attn_pool_data[sl] + states * D + row * p.chunks * 2;
      unsigned* counter = attn_pool_ctr[sl] + row * kCounterStride;
      if (kg == 0) {
        const auto rs = agent_rsrc(attn_pool_data[sl], uint32_t(kAttnPoolFloats * sizeof(float)));
        const uint32_t at = uint32_t(((row * p.chunks + chunk_id) * D + 8 * ds) * sizeof(float));
        st_agent4(rs, at, f32x4_t{acc[0], acc[1], acc[2], acc[3]});
        st_agent4(rs, at + 16, f32x4_t{acc[4], acc[5], acc[6], acc[7]});
        if (lane == 0) {
          st_agent(mlb + 2 * chunk_id, m);
          st_agent(mlb + 2 * chunk_id + 1, l);
        }
      }
      if (!arrive_last(counter, active)) return;
      constexpr int DPL = D / 64;  // dims per lane in the merge
      float gm = kNegInf;
      float tl = 0.f, tacc[DPL] = {};
      if (active <= 8) {
        // Up to 8 chunks (1024 keys at 128 per chunk): every state in one
        // round of loads, the common maximum and the sums from registers.
        float cm[8], cl[8], ca[8][DPL];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const int cc = min(c, active - 1);
          cm[c] = ld_agent(mlb + 2 * cc);
          cl[c] = ld_agent(mlb + 2 * cc + 1);
#pragma unroll
          for (int e = 0; e < DPL; ++e) ca[c][e] = ld_agent(base + cc * D + DPL * lane + e);
        }
#pragma unroll
        for (int c = 0; c < 8; ++c)
          if (c < active && cl[c] > 0.f) gm = fmaxf(gm, cm[c]);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          if (c >= active) break;
          const float f = cl[c] > 0.f ? __expf(cm[c] - gm) : 0.f;
          tl += cl[c] * f;
#pragma unroll
          for (int e = 0; e < DPL; ++e) tacc[e] += ca[c][e] * f;
        }
      }
      for (int c0 = 0; active > 8 && c0 < active; c0 += 8) {
        float cm[8], cl[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const int cc = min(c0 + c, active - 1);
          cm[c] = ld_agent(mlb + 2 * cc);
          cl[c] = ld_agent(mlb + 2 * cc + 1);
        }
#pragma unroll
        for (int c = 0; c < 8; ++c)
          if (c0 + c < active && cl[c] > 0.f) gm = fmaxf(gm, cm[c]);
      }
      for (int c0 = 0; active > 8 && c0 < active; c0 += 8) {
        float cm[8], cl[8], ca[8][DPL];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const int cc = min(c0 + c, active - 1);
          cm[c] = ld_agent(mlb + 2 * cc);
          cl[c] = ld_agent(mlb + 2 * cc + 1);
#pragma unroll
          for (int e = 0; e < DPL; ++e) ca[c][e] = ld_agent(base + cc * D + DPL * lane + e);
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          if (c0 + c >= active) break;
          const float f = cl[c] > 0.f ? __expf(cm[c] - gm) : 0.f;
          tl += cl[c] * f;
#pragma unroll
          for (int e = 0; e < DPL; ++e) tacc[e] += ca[c][e] * f;
        }
      }
      depart(counter);
      uint16_t* op = a.out + int64_t(b) * a.o_sb + int64_t(h) * a.o_sh + DPL * lane;
      const float inv = tl > 0.f ? 1.f / tl : 0.f;
#pragma unroll
      for (int e = 0; e < DPL; ++e) op[e] = f2h(tl > 0.f ? tacc[e] * inv : 0.f);
      return;
    }
    // The row's only chunk finishes as the one-pass kernel does (below).
  }
  if (qi >= written_queries(a, q_valid) || kg != 0) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  uint16_t* op = a.out + (a.out_p32 ? p32_off(b * a.q_len + qi, h * D + 8 * ds)
                                    : query_row(a, b, qi, a.o_sb, a.o_sq) + int64_t(h) * a.o_sh + 8 * ds);
  half8_t o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = f16r(l > 0.f ? acc[e] * inv : 0.f);
  if constexpr (VEC) *reinterpret_cast<half8_t*>(op) = o;
  else {
#pragma unroll
    for (int e = 0; e < 8; ++e) op[e] = __builtin_bit_cast(uint16_t, o[e]);
  }
}

// Prefill (several queries per request) on MFMA, flash-attention style in the
// transposed form, so that no operand ever moves between lanes:
//   S^T = K Q^T   v_mfma_f32_16x16x32_f16, A = 16 keys x 32 dims of K (LDS),
//                 B = Q^T (registers: lane (j, g) holds query j, dims 8g..8g+7);
//                 lane (j, g) receives the scores of query j for keys 4g..4g+3;
//   P^T = exp(S^T - m) rounded to fp16: two 16-key blocks of it side by side
//                 are exactly the B operand of
//   O^T += V^T P^T  v_mfma_f32_16x16x32_f16, A = 16 dims x (two 4-key runs per
//                 lane) of V^T (read from row-major V in LDS by the transposing
//                 ds_read_b64_tr_b16), lane (j, g) accumulates query j's dims
//                 16db + 4g + v;
//   l   += 1 P^T  the same MFMA with an A of ones: the row sums, in every lane.
// So a query's running max, sum and rescale stay in the four lanes (j, g) that
// hold it (cross-lane steps only on tiles that raise the maximum).  A wave
// takes QB blocks of 16 queries; every K and V^T fragment it reads from LDS
// feeds the MFMAs of all QB blocks (LDS reads per MFMA fall by QB: at QB = 1
// the K and V reads of a tile take more LDS cycles than its MFMAs).  A
// workgroup of 4 waves per key group takes 64 QB queries and walks 64-key
// tiles of K and V through double-buffered LDS, stopping at the last key any
// of its queries may see.  The global loads of the next two tiles are in
// flight during a tile's MFMAs (one tile ahead left every tile waiting a full
// memory round trip).  Staging gives each group of 8 lanes one whole key row
// (1 KiB contiguous per wave instruction, conflict-free 16-byte LDS stores).
// K and V rows sit at a pitch of D + 16 halves: measured on gfx950 with
// SQ_LDS_BANK_CONFLICT, the K fragment reads and the transposing V reads are
// conflict-free at D + 16 (64: 80, 128: 144) and conflict on 2/3 to 2x of
// their cycles at D + 8 (and at 160 for D = 128).
// Numerics: scores, max, sum and accumulation in fp32 (exponentials in base 2
// of the log2(e)-scaled scores), probabilities rounded to fp16 for the PV
// product and its row sum (numerator and denominator weigh each key alike);
// rows with no visible key, and padded queries, are exactly zero.  A query's
// sums do not depend on QB (each block's MFMAs see the same operands in the
// same order); they depend on KS (two key groups merge at the end).
// Waves per SIMD the register budget is sized for (two query blocks need
// about 1.5x the registers of one).
constexpr int prefill_waves_per_simd(int d, int ks, int qb) {
  return (d == 64 ? 4 : 2) / ks / qb > 0 ? (d == 64 ? 4 : 2) / ks / qb : 1;
}

// Causal prefill with few query tiles (C ABI): a query tile with at least
// kPrefillSplitTiles key tiles is split into two workgroups over the two halves
// of its key tiles, so the heaviest tiles spread over twice the CUs; each half
// stores its (m, l, acc) state in the calling queue's slot of this pool and the
// tile's last half to arrive merges both (half 0 first).  A queue that finds
// every slot taken runs each tile whole in its first workgroup.
constexpr int kPrefillSlots = 4;
constexpr int kPrefillPoolTiles = 256;
constexpr int kPrefillSplitTiles = 8;
constexpr size_t kPrefillPoolFloats = size_t(kPrefillPoolTiles) * 2 * 256 * (64 / 16 * 4 + 2);  // acc, then (m, l)
TIA_QUEUE_POOL_N(pf_pool, kPrefillSlots, kPrefillPoolFloats, kPrefillPoolTiles)

template <int D, int KS, int QB = 1, bool SPLITKV = false>
__global__ __launch_bounds__(256 * KS, prefill_waves_per_simd(D, KS, QB)) void prefill_mfma_kernel(AttnParams p) {
  static_assert(!SPLITKV || (D == 64 && QB == 1), "split prefill: 64-dim heads, one query block");
  constexpr int BQ = 64 * QB, BT = 64, KPK = D + 16, KPV = D + 16;
  constexpr int SEGS = D / 8;                 // 16-byte pieces per key row
  constexpr int PIECES = BT * SEGS / 256;     // per thread per tile (2 or 4)
  // Dynamic LDS: [2 buffers][KS tiles] of K rows, then of V rows (row-major;
  // the PV operand is read transposed by ds_read_b64_tr_b16).
  extern __shared__ __attribute__((aligned(16))) uint8_t lds_raw[];
  auto ks = reinterpret_cast<f16(*)[KS][BT][KPK]>(lds_raw);
  auto vs = reinterpret_cast<f16(*)[KS][BT][KPV]>(lds_raw + 2 * KS * BT * KPK * sizeof(f16));
  const AttnArgs& a = p.a;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // KS > 1: waves 4g .. 4g + 3 form key group g, which takes tile g of each
  // step (tiles KS s + g); each group stages its own tile and the groups merge
  // at the end.
  const int grp = wave >> 2, qw = wave & 3, gt = int(threadIdx.x & 255);
  const int j = lane & 15, g = lane >> 4;
  // Workgroups go to the 8 XCDs round-robin by linear id.  Taken as is, the
  // grid (query tiles, heads, batch) would give XCD x query tile x (mod 8) of
  // every row, so under the causal mask the XCDs' loads differ by up to 8x at
  // 8 query tiles, and the query tiles of one (b, h) would fetch its K and V into
  // eight L2s.  Instead ids are regrouped into 8 contiguous runs (one per XCD)
  // of whole (b, h) rows, and within a row the query tiles alternate light and
  // heavy (0, n-1, 1, n-2, ...), so a run that splits a row is balanced too.
  // SPLITKV: an XCD's run of R ids (R even) holds half 0 of its R / 2 tiles
  // in its first R / 2 ids and half 1 of the same tiles, in reverse order, in
  // the rest, so the two workgroups a CU takes in turn (run positions c and
  // c + R / 2) pair a light tile's half with a heavy tile's.
  int b, h, q0, part = 0, tile_id = 0;
  {
    constexpr int PARTS = SPLITKV ? 2 : 1;
    const int nx = int(gridDim.x), nq = nx / PARTS, nh = int(gridDim.y);
    const int n = nx * nh * int(gridDim.z);
    const int id = int(blockIdx.x) + nx * (int(blockIdx.y) + nh * int(blockIdx.z));
    int li;
    if constexpr (SPLITKV) {
      const int n16 = n & ~15;
      if (id < n16) {
        const int c = id >> 3, run = n16 >> 3, half = run >> 1;
        part = c < half ? 0 : 1;
        li = (id & 7) * half + (c < half ? c : run - 1 - c);
      } else {
        part = id & 1;
        li = id >> 1;
      }
    } else {
      const int n8 = n & ~7;
      li = id < n8 ? (id & 7) * (n8 >> 3) + (id >> 3) : id;
    }
    tile_id = li;
    const int k = li % nq, row = li / nq;
    h = row % nh;
    b = row / nh;
    q0 = ((k & 1) ? nq - 1 - (k >> 1) : (k >> 1)) * BQ;
  }

  const int q_valid = max(0, min(a.q_len, a.q_lengths[b]));
  const int64_t off = a.offsets ? int64_t(a.offsets[b]) : 0;
  const int kvv = int(a.kv_from_offsets ? off + q_valid : max(0, min(a.kv_len, a.kv_lengths[b])));
  const int last_q = min(q0 + BQ, q_valid) - 1;
  const int key_end = last_q < q0 ? 0 : int(min<int64_t>(kvv, a.causal ? off + last_q + 1 : kvv));
  const int ntiles = (key_end + BT - 1) / BT;
  // Key tiles [t_begin, t_end) of this workgroup.
  int t_begin = 0, t_end = ntiles, pf_slot = -1;
  if constexpr (SPLITKV) {
    if (ntiles >= kPrefillSplitTiles) pf_slot = queue_slot_claim(pf_pool_keys, kPrefillSlots);
    if (pf_slot < 0 && part == 1) return;  // the whole tile runs in part 0
    if (pf_slot >= 0) {
      const int half = (ntiles + 1) / 2;
      t_begin = part * half;
      t_end = min(ntiles, t_begin + half);
    }
  }
  const int nsteps = (t_end - t_begin + KS - 1) / KS;
  const int64_t slot = a.kv_slot ? int64_t(a.kv_slot[b]) : int64_t(b);
  const uint16_t* kbase = a.k + slot * a.kv_sb + int64_t(h) * a.kv_sh;
  const uint16_t* vbase = a.v + slot * a.kv_sb + int64_t(h) * a.kv_sh;
  // This wave's queries are wq0 .. wq0 + 16 QB - 1, block u holding wq0 + 16 u
  // + j in lane (j, g).  Query my_q[u] sees keys [0, my_end[u]); every valid
  // query of the wave sees at least [0, my_end_min) (its first query's range),
  // so tiles below that need no mask.
  const int wq0 = q0 + 16 * QB * qw;
  int my_q[QB], my_end[QB];
#pragma unroll
  for (int u = 0; u < QB; ++u) {
    my_q[u] = wq0 + 16 * u + j;
    my_end[u] = my_q[u] < q_valid ? int(min<int64_t>(kvv, a.causal ? off + my_q[u] + 1 : kvv)) : 0;
  }
  const int my_end_min = (wq0 + 16 * QB - 1 < q_valid) ? int(min<int64_t>(kvv, a.causal ? off + wq0 + 1 : kvv)) : 0;
  const int wave_end =
      wq0 < q_valid ? int(min<int64_t>(kvv, a.causal ? off + min(wq0 + 16 * QB - 1, q_valid - 1) + 1 : kvv)) : 0;

  half8_t qf[QB][D / 32];
#pragma unroll
  for (int u = 0; u < QB; ++u) {
    const uint16_t* qp =
        a.q + query_row(a, b, min(my_q[u], max(q_valid, 1) - 1), a.q_sb, a.q_sq) + int64_t(h) * a.q_sh;
#pragma unroll
    for (int s = 0; s < D / 32; ++s) {
      qf[u][s] = *reinterpret_cast<const half8_t*>(qp + 32 * s + 8 * g);
      if (my_q[u] >= q_valid) qf[u][s] = half8_t{};
    }
  }

  // Cooperative tile staging: each group of 256 threads stages its tile of a
  // step; piece r of group thread t is key (t + 256 r) / SEGS, 8 dims at
  // ((t + 256 r) % SEGS) * 8; keys past key_end re-read key_end - 1.  Two
  // register sets hold the next two steps.
  struct Staged {
    half8_t k[PIECES], v[PIECES];
  };
  Staged st0, st1;
  auto load_tile = [&](Staged& r_, int step) {
    const int t = t_begin + step * KS + grp;
#pragma unroll
    for (int r = 0; r < PIECES; ++r) {
      const int piece = gt + 256 * r, key = piece / SEGS, seg = piece % SEGS;
      const int64_t kk = min(t * BT + key, key_end - 1);
      r_.k[r] = *reinterpret_cast<const half8_t*>(kbase + kk * D + 8 * seg);
      r_.v[r] = *reinterpret_cast<const half8_t*>(vbase + kk * D + 8 * seg);
    }
  };
  auto store_tile = [&](const Staged& r_, int buf) {
#pragma unroll
    for (int r = 0; r < PIECES; ++r) {
      const int piece = gt + 256 * r, key = piece / SEGS, seg = piece % SEGS;
      *reinterpret_cast<half8_t*>(&ks[buf][grp][key][8 * seg]) = r_.k[r];
      *reinterpret_cast<half8_t*>(&vs[buf][grp][key][8 * seg]) = r_.v[r];
    }
  };

  float m[QB];
  float4_t accl[QB];  // every entry: the running sum l of this lane's query
  float4_t acc[QB][D / 16];
#pragma unroll
  for (int u = 0; u < QB; ++u) {
    m[u] = kNegInf;
    accl[u] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < D / 16; ++d) acc[u][d] = float4_t{0.f, 0.f, 0.f, 0.f};
  }

  // Step s (tiles s * KS + group) sits in LDS buffer s & 1; its registers were
  // set s & 1 (st0 / st1).
  if (nsteps > 0) {
    load_tile(st0, 0);
    store_tile(st0, 0);
  }
  if (nsteps > 1) load_tile(st1, 1);
  if (nsteps > 2) load_tile(st0, 2);
  __syncthreads();
  // One step: the math on buffer s & 1, then step s + 1 from its registers into
  // the other buffer (its loads were issued two steps ago), then the loads of
  // step s + 3 into the registers just freed.
  auto step = [&](int s_, Staged& next) {
    const int buf = s_ & 1, t = t_begin + s_ * KS + grp;
    // This wave's queries see nothing of this tile: skip the math, keep the barriers.
    if (t < t_end && wq0 < q_valid && t * BT < wave_end) {
      float4_t sc[QB][4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int u = 0; u < QB; ++u) sc[u][kb] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < D / 32; ++s) {
          const half8_t kf = *reinterpret_cast<const half8_t*>(&ks[buf][grp][16 * kb + j][32 * s + 8 * g]);
#pragma unroll
          for (int u = 0; u < QB; ++u) sc[u][kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[u][s], sc[u][kb], 0, 0, 0);
        }
      }
      // Scores in base 2: x = s * D^-1/2 * log2(e), p = 2^(x - ref), the scaling
      // folded into the exponent's fma (the maximum is taken on the raw scores:
      // scaling by a positive constant keeps their order).  Keys past a
      // query's end are masked only on tiles that reach some query's end (a
      // wave-uniform test).  The reference ref is raised only when a score
      // exceeds it by more than 8 (p <= 256 stays exact enough in fp16 and the
      // sums are fp32), so acc and l are rescaled on few tiles, not every tile;
      // a lane's own maximum decides whether any query of the block may raise,
      // and only then are the four lanes of each query reduced.
      // P^T as two B operands of v_mfma_f32_16x16x32_f16: pair c holds, in
      // lane (j, g), the probabilities of keys 32c + 4g + v and 32c + 16 + 4g + v
      // (v < 4), and the A operand (V^T) takes the same two 4-key runs of each
      // dim row.  A third A operand of ones gives every lane the row sum
      // l = sum of the fp16 probabilities, in fp32, with no cross-lane step.
      // ds_read_b64_tr_b16 on 16-lane groups: value k of lane r comes from the
      // address of lane 4k + r/4 of its group, element r % 4.  Lane (j, g)
      // therefore points at row 4g + j/4 (+ 32c, + 16 for the second run),
      // dims 16d + 4 (j % 4) .. + 3, so that lane (j, g) receives V[32c + 4g +
      // k][16d + j], k < 4: the A operand V^T of the key runs described above.
      auto vfrag = [&](half8_t (&vf)[D / 16], int c) {
#pragma unroll
        for (int d = 0; d < D / 16; ++d) {
          typedef __fp16 tr_vec __attribute__((vector_size(8)));
          typedef __attribute__((address_space(3))) tr_vec lds_tr_vec;
          const f16* vrow = &vs[buf][grp][32 * c + 4 * g + (j >> 2)][16 * d + 4 * (j & 3)];
          const half4_t lo = __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_tr_vec*)(vrow)));
          const half4_t hi =
              __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_tr_vec*)(vrow + 16 * KPV)));
          vf[d] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        }
      };
      // The first key pair's V^T fragments are read while the exponentials run,
      // the second's during the first pair's MFMAs.
      half8_t vf[D / 16];
      vfrag(vf, 0);
      const float l2s = p.scale * 1.4426950408889634f;
      const bool full = t * BT + BT <= my_end_min;
      half8_t pp[QB][2];
#pragma unroll
      for (int u = 0; u < QB; ++u) {
        float tmax = kNegInf;
        if (full) {
#pragma unroll
          for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int v = 0; v < 4; ++v) tmax = fmaxf(tmax, sc[u][kb][v]);
        } else {
          const int lim = my_end[u] - t * BT - 4 * g;  // key 16 kb + v of this lane is visible iff < lim
#pragma unroll
          for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              sc[u][kb][v] = 16 * kb + v < lim ? sc[u][kb][v] : kNegInf;
              tmax = fmaxf(tmax, sc[u][kb][v]);
            }
        }
        if (__ballot(tmax * l2s > m[u] + 8.f)) {
          tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
          tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64)) * l2s;
          const bool raise = tmax > m[u] + 8.f;
          const float nref = raise ? tmax : m[u];
          const float alpha = accl[u][0] == 0.f ? 0.f : __builtin_amdgcn_exp2f(m[u] - nref);
          accl[u][0] *= alpha;
#pragma unroll
          for (int d = 0; d < D / 16; ++d) acc[u][d] *= alpha;
          m[u] = nref;
        }
        const float base = m[u] == kNegInf ? 0.f : m[u];  // -inf only while every key so far is masked
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int v = 0; v < 4; ++v)
            pp[u][kb >> 1][4 * (kb & 1) + v] = f16r(__builtin_amdgcn_exp2f(fmaf(sc[u][kb][v], l2s, -base)));
      }
      const half8_t ones = {f16(1.f), f16(1.f), f16(1.f), f16(1.f), f16(1.f), f16(1.f), f16(1.f), f16(1.f)};
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        half8_t vn[D / 16];
        if (c == 0) vfrag(vn, 1);
#pragma unroll
        for (int d = 0; d < D / 16; ++d)
#pragma unroll
          for (int u = 0; u < QB; ++u) acc[u][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[d], pp[u][c], acc[u][d], 0, 0, 0);
#pragma unroll
        for (int u = 0; u < QB; ++u) accl[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pp[u][c], accl[u], 0, 0, 0);
        if (c == 0) {
#pragma unroll
          for (int d = 0; d < D / 16; ++d) vf[d] = vn[d];
        }
      }
    }
    if (s_ + 1 < nsteps) store_tile(next, buf ^ 1);
    __syncthreads();
    if (s_ + 3 < nsteps) load_tile(next, s_ + 3);
  };
  for (int s_ = 0; s_ < nsteps; s_ += 2) {
    step(s_, st1);
    if (s_ + 1 < nsteps) step(s_ + 1, st0);
  }
  if constexpr (KS > 1) {
    // Groups 1 .. KS - 1 hand their (m, l, acc) per lane and block to group 0
    // through LDS (free after the last barrier); group 0 merges them in group
    // order on the largest reference: the states are sums of 2^(x - m).
    constexpr int PER = D / 16 * 4 + 2;
    auto slot = [&](int g) {
      return reinterpret_cast<float*>(lds_raw) + ((g - 1) * 256 + qw * 64 + lane) * PER * QB;
    };
    if (grp >= 1) {
      float* xs = slot(grp);
#pragma unroll
      for (int u = 0; u < QB; ++u) {
#pragma unroll
        for (int d = 0; d < D / 16; ++d)
#pragma unroll
          for (int v = 0; v < 4; ++v) xs[u * PER + 4 * d + v] = acc[u][d][v];
        xs[u * PER + PER - 2] = m[u];
        xs[u * PER + PER - 1] = accl[u][0];
      }
    }
    __syncthreads();
    // (A split tile's groups all take part in the arrival below.)
    if (grp >= 1 && pf_slot < 0) return;
#pragma unroll
    for (int u = 0; grp == 0 && u < QB; ++u) {
      const float l = accl[u][0];
      float nm = l > 0.f ? m[u] : kNegInf;
#pragma unroll
      for (int g = 1; g < KS; ++g) {
        const float* xs = slot(g);
        if (xs[u * PER + PER - 1] > 0.f) nm = fmaxf(nm, xs[u * PER + PER - 2]);
      }
      const float f0 = l > 0.f ? __builtin_amdgcn_exp2f(m[u] - nm) : 0.f;
      // Explicit fmas: with contraction left to the compiler, a * f0 + b * f1
      // may fuse either product, and differently per instantiation (the bits
      // of a query would then depend on QB).
      float tl = l * f0;
#pragma unroll
      for (int d = 0; d < D / 16; ++d)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[u][d][v] *= f0;
#pragma unroll
      for (int g = 1; g < KS; ++g) {
        const float* xs = slot(g);
        const float lg = xs[u * PER + PER - 1];
        const float fg = lg > 0.f ? __builtin_amdgcn_exp2f(xs[u * PER + PER - 2] - nm) : 0.f;
        tl = fmaf(lg, fg, tl);
#pragma unroll
        for (int d = 0; d < D / 16; ++d)
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[u][d][v] = fmaf(xs[u * PER + 4 * d + v], fg, acc[u][d][v]);
      }
      accl[u][0] = tl;
      m[u] = nm;  // the merged state's reference (a split tile's half stores it)
    }
  }
  if constexpr (SPLITKV) {
    if (pf_slot >= 0) {
      // This half's state (group 0's lanes) to the pool, then the arrival;
      // the tile's last half merges half 0's state, then half 1's.  Layout:
      // acc as float4 [tile][half][d][lane] (every store and load instruction
      // one contiguous KiB), then (m, l) pairs [tile][half][lane].
      const int lid = qw * 64 + lane;
      const auto rs = agent_rsrc(pf_pool_data[pf_slot], uint32_t(kPrefillPoolFloats * sizeof(float)));
      auto acc_at = [&](int pt, int d) {
        return uint32_t((((tile_id * 2 + pt) * (D / 16) + d) * 256 + lid) * 16);
      };
      auto ml_at = [&](int pt) {
        return pf_pool_data[pf_slot] + size_t(kPrefillPoolTiles) * 2 * (D / 16) * 256 * 4 +
               (size_t(tile_id * 2 + pt) * 256 + lid) * 2;
      };
      if (grp == 0) {
#pragma unroll
        for (int d = 0; d < D / 16; ++d)
          st_agent4(rs, acc_at(part, d), f32x4_t{acc[0][d][0], acc[0][d][1], acc[0][d][2], acc[0][d][3]});
        st_agent(ml_at(part), m[0]);
        st_agent(ml_at(part) + 1, accl[0][0]);
      }
      unsigned* counter = pf_pool_ctr[pf_slot] + tile_id * kCounterStride;
      // The flag reuses the first word of the tile buffers (read by now): a
      // static LDS word would push two workgroups of 80 KiB past a CU's LDS.
      if (!wg_arrive_last(counter, 2, reinterpret_cast<int*>(lds_raw)) || grp >= 1) return;
      float oacc[D / 16][4];
#pragma unroll
      for (int d = 0; d < D / 16; ++d) {
        const f32x4_t o = ld_agent4(rs, acc_at(1 - part, d));
#pragma unroll
        for (int v = 0; v < 4; ++v) oacc[d][v] = o[v];
      }
      const float om = ld_agent(ml_at(1 - part)), ol = ld_agent(ml_at(1 - part) + 1);
      depart(counter);
      const float mA = part == 0 ? m[0] : om, lA = part == 0 ? accl[0][0] : ol;
      const float mB = part == 0 ? om : m[0], lB = part == 0 ? ol : accl[0][0];
      const float nm = fmaxf(lA > 0.f ? mA : kNegInf, lB > 0.f ? mB : kNegInf);
      const float fA = lA > 0.f ? __builtin_amdgcn_exp2f(mA - nm) : 0.f;
      const float fB = lB > 0.f ? __builtin_amdgcn_exp2f(mB - nm) : 0.f;
      accl[0][0] = fmaf(lB, fB, lA * fA);
#pragma unroll
      for (int d = 0; d < D / 16; ++d)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float aA = part == 0 ? acc[0][d][v] : oacc[d][v], aB = part == 0 ? oacc[d][v] : acc[0][d][v];
          acc[0][d][v] = fmaf(aB, fB, aA * fA);
        }
    }
  }

#pragma unroll
  for (int u = 0; u < QB; ++u) {
    if (my_q[u] >= written_queries(a, q_valid)) continue;
    const float l = accl[u][0];
    const float inv = l > 0.f ? 1.f / l : 0.f;
    uint16_t* op = a.out + query_row(a, b, my_q[u], a.o_sb, a.o_sq) + int64_t(h) * a.o_sh;
#pragma unroll
    for (int d = 0; d < D / 16; ++d) {
      half4_t o;
#pragma unroll
      for (int v = 0; v < 4; ++v) o[v] = f16r(l > 0.f ? acc[u][d][v] * inv : 0.f);
      *reinterpret_cast<half4_t*>(op + 16 * d + 4 * g) = o;
    }
  }
}

// LDS bytes a workgroup may use on the current device (cached per device).
size_t max_lds_per_block() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n > 0) return size_t(n);
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || n <= 0) return 0;
  cached[dev].store(n, std::memory_order_relaxed);
  return size_t(n);
}

// K and V rows (pitch D + 16), two buffers per key group; the key-group merge
// reuses them.
template <int D, int KS, int QB, bool SPLITKV = false>
hipError_t launch_prefill(dim3 grid, const AttnParams& p, hipStream_t stream) {
  constexpr size_t lds = size_t(KS) * 2 * 2 * 64 * (D + 16) * 2;
  static_assert(KS == 1 || size_t(KS - 1) * 256 * (D / 16 * 4 + 2) * QB * 4 <= lds, "merge fits the tile buffers");
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&prefill_mfma_kernel<D, KS, QB, SPLITKV>), hipFuncAttributeMaxDynamicSharedMemorySize,
      int(lds));
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL((prefill_mfma_kernel<D, KS, QB, SPLITKV>), grid, dim3(256 * KS), lds, stream, p);
  return hipGetLastError();
}

template <int D, bool VEC>
hipError_t launch(const AttnParams& p, hipStream_t stream) {
  const AttnArgs& a = p.a;
  const dim3 blocks_per(1, unsigned(a.heads), unsigned(a.batch));
  if (a.q_len == 1) {
    // Decode: one workgroup per (b, h) whose KW waves split the keys.  Each
    // wave keeps at least 4 tiles of 32/16 keys (two double-buffered rounds;
    // fewer make the LDS merge of the waves cost more than the parallelism
    // gains; timed on GPT-2 XL, 640 keys and 800 heads: KW 4), except that a
    // cache of 3 to 7 tiles takes two waves, so every tile's loads go out in
    // one round (GPT-2 small, 96 / 192 keys: b = 1 decode 3.55 -> 3.65 K tok/s
    // at 192, b = 32 unchanged or +0.6 %).  KW follows the cache length only,
    // not the batch, so a request's result does not depend on the requests
    // decoded with it.
    const int tile_keys = D == 64 ? 32 : 16;
    const int tiles = (a.kv_len + tile_keys - 1) / tile_keys;
    int kw = 1;
    while (kw < 8 && kw * 2 * 4 <= tiles) kw *= 2;
    if (kw == 1 && tiles >= 3) kw = 2;
    dim3 grid = blocks_per;
    grid.x = 1;
    if (p.split) {
      // Long caches: 2-wave workgroups over chunks of 2 * 2 tiles (all of a
      // wave's loads in flight at once; 4- and 8-wave chunks of 256 / 512 keys
      // measured slower on configs[3]), spread over every CU; each row's last
      // chunk merges the row.
      const dim3 split_grid(unsigned(a.heads), unsigned(a.batch), unsigned(p.chunks));
      hipLaunchKernelGGL((attention_kernel<D, 1, 2, VEC, false, true>), split_grid, dim3(128), 0, stream, p);
      return hipGetLastError();
    }
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
    if constexpr (VEC) {
      // Few query tiles (<= 512 workgroups of 64 queries, e.g. one long
      // sequence of a few heads): 8 waves per tile in two key groups, so each
      // SIMD holds two waves (causal B1 H4 4096^2: 75 -> 54 us, B1 H12 2048^2:
      // 54 -> 48 us); from 768 workgroups the 4-wave kernel is as fast or
      // faster (B8 H12 512^2: 26 against 28 us, B32 H25 320^2: 55 against 65 us).
      // batch_invariant (the runtime's prefill) always takes one key group,
      // so a query's sums never depend on the grid: batched prefills are the
      // runtime's common case (GPT-2 XL, 32 prompts of ~335
      // tokens: TTFT 56 -> 53.5 ms against the key-split kernel; b = 1 and
      // 32 with 32- and 128-token prompts as fast or faster), and a single
      // long prompt loses only the key split's gain above.  64-dim heads take
      // two 16-query blocks per wave (128 queries per workgroup) once that
      // still leaves enough workgroups (at 128 dims the second block's
      // registers spill).
      const int64_t heads_rows = int64_t(grid.y) * grid.z;
      const int64_t wgs = (a.q_len + 63) / 64 * heads_rows, wgs2 = (a.q_len + 127) / 128 * heads_rows;
      const bool split_keys = wgs <= 512 && !a.batch_invariant;
      const bool two_blocks = D == 64 && (split_keys ? wgs2 >= 512 : wgs2 >= 768);
      grid.x = unsigned(two_blocks ? (a.q_len + 127) / 128 : (a.q_len + 63) / 64);
      if constexpr (D == 64) {
        if (two_blocks)
          return split_keys ? launch_prefill<D, 2, 2>(grid, p, stream) : launch_prefill<D, 1, 2>(grid, p, stream);
        // At most one workgroup per CU.  Causal: the heavy query tiles split
        // their key tiles over two workgroups (the tile count per CU evens
        // out); otherwise every tile is equally heavy, and four key groups
        // (16 waves, all 160 KiB of LDS) give each CU more waves to hide
        // latency with.
        if (split_keys && wgs <= 256 && a.causal && wgs <= kPrefillPoolTiles) {
          dim3 g2 = grid;
          g2.x *= 2;
          return launch_prefill<D, 2, 1, true>(g2, p, stream);
        }
        if (split_keys && wgs <= 256 && max_lds_per_block() >= size_t(4) * 2 * 2 * 64 * (D + 16) * 2)
          return launch_prefill<D, 4, 1>(grid, p, stream);
      }
      return split_keys ? launch_prefill<D, 2, 1>(grid, p, stream) : launch_prefill<D, 1, 1>(grid, p, stream);
    } else {
      grid.x = unsigned((a.q_len + 3) / 4);
      hipLaunchKernelGGL((attention_kernel<D, 4, 1, VEC>), grid, dim3(256), 0, stream, p);
    }
  }
  return hipGetLastError();
}

bool al16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace

hipError_t attention(const AttnArgs& a, hipStream_t stream, const Scratch* scratch) {
  if (a.batch <= 0 || a.heads <= 0 || a.q_len <= 0) return hipSuccess;
  // P32 output: decode rows only (the MFMA prefill kernel writes row-major).
  if (a.out_p32 && (a.q_len != 1 || a.batch > 32 || (a.heads * a.head_dim) % 64 != 0 || !al16(a.out)))
    return hipErrorInvalidValue;
  AttnParams p{};
  p.a = a;
  // Decode over a long cache (at least 4 chunks of 128/64 keys per (b, h)) in
  // the ABI's layout, whose chunk states fit the queue pool slot: split the
  // keys across workgroups.  (The split kernel loads chunk 0 before the
  // lengths, clamped to kv_len - 1, which holds for this layout only: with
  // lengths from offsets a row could see keys past kv_len.)  The choice
  // follows the shape alone.
  if (scratch && scratch->queue_pool && a.q_len == 1 && !a.qkv_partials && !a.kv_slot && !a.kv_from_offsets &&
      !a.q_row_start && !a.out_p32 && (a.head_dim == 64 || a.head_dim == 128)) {
    const int chunk = a.head_dim == 64 ? 128 : 64;  // 2 waves x 2 tiles
    const int chunks = (a.kv_len + chunk - 1) / chunk;
    const int64_t rows = int64_t(a.batch) * a.heads;
    const int64_t need = rows * chunks * (2 + a.head_dim);
    if (chunks >= 4 && chunks <= 32 && rows <= kAttnPoolRows && need <= int64_t(kAttnPoolFloats)) {
      p.split = true;
      p.chunks = chunks;
    }
  }
  p.scale = float(1.0 / __builtin_sqrt(double(a.head_dim)));
  p.vec = al16(a.q) && al16(a.k) && al16(a.v) && al16(a.out) && a.q_sb % 8 == 0 && a.q_sh % 8 == 0 &&
          a.q_sq % 8 == 0 && a.kv_sb % 8 == 0 && a.kv_sh % 8 == 0 && a.o_sb % 8 == 0 &&
          a.o_sh % 8 == 0 && a.o_sq % 8 == 0;
  if (a.head_dim == 64) return p.vec ? launch<64, true>(p, stream) : launch<64, false>(p, stream);
  if (a.head_dim == 128) return p.vec ? launch<128, true>(p, stream) : launch<128, false>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace tia
