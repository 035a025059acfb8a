// libtinyinfer_llm.so: the GPT-2 runtime ABI (include/tinyinfer_llm.h) on gfx950.
//
// Semantics follow reference llm/src/runtime.cu:86-211 (validation rules,
// absolute positions, greedy loop, poisoning, internal scoring slot, trace
// counters); the execution plan is MI355X-native:
//  * the embedding kernel also computes layer 0's LN1; per layer: c_attn GEMM
//    whose epilogue also writes K/V into the slot cache (no split/scatter/
//    gather/pack kernels) -> attention reading the [slot][layer][head][pos][64]
//    cache in place and writing merged heads -> c_proj GEMM -> one kernel that
//    reduces its split-K partials, adds bias and residual (in place) and applies
//    LN2 -> c_fc GEMM with fused bias + GELU -> mlp.c_proj GEMM -> the same
//    reduce + residual kernel applying the next layer's LN1 (ln_f after the last);
//  * decode of up to 32 requests over packed int8 weights instead runs ln_1
//    and ln_2 in the prologue of the GEMV that consumes them (c_attn, c_fc)
//    and each residual add in the epilogue of the GEMV that produces it: per
//    layer c_attn (split-K partials) -> attention (finishes q/k/v) -> c_proj
//    (+residual) -> c_fc (LN2, GELU) -> mlp.c_proj (+residual), five launches,
//    and ln_f as a row kernel before the head;
//  * the lm_head GEMM writes fp32 logits of each request's last row (padded row
//    pitch), a block-per-row argmax picks the lowest id on ties;
//  * a decode step (every request appends one token) is captured once per
//    batch size into a hipGraph whose kernels read all lengths, offsets and slots
//    from device memory, so later steps are one graph launch between a pinned
//    H2D copy of the step metadata and a D2H copy of the next tokens;
//  * the captured step ends with greedy_feed_kernel (each greedy id is
//    recorded, becomes the next step's input with its embedding and ln_1
//    written, positions advance by one), so ti_llm_greedy_batch queues each
//    run of decode steps over an unchanged set of requests back to back and
//    waits once per run;
//  * such a run of more than kLaneRows requests, over int8 weights that fit
//    the Infinity Cache, splits evenly over lanes of at most kLaneRows, each
//    with its own stream, activations, scratch and captured graph over the
//    shared weights and KV cache, queued side by side: one lane's chain of 63
//    dependent launches leaves most CUs idle, and free-running chains fill
//    them.  A request's logits are the same bits in any lane, since the
//    decode kernels sum every row in one K order at every batch size.
#include <algorithm>
#include <chrono>
#include <climits>
#include <cmath>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <vector>

#include "../../include/tinyinfer_backend_v2.h"
#include "../../include/tinyinfer_llm.h"
#include "artifact.hpp"
#include "common.hpp"
#include "kernels.hpp"

using tia::art::Invalid;
using tia::art::IOError;

namespace {

thread_local std::string error_text;
constexpr int kScoreRows = 16;
constexpr int kHeadDim = 64;
// Workgroups a split residual GEMV (decode above hidden 1024) aims at: two K
// splits of the XL residual GEMVs (100 column blocks).  Timed at XL decode,
// 64 requests: 192 -> 12.06 K tok/s, 384 -> 11.66 K (unsplit with a separate
// LayerNorm row kernel: 11.4 K).
constexpr int kResidualSplitWorkgroups = 192;
// Decode steps of more than this many requests run as two concurrent lanes.
constexpr int kLanes = 2, kLaneRows = 16;
// Lanes pay when the second lane finds the weight records the first just read
// in cache: the decode's int8 weights must fit the 256 MiB Infinity Cache
// (GPT-2 small, 124 MB: b = 32 102 K tok/s with two lanes against 90 K with
// one; GPT-2 XL, 1.6 GB: 11.1 K with two against 11.8 K with one).
constexpr size_t kLaneWeightBytes = size_t(256) << 20;
static_assert(kLanes * kLaneRows >= 32, "the lanes must hold a full decode batch");

struct GpuError : std::runtime_error {
  using std::runtime_error::runtime_error;
};
void ck(hipError_t e) {
  if (e != hipSuccess) throw GpuError(hipGetErrorString(e));
}

struct DeviceScope {
  int previous = -1;
  bool changed = false;
  explicit DeviceScope(int device) {
    ck(hipGetDevice(&previous));
    if (previous != device) {
      ck(hipSetDevice(device));
      changed = true;
    }
  }
  ~DeviceScope() {
    if (changed) (void)hipSetDevice(previous);
  }
};

// ---------------------------------------------------------------- kernels
// out[b] = x[b * qlen + qlens[b] - 1] (reference runtime.cu:56-58), or
// x[row_start[b] + qlens[b] - 1] over compact rows.
__global__ void gather_last_kernel(const uint16_t* x, uint16_t* out, const int32_t* qlens,
                                   const int32_t* row_start, int batch, int qlen, int hidden) {
  const int per_row = hidden / 8;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= batch * per_row) return;
  const int b = i / per_row, c = (i % per_row) * 8;
  const int64_t first = row_start ? int64_t(row_start[b]) : int64_t(b) * qlen;  // compact or padded rows
  *reinterpret_cast<tia::half8_t*>(out + int64_t(b) * hidden + c) =
      *reinterpret_cast<const tia::half8_t*>(x + (first + qlens[b] - 1) * hidden + c);
}

// One embedding row, x = fp16(wte[id] + wpe[pos]) (zeros when !valid;
// reference runtime.cu:25-30), and the first layer's LayerNorm of it into
// norm: one wave, lane owns the 8-wide column groups lane + 64 i (hidden <=
// 2048).  p32: x and norm are written P32 fragment-packed (rows <= 32, hidden
// % 64 == 0).  The position row and gamma/beta do not depend on the token, so
// a caller that knows the position early fetches them first (EmbedRow::fetch)
// and issues the token-row load alone once the id is known.
struct EmbedRow {
  static constexpr int NV = 4;
  tia::half8_t p[NV], gg[NV], bb[NV];
  __device__ __forceinline__ void fetch(int lane, bool valid, int pos, const uint16_t* wpe, const uint16_t* g,
                                        const uint16_t* bt, int hidden) {
    const int groups = hidden / 8;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int gi = min(lane + 64 * i, groups - 1);
      p[i] = *reinterpret_cast<const tia::half8_t*>(wpe + int64_t(valid ? pos : 0) * hidden + 8 * gi);
      gg[i] = *reinterpret_cast<const tia::half8_t*>(g + 8 * gi);
      bb[i] = *reinterpret_cast<const tia::half8_t*>(bt + 8 * gi);
    }
  }
  __device__ __forceinline__ void finish(int lane, bool valid, int id, const uint16_t* wte, uint16_t* x,
                                         uint16_t* norm, int row, int hidden, bool p32) const {
    const int groups = hidden / 8;
    float v[NV][8];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int gi = lane + 64 * i;
#pragma unroll
      for (int k = 0; k < 8; ++k) v[i][k] = 0.f;
      if (gi < groups) {
        if (valid) {
          const tia::half8_t e = *reinterpret_cast<const tia::half8_t*>(wte + int64_t(id) * hidden + 8 * gi);
#pragma unroll
          for (int k = 0; k < 8; ++k) v[i][k] = float(tia::f16r(float(e[k]) + float(p[i][k])));
        }
        tia::half8_t o;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          o[k] = tia::f16(v[i][k]);
          s += v[i][k];
        }
        *reinterpret_cast<tia::half8_t*>(x + (p32 ? tia::p32_off(row, 8 * gi) : int64_t(row) * hidden + 8 * gi)) = o;
      }
    }
    const float mean = tia::wave_sum(s) / float(hidden);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (lane + 64 * i < groups) {
#pragma unroll
        for (int k = 0; k < 8; ++k) ss += (v[i][k] - mean) * (v[i][k] - mean);
      }
    const float inv = rsqrtf(tia::wave_sum(ss) / float(hidden) + 1e-5f);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int gi = lane + 64 * i;
      if (gi < groups) {
        tia::half8_t o;
#pragma unroll
        for (int k = 0; k < 8; ++k) o[k] = tia::f16r((v[i][k] - mean) * inv * float(gg[i][k]) + float(bb[i][k]));
        *reinterpret_cast<tia::half8_t*>(norm + (p32 ? tia::p32_off(row, 8 * gi) : int64_t(row) * hidden + 8 * gi)) = o;
      }
    }
  }
};

__device__ __forceinline__ void embed_ln_row(int lane, bool valid, int id, int pos, const uint16_t* wte,
                                             const uint16_t* wpe, const uint16_t* g, const uint16_t* bt,
                                             uint16_t* x, uint16_t* norm, int row, int hidden, bool p32) {
  EmbedRow r;
  r.fetch(lane, valid, pos, wpe, g, bt, hidden);
  r.finish(lane, valid, id, wte, x, norm, row, hidden, p32);
}

// Embedding rows of a pass, row = b * qlen + t (or, over compact rows,
// row_start[b] + t), position offsets[b] + t, zero for t >= qlens[b]: one wave
// per row.
__global__ __launch_bounds__(256) void embed_ln_kernel(const int32_t* ids, const int32_t* qlens,
                                                       const int32_t* offsets, const int32_t* row_start, int batch,
                                                       const uint16_t* wte, const uint16_t* wpe, const uint16_t* g,
                                                       const uint16_t* bt, uint16_t* x, uint16_t* norm, int rows,
                                                       int qlen, int hidden, bool p32) {
  const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  int b = row / qlen, t = row - b * qlen;
  if (row_start) {
    int lo = 0, hi = batch;  // row_start[lo] <= row < row_start[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (row_start[mid] <= row) lo = mid;
      else hi = mid;
    }
    b = lo;
    t = row - row_start[lo];
  }
  const bool valid = t < qlens[b];
  const int id = valid ? ids[row] : 0, pos = valid ? offsets[b] + t : 0;
  embed_ln_row(lane, valid, id, pos, wte, wpe, g, bt, x, norm, row, hidden, p32);
}

// Greedy id per row: largest logit, lowest id on ties (reference runtime.cu:59-66).
// One 1024-thread block per row, 16-byte loads over a row pitch `ld` (a multiple
// of 4 floats).
__global__ __launch_bounds__(1024) void argmax_kernel(const float* logits, int32_t* out, int vocab, int64_t ld) {
  __shared__ float sv[16];
  __shared__ int si[16];
  const float* row = logits + int64_t(blockIdx.x) * ld;
  float best = -__builtin_huge_valf();
  int idx = INT_MAX;
  const int vec = vocab / 4;
  // Four 16-byte loads per thread in flight at a time.
  for (int j0 = threadIdx.x; j0 < vec; j0 += 4 * 1024) {
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const float4*>(row + 4 * min(j0 + u * 1024, vec - 1));
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j4 = j0 + u * 1024;
      const float e[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (j4 < vec && e[k] > best) {  // ids visited in increasing order: equality keeps the lower id
          best = e[k];
          idx = 4 * j4 + k;
        }
    }
  }
  for (int j = 4 * vec + threadIdx.x; j < vocab; j += 1024)
    if (row[j] > best) {
      best = row[j];
      idx = j;
    }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(idx, o, 64);
    if (ov > best || (ov == best && oi < idx)) {
      best = ov;
      idx = oi;
    }
  }
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = best;
    si[threadIdx.x >> 6] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 16; ++w)
      if (sv[w] > best || (sv[w] == best && si[w] < idx)) {
        best = sv[w];
        idx = si[w];
      }
    out[blockIdx.x] = idx;
  }
}

// Shifted-target NLL of one row in fp64 (reference runtime.cu:67-76).
__global__ __launch_bounds__(256) void nll_kernel(const float* logits, const int32_t* tokens,
                                                  const uint8_t* mask, double* loss, int first_position,
                                                  int vocab, int64_t ld) {
  __shared__ float smax[4];
  __shared__ double ssum[4];
  const int row = blockIdx.x, pos = first_position + row;
  const float* l = logits + int64_t(row) * ld;
  float m = -__builtin_huge_valf();
  for (int j = threadIdx.x; j < vocab; j += 256) m = fmaxf(m, l[j]);
  m = tia::wave_max(m);
  if ((threadIdx.x & 63) == 0) smax[threadIdx.x >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(smax[0], smax[1]), fmaxf(smax[2], smax[3]));
  double s = 0;
  for (int j = threadIdx.x; j < vocab; j += 256) s += exp(double(l[j]) - double(m));
  s = tia::wave_sum_d(s);
  if ((threadIdx.x & 63) == 0) ssum[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    const double total = ssum[0] + ssum[1] + ssum[2] + ssum[3];
    loss[pos] = mask[pos] ? double(m) + log(total) - double(l[tokens[pos]]) : 0.0;
  }
}

__global__ __launch_bounds__(256) void sum_kernel(const double* v, double* out, int n) {
  __shared__ double s[4];
  double acc = 0;
  for (int i = threadIdx.x; i < n; i += 256) acc += v[i];
  acc = tia::wave_sum_d(acc);
  if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) *out = s[0] + s[1] + s[2] + s[3];
}

// End of a captured decode step, one workgroup per request row (1024 threads
// over partials, else 64):
//  * the row's greedy id: from the head GEMV's per-workgroup partials (largest
//    value, lowest id on ties: the same id in any merge order), or already in
//    next[row] when groups == 0;
//  * next[row] = id and run[pos * b + row] = id, pos = offsets[row] the
//    position of the step's input token, so a run of steps leaves every id on
//    the device;
//  * the id is the next step's input: ids[row] = id, offsets[row] = pos + 1,
//    and its embedding row with the first LayerNorm is written now (the
//    embedding kernel's work), so the next step starts at layer 0.  An id
//    outside the vocabulary (non-finite logits) is recorded as is for the host
//    to reject and embedded as 0; no embedding is written past the last
//    position.
struct FeedArgs {
  const float* vals;
  const int32_t* idx;
  int groups;
  int32_t *next, *ids, *offsets, *run;
  int b, vocab, positions, hidden;
  const uint16_t *wte, *wpe, *g, *bt;
  uint16_t *x, *norm;
  bool p32;
};

__global__ __launch_bounds__(1024) void greedy_feed_kernel(FeedArgs a) {
  __shared__ float sv[16];
  __shared__ int si[16];
  const int row = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nt = blockDim.x;
  // Wave 0 reads the row's position and fetches the next position's wpe row
  // and ln_1's gamma/beta while the partials are merged: only the token row
  // waits for the id.
  int pos = 0;
  EmbedRow emb;
  if (wave == 0) {
    pos = a.offsets[row];
    emb.fetch(lane, pos + 1 < a.positions, pos + 1, a.wpe, a.g, a.bt, a.hidden);
  }
  int id;
  if (a.groups > 0) {
    // Four partials per thread in flight at a time.
    float v = -__builtin_huge_valf();
    int i = INT_MAX;
    for (int g0 = threadIdx.x; g0 < a.groups; g0 += 4 * nt) {
      float pv[4];
      int pi[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int gi = min(g0 + u * nt, a.groups - 1);
        pv[u] = a.vals[row * a.groups + gi];
        pi[u] = a.idx[row * a.groups + gi];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (g0 + u * nt < a.groups) tia::amax_merge(v, i, pv[u], pi[u]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) tia::amax_merge(v, i, __shfl_xor(v, o, 64), __shfl_xor(i, o, 64));
    if (lane == 0) {
      sv[wave] = v;
      si[wave] = i;
    }
    __syncthreads();
    if (wave != 0) return;
    v = sv[0];
    i = si[0];
    for (int w = 1; w < nt / 64; ++w) tia::amax_merge(v, i, sv[w], si[w]);
    id = i;
  } else {
    if (wave != 0) return;
    id = a.next[row];
  }
  if (lane == 0) {
    a.next[row] = id;
    a.run[int64_t(pos) * a.b + row] = id;
    a.ids[row] = id;
    a.offsets[row] = pos + 1;
  }
  if (pos + 1 < a.positions) {
    const bool ok = id >= 0 && id < a.vocab;
    emb.finish(lane, true, ok ? id : 0, a.wte, a.x, a.norm, row, a.hidden, a.p32);
  }
}

__global__ void zero_f64_kernel(double* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0;
}

unsigned blocks_for(int64_t n, int per = 256) { return unsigned((n + per - 1) / per); }
using Clock = std::chrono::steady_clock;
double ms_since(Clock::time_point t0) {
  return std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
}

}  // namespace

struct ti_llm_model {
  struct Linear {
    const void* w = nullptr;
    const float* scales = nullptr;
    const uint16_t* bias = nullptr;
    int k = 0, n = 0;
    int64_t ldw = 0;
    const void* packed = nullptr;  // panel-packed int8 copy for the decode GEMV
    const void* f16p = nullptr;    // pre-dequantised fp16 copy for large prefill GEMMs
  };

  ti_llm_options opt{};
  hipStream_t stream = nullptr;
  bool poisoned = false;
  bool quantized = true;
  tia::art::Arch arch;
  int L = 0, NH = 0, H = 0, V = 0;
  std::vector<void*> allocations;
  void* pinned = nullptr;
  std::vector<Linear> c_attn, c_proj, c_fc, c_proj2;
  Linear head;
  const uint16_t *wte = nullptr, *wpe = nullptr, *lnf_g = nullptr, *lnf_b = nullptr;
  std::vector<const uint16_t*> ln1_g, ln1_b, ln2_g, ln2_b;
  uint16_t *x = nullptr, *norm = nullptr, *qkv = nullptr, *attn = nullptr, *mlp = nullptr, *last = nullptr;
  uint16_t *kc = nullptr, *vc = nullptr;
  float* logits = nullptr;
  int32_t *d_meta = nullptr, *d_ids = nullptr, *d_slots = nullptr, *d_qlens = nullptr, *d_offsets = nullptr,
          *d_row_start = nullptr;
  int32_t *d_next = nullptr, *d_score_tokens = nullptr;
  // Greedy partials of the wide head GEMV: [group][32] (value, column).
  static constexpr size_t kAmaxEntries = size_t(4096) * 32;
  float* d_amax_v = nullptr;
  int32_t* d_amax_i = nullptr;
  uint8_t* d_score_mask = nullptr;
  double *d_loss = nullptr, *d_loss_sum = nullptr;
  int32_t *h_meta = nullptr, *h_ids = nullptr, *h_slots = nullptr, *h_qlens = nullptr, *h_offsets = nullptr,
          *h_row_start = nullptr;
  int32_t* h_next = nullptr;
  size_t meta_ints = 0;
  tia::Scratch scratch;
  std::vector<int32_t> lengths;
  ti_llm_trace trace{};
  bool norm_p32 = false;  // the last layers() pass left x and norm P32-packed

  // Per-lane state of a decode step: the members above (stream, activations,
  // step metadata, head outputs, scratch) are the active lane's copy;
  // select_lane() swaps them.  Lane 0 also serves prefill, eager passes and
  // scoring, with buffers sized for max_batch x capacity rows; lane 1 only
  // decodes, with buffers for 32 rows.
  struct Lane {
    hipStream_t stream = nullptr;
    uint16_t *x = nullptr, *norm = nullptr, *qkv = nullptr, *attn = nullptr, *mlp = nullptr, *last = nullptr;
    float* logits = nullptr;
    int32_t *d_meta = nullptr, *d_next = nullptr;
    float* d_amax_v = nullptr;
    int32_t* d_amax_i = nullptr;
    int32_t *h_meta = nullptr, *h_next = nullptr;
    tia::Scratch scratch;
    bool norm_p32 = false;
    std::map<int, hipGraphExec_t> decode_graphs;
    // Greedy ids of a run of decode steps: device [position][rows] (the
    // position of the step's input token) and the pinned host copy.
    int32_t* d_run = nullptr;
    int32_t* h_run = nullptr;
  };
  Lane lanes[kLanes];
  int lane = 0;
  int lane_count = 1;
  void* pinned_lanes[kLanes] = {};
  void* pinned_runs[kLanes] = {};

  void save_lane() {
    Lane& l = lanes[lane];
    l.stream = stream;
    l.x = x; l.norm = norm; l.qkv = qkv; l.attn = attn; l.mlp = mlp; l.last = last;
    l.logits = logits;
    l.d_meta = d_meta; l.d_next = d_next;
    l.d_amax_v = d_amax_v; l.d_amax_i = d_amax_i;
    l.h_meta = h_meta; l.h_next = h_next;
    l.scratch = scratch;
    l.norm_p32 = norm_p32;
  }
  void select_lane(int i) {
    save_lane();
    lane = i;
    const Lane& l = lanes[i];
    stream = l.stream;
    x = l.x; norm = l.norm; qkv = l.qkv; attn = l.attn; mlp = l.mlp; last = l.last;
    logits = l.logits;
    d_meta = l.d_meta; d_next = l.d_next;
    d_amax_v = l.d_amax_v; d_amax_i = l.d_amax_i;
    h_meta = l.h_meta; h_next = l.h_next;
    scratch = l.scratch;
    norm_p32 = l.norm_p32;
    // The metadata layout ids[rows] | slots[B] | qlens[B] | offsets[B] |
    // row_start[B + 1] of each lane, B = max_batch.
    const size_t rows = i == 0 ? std::max<size_t>(size_t(opt.max_batch) * opt.capacity, 32) : 32;
    d_ids = d_meta;
    d_slots = d_ids + rows;
    d_qlens = d_slots + opt.max_batch;
    d_offsets = d_qlens + opt.max_batch;
    d_row_start = d_offsets + opt.max_batch;
    h_ids = h_meta;
    h_slots = h_ids + rows;
    h_qlens = h_slots + opt.max_batch;
    h_offsets = h_qlens + opt.max_batch;
    h_row_start = h_offsets + opt.max_batch;
  }

  template <class T>
  T* alloc(size_t count) {
    void* p = nullptr;
    ck(hipMalloc(&p, std::max<size_t>(count, 1) * sizeof(T)));
    allocations.push_back(p);
    return static_cast<T*>(p);
  }

  ~ti_llm_model() {
    int previous = -1;
    (void)hipGetDevice(&previous);
    (void)hipSetDevice(opt.device);
    if (stream) save_lane();
    for (Lane& l : lanes) {
      if (l.stream) (void)hipStreamSynchronize(l.stream);
      for (auto& g : l.decode_graphs) (void)hipGraphExecDestroy(g.second);
    }
    for (void* p : allocations) (void)hipFree(p);
    if (pinned) (void)hipHostFree(pinned);
    for (void* p : pinned_lanes)
      if (p) (void)hipHostFree(p);
    for (void* p : pinned_runs)
      if (p) (void)hipHostFree(p);
    for (Lane& l : lanes)
      if (l.stream) (void)hipStreamDestroy(l.stream);
    if (previous >= 0) (void)hipSetDevice(previous);
  }

  void check() const {
    if (poisoned) throw GpuError("model poisoned by an earlier execution failure; destroy and recreate it");
  }

  void init(const tia::art::Artifact& a) {
    arch = a.arch;
    L = arch.layers;
    NH = arch.heads;
    H = arch.hidden;
    V = arch.vocab;
    if (opt.capacity > arch.capacity) throw Invalid("capacity exceeds the model's position table");
    if (H > 2048) throw Invalid("hidden size above 2048 is not supported by the fused row kernels");
    quantized = a.precision == "int8";
    const std::string lin = quantized ? "int8" : "float16";
    std::set<std::string> used;
    uint8_t* base = alloc<uint8_t>(a.binary.size());
    ck(hipMemcpy(base, a.binary.data(), a.binary.size(), hipMemcpyHostToDevice));
    auto tensor = [&](const std::string& name, std::vector<int> shape, const std::string& dtype) {
      const auto& t = a.require(name, shape, dtype);
      used.insert(name);
      return static_cast<const void*>(base + t.offset);
    };
    auto half = [&](const std::string& name, std::vector<int> shape) {
      return static_cast<const uint16_t*>(tensor(name, shape, "float16"));
    };
    wte = half("transformer.wte.weight", {V, H});
    wpe = half("transformer.wpe.weight", {arch.capacity, H});
    lnf_g = half("transformer.ln_f.weight", {H});
    lnf_b = half("transformer.ln_f.bias", {H});
    auto linear = [&](const std::string& p, int k, int n) {
      Linear l;
      l.k = k;
      l.n = n;
      l.ldw = n;
      l.w = tensor(p + ".weight", {k, n}, lin);
      l.bias = half(p + ".bias", {n});
      if (quantized) l.scales = static_cast<const float*>(tensor(p + ".weight.scales", {n}, "float32"));
      return l;
    };
    for (int l = 0; l < L; ++l) {
      const std::string p = "transformer.h." + std::to_string(l) + ".";
      ln1_g.push_back(half(p + "ln_1.weight", {H}));
      ln1_b.push_back(half(p + "ln_1.bias", {H}));
      ln2_g.push_back(half(p + "ln_2.weight", {H}));
      ln2_b.push_back(half(p + "ln_2.bias", {H}));
      c_attn.push_back(linear(p + "attn.c_attn", H, 3 * H));
      c_proj.push_back(linear(p + "attn.c_proj", H, H));
      c_fc.push_back(linear(p + "mlp.c_fc", H, 4 * H));
      c_proj2.push_back(linear(p + "mlp.c_proj", 4 * H, H));
    }
    // The tied head [H, V] gets a 64-column-aligned row pitch so every row is
    // dword aligned for the vectorized weight loads.
    {
      const size_t width = quantized ? 1 : 2;
      const void* src = tensor("lm_head.weight", {H, V}, lin);
      (void)src;
      const auto& t = a.require("lm_head.weight", {H, V}, lin);
      head.k = H;
      head.n = V;
      head.ldw = (int64_t(V) + 63) / 64 * 64;
      uint8_t* padded = alloc<uint8_t>(size_t(H) * size_t(head.ldw) * width);
      ck(hipMemset(padded, 0, size_t(H) * size_t(head.ldw) * width));
      ck(hipMemcpy2D(padded, size_t(head.ldw) * width, a.binary.data() + t.offset, size_t(V) * width,
                     size_t(V) * width, size_t(H), hipMemcpyHostToDevice));
      head.w = padded;
      if (quantized) head.scales = static_cast<const float*>(tensor("lm_head.weight.scales", {V}, "float32"));
    }
    if (used.size() != a.tensors.size()) throw Invalid("unexpected tensor(s) in artifact");
    // The LayerNorm parameters get 16-byte aligned copies (the GEMV prologue
    // reads them 8 halves at a time; artifact offsets need not be aligned).
    {
      const size_t n = size_t(4 * L + 2);
      uint16_t* ln = alloc<uint16_t>(n * size_t(H));
      size_t i = 0;
      auto place = [&](const uint16_t*& p) {
        ck(hipMemcpy(ln + i * H, p, size_t(H) * sizeof(uint16_t), hipMemcpyDeviceToDevice));
        p = ln + i++ * H;
      };
      place(lnf_g);
      place(lnf_b);
      for (int l = 0; l < L; ++l) {
        place(ln1_g[l]);
        place(ln1_b[l]);
        place(ln2_g[l]);
        place(ln2_b[l]);
      }
    }
    // Decode GEMVs read every int8 linear (and the head) from a panel-packed copy
    // (one contiguous KiB per wave load, already in MFMA B-operand order); the
    // row-major copy stays for the prefill GEMM.
    if (quantized && H % 64 == 0) {
      auto pack = [&](Linear& w) {
        void* out = alloc<uint8_t>(tia::packed_w8_bytes(w.k, w.n));
        ck(tia::pack_w8(static_cast<const int8_t*>(w.w), w.ldw, w.k, w.n, out, stream));
        w.packed = out;
      };
      // Prefills of 2048 rows and more read a pre-dequantised fp16 copy where
      // its GEMM beats the int8 panels (2 bytes per weight; the decode GEMVs
      // keep reading int8).
      const bool f16_copies = int64_t(opt.max_batch) * opt.capacity >= 2048;
      auto pack16 = [&](Linear& w) {
        if (!f16_copies) return;
        void* out = alloc<uint8_t>(tia::packed_w16_bytes(w.k, w.n));
        ck(tia::pack_w16(static_cast<const int8_t*>(w.w), w.ldw, w.scales, w.k, w.n, out, stream));
        w.f16p = out;
      };
      for (int l = 0; l < L; ++l) {
        for (Linear* w : {&c_attn[l], &c_proj[l], &c_fc[l], &c_proj2[l]}) {
          pack(*w);
          pack16(*w);
        }
      }
      pack(head);
    }

    // At least 32 rows: decode keeps activations P32 fragment-packed (32 x K).
    const size_t rows = std::max<size_t>(size_t(opt.max_batch) * opt.capacity, 32);
    x = alloc<uint16_t>(rows * H);
    norm = alloc<uint16_t>(rows * H);
    qkv = alloc<uint16_t>(rows * 3 * H);
    attn = alloc<uint16_t>(rows * H);
    mlp = alloc<uint16_t>(rows * 4 * H);
    last = alloc<uint16_t>(size_t(std::max(opt.max_batch, kScoreRows)) * H);
    const size_t cache = size_t(opt.cache_slots + 1) * L * NH * opt.capacity * kHeadDim;
    kc = alloc<uint16_t>(cache);
    vc = alloc<uint16_t>(cache);
    logits = alloc<float>(size_t(std::max(opt.max_batch, kScoreRows)) * size_t(head.ldw));
    // Step metadata: ids[rows] | slots[B] | qlens[B] | offsets[B] | row_start[B + 1],
    // mirrored in pinned host memory.
    meta_ints = rows + 4 * size_t(opt.max_batch) + 1;
    d_meta = alloc<int32_t>(meta_ints);
    d_ids = d_meta;
    d_slots = d_ids + rows;
    d_qlens = d_slots + opt.max_batch;
    d_offsets = d_qlens + opt.max_batch;
    d_row_start = d_offsets + opt.max_batch;
    d_next = alloc<int32_t>(opt.max_batch);
    d_amax_v = alloc<float>(kAmaxEntries);
    d_amax_i = alloc<int32_t>(kAmaxEntries);
    d_score_tokens = alloc<int32_t>(opt.capacity);
    d_score_mask = alloc<uint8_t>(opt.capacity);
    d_loss = alloc<double>(opt.capacity);
    d_loss_sum = alloc<double>(1);
    ck(hipHostMalloc(&pinned, (meta_ints + opt.max_batch) * sizeof(int32_t), hipHostMallocDefault));
    h_meta = static_cast<int32_t*>(pinned);
    h_ids = h_meta;
    h_slots = h_ids + rows;
    h_qlens = h_slots + opt.max_batch;
    h_offsets = h_qlens + opt.max_batch;
    h_row_start = h_offsets + opt.max_batch;
    h_next = h_meta + meta_ints;
    scratch.partials = alloc<float>(tia::kScratchPartialFloats);
    scratch.partial_floats = tia::kScratchPartialFloats;
    lengths.assign(opt.cache_slots + 1, 0);
    save_lane();
    // Lanes 1.. (decode runs of more than kLaneRows requests over the packed
    // INT8 weights): own stream, 32-row activations, metadata, head outputs
    // and scratch.
    size_t decode_weights = size_t(head.k) * size_t(head.n);
    for (const auto* ls : {&c_attn, &c_proj, &c_fc, &c_proj2})
      for (const Linear& w : *ls) decode_weights += size_t(w.k) * size_t(w.n);
    if (opt.max_batch > kLaneRows && quantized && head.packed && H % 64 == 0 && decode_weights <= kLaneWeightBytes)
      lane_count = std::min(kLanes, (opt.max_batch + kLaneRows - 1) / kLaneRows);
    for (int i = 1; i < lane_count; ++i) {
      Lane& l = lanes[i];
      ck(hipStreamCreateWithFlags(&l.stream, hipStreamNonBlocking));
      l.x = alloc<uint16_t>(32 * size_t(H));
      l.norm = alloc<uint16_t>(32 * size_t(H));
      l.qkv = alloc<uint16_t>(32 * 3 * size_t(H));
      l.attn = alloc<uint16_t>(32 * size_t(H));
      l.mlp = alloc<uint16_t>(32 * 4 * size_t(H));
      l.last = alloc<uint16_t>(32 * size_t(H));
      l.logits = alloc<float>(size_t(kLaneRows) * size_t(head.ldw));
      const size_t ints = 32 + 4 * size_t(opt.max_batch) + 1;
      l.d_meta = alloc<int32_t>(ints);
      l.d_next = alloc<int32_t>(opt.max_batch);
      l.d_amax_v = alloc<float>(kAmaxEntries);
      l.d_amax_i = alloc<int32_t>(kAmaxEntries);
      ck(hipHostMalloc(&pinned_lanes[i], (ints + opt.max_batch) * sizeof(int32_t), hipHostMallocDefault));
      l.h_meta = static_cast<int32_t*>(pinned_lanes[i]);
      l.h_next = l.h_meta + ints;
      l.scratch.partials = alloc<float>(tia::kScratchPartialFloats);
      l.scratch.partial_floats = tia::kScratchPartialFloats;
    }
    for (int i = 0; i < lane_count; ++i) {
      Lane& l = lanes[i];
      const size_t ids = size_t(opt.capacity) * size_t(i == 0 ? opt.max_batch : kLaneRows);
      l.d_run = alloc<int32_t>(ids);
      ck(hipHostMalloc(&pinned_runs[i], ids * sizeof(int32_t), hipHostMallocDefault));
      l.h_run = static_cast<int32_t*>(pinned_runs[i]);
    }
    ck(hipStreamSynchronize(stream));
  }

  // ---------------------------------------------------------------- launch helpers
  void gemm(const uint16_t* a, int m, const Linear& w, tia::Epilogue epi, int* deferred = nullptr,
            const uint16_t* ln_g = nullptr, const uint16_t* ln_b = nullptr, bool a_p32 = false,
            int* amax_groups = nullptr, int defer_workgroups = 192) {
    tia::GemmArgs g;
    g.a = a;
    g.lda = w.k;
    g.w = w.w;
    g.w_int8 = quantized;
    g.scales = w.scales;
    g.m = m;
    g.n = w.n;
    g.k = w.k;
    g.ldw = w.ldw;
    g.w_packed = w.packed;
    g.w_f16p = w.f16p;
    g.a_p32 = a_p32;
    if (amax_groups) {
      g.amax_v = d_amax_v;
      g.amax_i = d_amax_i;
      g.amax_capacity = kAmaxEntries;
      g.amax_groups = amax_groups;
    }
    g.ln_gamma = ln_g;
    g.ln_beta = ln_b;
    g.ln_eps = 1e-5f;
    g.epi = epi;
    g.canonical = prefill_pass;
    g.decode_batches = !prefill_pass;
    g.weights_shared = !prefill_pass && lane_count > 1;  // two lanes stream the same records
    g.defer_workgroups = defer_workgroups;
    ck(tia::gemm(g, &scratch, stream, deferred));
  }

  // Set for the GEMMs of a prefill pass (several tokens per request) and the head
  // over its last rows: their rows are then summed in one order whatever the
  // batch (tia::GemmArgs::canonical), so a prompt decodes the same alone or
  // beside others, as the reference runtime does (the epoll server batches
  // prompts as they arrive).  Decode GEMVs of 1..16 rows are batch-invariant by
  // construction: one kernel and one K split per shape for every M up to 16
  // (tia::GemmArgs::decode_batches).
  bool prefill_pass = false;
  // Rows of the next pass when its requests' tokens are compact (request b at
  // rows row_start[b] .. row_start[b] + qlens[b] - 1 of x, norm, qkv, attn,
  // mlp; d_row_start uploaded), 0 when a pass is b x qlen rows.
  int compact_rows = 0;

  // x += a @ w + bias (fp16 rounding points of reference runtime.cu:149/153), then
  // norm = LayerNorm(x; g, beta).  Decode-sized GEMMs leave split-K partials that
  // one fused kernel reduces, adds and normalizes.  p32: a, x and norm are P32
  // fragment-packed (a decode pass); the split then aims at `workgroups`.
  void residual_ln(const uint16_t* a, int rows, const Linear& w, const uint16_t* g, const uint16_t* beta,
                   bool p32 = false, int workgroups = 192) {
    tia::Epilogue r;
    r.kind = tia::EPI_RESIDUAL;
    r.bias = w.bias;
    r.y = x;
    r.ldy = H;
    r.residual = x;
    r.ldr = H;
    // (A deferred launch runs no epilogue: x is written by the finisher, so the
    // epilogue keeps its row-major default.)
    int splits = 0;
    gemm(a, rows, w, r, &splits, nullptr, nullptr, p32, nullptr, workgroups);
    if (splits > 0)
      ck(tia::splitk_residual_layernorm(scratch.partials, splits, rows, H, w.bias, x, g, beta, norm, 1e-5f, stream,
                                        p32));
    else
      ck(p32 ? tia::layernorm_f16_p32(x, g, beta, norm, rows, H, 1e-5f, stream)
             : tia::layernorm_f16(x, g, beta, norm, rows, H, 1e-5f, stream));
  }

  // x += a @ w + bias in the GEMM's epilogue (no LayerNorm after it); a and x
  // P32 fragment-packed or row-major.
  void residual_add(const uint16_t* a, int rows, const Linear& w, bool p32) {
    tia::Epilogue r;
    r.kind = tia::EPI_RESIDUAL;
    r.bias = w.bias;
    r.y = x;
    r.ldy = H;
    r.residual = x;
    r.ldr = H;
    r.p32 = p32;
    gemm(a, rows, w, r, nullptr, nullptr, nullptr, p32);
  }

  // Decode of up to 32 requests over packed weights: each LayerNorm runs in the
  // prologue of the GEMV that consumes it (c_attn: ln_1, c_fc: ln_2, head: ln_f)
  // and each residual add in the epilogue of the GEMV that produces it.
  // (hidden <= 2048: one round of at most 8 waves x 4 chunks covers K.)
  bool ln_fused(int b, int qlen) const {
    return qlen == 1 && quantized && head.packed && c_attn[0].packed &&
           tia::gemm_ln_supported(b, H, H);
  }

  // One pass of the transformer over rows [b, qlen] whose metadata is already on
  // the device; leaves the residual stream in x and ln_f(x) of every row in norm
  // (both P32 fragment-packed after an ln_fused pass, row-major otherwise).
  // Fragment-packed activations from two rows up: a single row reads one
  // cache line per A fragment either way, and its row-major output writes are
  // contiguous.
  bool p32_pass(int b, int qlen) const { return ln_fused(b, qlen) && b * qlen > 1; }

  // Embedding rows and layer 0's ln_1 of a pass whose metadata is on the device.
  void embed(int b, int qlen) {
    const int rows = compact_rows ? compact_rows : b * qlen;
    embed_ln_kernel<<<blocks_for(rows, 4), 256, 0, stream>>>(d_ids, d_qlens, d_offsets,
                                                             compact_rows ? d_row_start : nullptr, b, wte, wpe,
                                                             ln1_g[0], ln1_b[0], x, norm, rows, qlen, H,
                                                             p32_pass(b, qlen));
    ck(hipGetLastError());
  }

  // `embedded`: x and norm already hold the embedding rows (the previous
  // decode step's greedy_feed_kernel, or embed()).
  void layers(int b, int qlen, bool embedded = false) {
    const int rows = compact_rows ? compact_rows : b * qlen;
    const int32_t* row_start = compact_rows ? d_row_start : nullptr;
    prefill_pass = qlen > 1;
    const bool fuse = ln_fused(b, qlen);
    const bool p32 = p32_pass(b, qlen);
    norm_p32 = p32;
    if (!embedded) embed(b, qlen);
    // The LayerNorm before c_attn / c_fc: in the GEMV's prologue up to hidden
    // 1024; above, every one of the GEMV's workgroups normalising all rows
    // costs more VALU time than a row kernel (measured at GPT-2 XL's 1600).
    // There the residual GEMVs (c_proj, mlp c_proj: N = hidden, too few column
    // blocks to fill the machine unsplit) split K and one finisher per row sums
    // the partials, adds bias and residual and writes the next LayerNorm into
    // norm (ln_2, the next layer's ln_1, or ln_f): the same launch count as
    // GEMV + LayerNorm row kernel.  Layer 0's ln_1 is already in norm
    // (embedding kernel).
    const bool ln_prologue = H <= 1024;
    const bool split_residual = fuse && !ln_prologue;
    auto ln_then_gemm = [&](const Linear& w, const tia::Epilogue& epi, int* defer, const uint16_t* g,
                            const uint16_t* beta, bool in_norm) {
      if (ln_prologue) return gemm(x, rows, w, epi, defer, g, beta, p32);
      if (!in_norm)
        ck(p32 ? tia::layernorm_f16_p32(x, g, beta, norm, rows, H, 1e-5f, stream)
               : tia::layernorm_f16(x, g, beta, norm, rows, H, 1e-5f, stream));
      gemm(norm, rows, w, epi, defer, nullptr, nullptr, p32);
    };
    for (int l = 0; l < L; ++l) {
      tia::Epilogue e;
      e.kind = tia::EPI_QKV;
      e.bias = c_attn[l].bias;
      e.y = qkv;
      e.ldy = 3 * H;
      e.kcache = kc;
      e.vcache = vc;
      e.slots = d_slots;
      e.offsets = d_offsets;
      e.qlens = d_qlens;
      e.qrows = qlen;
      e.row_start = row_start;
      e.batch = b;
      e.hidden = H;
      e.heads = NH;
      e.layer = l;
      e.layers = L;
      e.capacity = opt.capacity;
      // Decode: the skinny GEMM leaves split-K partials and the attention kernel
      // finishes q, k, v itself (one launch fewer per layer).
      int qkv_splits = 0;
      int* defer_qkv = qlen == 1 && c_attn[l].bias ? &qkv_splits : nullptr;
      if (fuse) ln_then_gemm(c_attn[l], e, defer_qkv, ln1_g[l], ln1_b[l], l == 0 || split_residual);
      else gemm(norm, rows, c_attn[l], e, defer_qkv);

      tia::AttnArgs at;
      if (qkv_splits > 0) {
        at.qkv_partials = scratch.partials;
        at.qkv_splits = qkv_splits;
        at.qkv_bias = c_attn[l].bias;
        at.hidden = H;
      }
      const int64_t head_stride = int64_t(opt.capacity) * kHeadDim;
      at.q = qkv;
      at.q_sb = int64_t(qlen) * 3 * H;
      at.q_sh = kHeadDim;
      at.q_sq = 3 * H;
      at.k = kc + int64_t(l) * NH * head_stride;
      at.v = vc + int64_t(l) * NH * head_stride;
      at.kv_sb = int64_t(L) * NH * head_stride;
      at.kv_sh = head_stride;
      at.kv_slot = d_slots;
      at.out = attn;
      at.q_row_start = row_start;
      at.o_sb = int64_t(qlen) * H;
      at.o_sh = kHeadDim;
      at.o_sq = H;
      at.q_lengths = d_qlens;
      at.kv_lengths = d_qlens;
      at.offsets = d_offsets;
      at.kv_from_offsets = true;
      at.batch = b;
      at.heads = NH;
      at.q_len = qlen;
      at.kv_len = opt.capacity;
      at.head_dim = kHeadDim;
      at.causal = true;
      at.out_p32 = p32;
      at.batch_invariant = true;
      ck(tia::attention(at, stream));

      tia::Epilogue gl;
      gl.kind = tia::EPI_GELU;
      gl.bias = c_fc[l].bias;
      gl.y = mlp;
      gl.ldy = 4 * H;
      const bool final_layer = l + 1 == L;
      if (split_residual) {
        gl.p32 = p32;
        residual_ln(attn, rows, c_proj[l], ln2_g[l], ln2_b[l], p32, kResidualSplitWorkgroups);
        gemm(norm, rows, c_fc[l], gl, nullptr, nullptr, nullptr, p32);
        residual_ln(mlp, rows, c_proj2[l], final_layer ? lnf_g : ln1_g[l + 1], final_layer ? lnf_b : ln1_b[l + 1],
                    p32, kResidualSplitWorkgroups);
        continue;
      }
      if (fuse) {
        gl.p32 = p32;
        residual_add(attn, rows, c_proj[l], p32);
        ln_then_gemm(c_fc[l], gl, nullptr, ln2_g[l], ln2_b[l], false);
      } else {
        residual_ln(attn, rows, c_proj[l], ln2_g[l], ln2_b[l]);
        gemm(norm, rows, c_fc[l], gl);
      }
      if (!fuse) {
        residual_ln(mlp, rows, c_proj2[l], final_layer ? lnf_g : ln1_g[l + 1], final_layer ? lnf_b : ln1_b[l + 1]);
        continue;
      }
      residual_add(mlp, rows, c_proj2[l], p32);
      // ln_f as its own row kernel: in the head GEMV's prologue every one of its
      // thousands of workgroups would normalize the same rows again.
      if (final_layer)
        ck(p32 ? tia::layernorm_f16_p32(x, lnf_g, lnf_b, norm, rows, H, 1e-5f, stream)
               : tia::layernorm_f16(x, lnf_g, lnf_b, norm, rows, H, 1e-5f, stream));
    }
  }

  // Logits of each request's last row (norm already holds ln_f), fp32 without
  // bias over the padded row pitch head.ldw, then the greedy argmax.
  // `feed` (a captured decode step): greedy_feed_kernel ends the step.
  void head_and_argmax(int b, int qlen, bool greedy, bool feed = false) {
    const uint16_t* rows_in = norm;
    if (qlen > 1) {
      gather_last_kernel<<<blocks_for(int64_t(b) * H / 8), 256, 0, stream>>>(
          norm, last, d_qlens, compact_rows ? d_row_start : nullptr, b, qlen, H);
      ck(hipGetLastError());
      rows_in = last;
    }
    tia::Epilogue e;
    e.kind = tia::EPI_F32;
    e.y = logits;
    e.ldy = head.ldw;
    // The wide head GEMV leaves per-workgroup argmax partials: then a small
    // finishing kernel replaces the pass over all logits.
    int groups = 0;
    gemm(rows_in, b, head, e, nullptr, nullptr, nullptr, norm_p32 && qlen == 1, greedy ? &groups : nullptr);
    if (greedy && groups == 0) {
      argmax_kernel<<<b, 1024, 0, stream>>>(logits, d_next, V, head.ldw);
      ck(hipGetLastError());
    }
    if (feed) {
      FeedArgs f;
      f.vals = d_amax_v;
      f.idx = d_amax_i;
      f.groups = groups;
      f.next = d_next;
      f.ids = d_ids;
      f.offsets = d_offsets;
      f.run = lanes[lane].d_run;
      f.b = b;
      f.vocab = V;
      f.positions = opt.capacity;
      f.hidden = H;
      f.wte = wte;
      f.wpe = wpe;
      f.g = ln1_g[0];
      f.bt = ln1_b[0];
      f.x = x;
      f.norm = norm;
      f.p32 = p32_pass(b, 1);
      greedy_feed_kernel<<<b, groups > 0 ? 1024 : 64, 0, stream>>>(f);
      ck(hipGetLastError());
    } else if (greedy && groups > 0) {
      ck(tia::argmax_partials(d_amax_v, d_amax_i, groups, b, d_next, stream));
    }
  }

  void count_forward(bool head_used, bool greedy) {
    ++trace.forward_calls;
    ++trace.embedding;
    for (int l = 0; l < L; ++l) {
      trace.layernorm += 2;
      if (quantized) trace.gemm_int8 += 4;
      else trace.gemm_fp16 += 4;
      ++trace.kv_scatter_gather;
      ++trace.attention;
      trace.residual += 2;
      ++trace.gelu;
    }
    ++trace.layernorm;  // ln_f
    if (head_used) {
      ++trace.lm_head;
      if (quantized) ++trace.gemm_int8;
      else ++trace.gemm_fp16;
    }
    if (greedy) ++trace.argmax;
  }

  // `ids`: the token rows of the pass (b x qlen padded, or the compact count).
  void upload_meta(size_t ids) {
    const size_t rows = size_t(opt.max_batch) * opt.capacity;
    ck(hipMemcpyAsync(d_ids, h_ids, ids * sizeof(int32_t), hipMemcpyHostToDevice, stream));
    ck(hipMemcpyAsync(d_slots, h_slots, (4 * size_t(opt.max_batch) + 1) * sizeof(int32_t), hipMemcpyHostToDevice,
                      stream));
    (void)rows;
  }

  // One greedy decode step of b rows as a graph launch: layers over the
  // embedding rows already in x / norm, head, greedy_feed_kernel.
  void decode_step_graph(int b) {
    auto& decode_graphs = lanes[lane].decode_graphs;
    auto it = decode_graphs.find(b);
    if (it == decode_graphs.end()) {
      hipGraph_t graph = nullptr;
      ck(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
      try {
        layers(b, 1, true);
        head_and_argmax(b, 1, true, true);
      } catch (...) {
        hipGraph_t dropped = nullptr;
        (void)hipStreamEndCapture(stream, &dropped);
        if (dropped) (void)hipGraphDestroy(dropped);
        throw;
      }
      ck(hipStreamEndCapture(stream, &graph));
      hipGraphExec_t exec = nullptr;
      const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
      (void)hipGraphDestroy(graph);
      ck(e);
      it = decode_graphs.emplace(b, exec).first;
    }
    ck(hipGraphLaunch(it->second, stream));
  }

  // reference runtime.cu:157-168
  void forward(const int32_t* s, const int32_t* tokens, const int32_t* lens, int b, int stride, float* out,
               int32_t* greedy, bool internal = false) {
    check();
    if (!s || !tokens || !lens || b < 1 || b > opt.max_batch || stride < 1 || stride > opt.capacity)
      throw Invalid("invalid batch/host pointers/stride");
    std::set<int32_t> unique;
    int qlen = 0;
    for (int i = 0; i < b; ++i) {
      if (s[i] < 0 || s[i] >= opt.cache_slots + (internal ? 1 : 0) || !unique.insert(s[i]).second || lens[i] < 1 ||
          lens[i] > stride || lengths[s[i]] + lens[i] > opt.capacity)
        throw Invalid("duplicate/invalid slot, length or capacity");
      qlen = std::max(qlen, lens[i]);
      for (int j = 0; j < lens[i]; ++j)
        if (tokens[int64_t(i) * stride + j] < 0 || tokens[int64_t(i) * stride + j] >= V)
          throw Invalid("token ID outside the model vocabulary");
    }
    // A ragged prefill runs over compact rows (request i's tokens at rows
    // row_start[i] ..), not padded to the longest prompt: the GEMMs, row
    // kernels and attention then do no work for padding.
    const bool compact = b > 1 && qlen > 1 && std::any_of(lens, lens + b, [&](int32_t n) { return n != qlen; });
    int rows = 0;
    for (int i = 0; i < b; ++i) {
      h_row_start[i] = rows;
      if (compact) {
        for (int j = 0; j < lens[i]; ++j) h_ids[rows + j] = tokens[int64_t(i) * stride + j];
        rows += lens[i];
      } else {
        for (int j = 0; j < qlen; ++j) h_ids[int64_t(i) * qlen + j] = j < lens[i] ? tokens[int64_t(i) * stride + j] : 0;
        rows += qlen;
      }
      h_slots[i] = s[i];
      h_qlens[i] = lens[i];
      h_offsets[i] = lengths[s[i]];
    }
    h_row_start[b] = rows;
    const bool need_head = out || greedy;
    upload_meta(size_t(rows));
    // Compact rows for this pass only, also when it throws (decode passes and
    // captured decode graphs must see b x 1 rows).
    struct CompactScope {
      int& rows;
      ~CompactScope() { rows = 0; }
    } compact_scope{compact_rows};
    compact_rows = compact ? rows : 0;
    if (qlen == 1 && greedy) {
      embed(b, 1);
      decode_step_graph(b);
    } else {
      layers(b, qlen);
      if (need_head) head_and_argmax(b, qlen, greedy != nullptr);
    }
    count_forward(need_head, greedy != nullptr);
    if (out)
      ck(hipMemcpy2DAsync(out, size_t(V) * sizeof(float), logits, size_t(head.ldw) * sizeof(float),
                          size_t(V) * sizeof(float), size_t(b), hipMemcpyDeviceToHost, stream));
    if (greedy) ck(hipMemcpyAsync(h_next, d_next, size_t(b) * sizeof(int32_t), hipMemcpyDeviceToHost, stream));
    ck(hipStreamSynchronize(stream));
    if (greedy) std::copy(h_next, h_next + b, greedy);
    for (int i = 0; i < b; ++i) lengths[s[i]] += lens[i];
  }

  // Greedy-decode `steps` tokens for each of b requests (slots s, last ids
  // `ids`) as one run: the steps are queued back to back (the captured step
  // feeds its own ids forward) and the host waits once, at the end.  More
  // than kLaneRows requests split evenly over ceil(b / kLaneRows) lanes,
  // queued side by side.  tokens[t * b + i] is request i's token after step t.
  // Returns the steps that count: `steps`, or, when some step t produced an
  // id outside the vocabulary (non-finite logits), t + 1 -- the reference's
  // greedy loop runs the forwards of steps 0..t and then rejects that id as
  // the next forward's input (reference runtime.cu:160, :197-199), so only
  // those steps advance the lengths and the caller reports it as invalid.
  int decode_run(const int32_t* s, const int32_t* ids, int b, int steps, int32_t* tokens) {
    check();
    if (b < 1 || b > opt.max_batch || steps < 1) throw Invalid("invalid decode run");
    for (int i = 0; i < b; ++i) {
      if (lengths[s[i]] + steps > opt.capacity) throw Invalid("decode run exceeds the cache capacity");
      if (ids[i] < 0 || ids[i] >= V) throw Invalid("token ID outside the model vocabulary");
    }
    const int parts = lane_count > 1 && b > kLaneRows && ln_fused(kLaneRows, 1) ? (b + kLaneRows - 1) / kLaneRows : 1;
    int first[kLanes] = {}, count[kLanes] = {};
    for (int l = 0; l < parts; ++l) {
      count[l] = b / parts + (l < b % parts ? 1 : 0);
      first[l] = l ? first[l - 1] + count[l - 1] : 0;
    }
    for (int l = 0; l < parts; ++l) {
      select_lane(l);
      for (int j = 0; j < count[l]; ++j) {
        const int i = first[l] + j;
        h_ids[j] = ids[i];
        h_slots[j] = s[i];
        h_qlens[j] = 1;
        h_offsets[j] = lengths[s[i]];
      }
      upload_meta(size_t(count[l]));
      embed(count[l], 1);
    }
    for (int t = 0; t < steps; ++t)
      for (int l = 0; l < parts; ++l) {
        select_lane(l);
        decode_step_graph(count[l]);
      }
    // Lane l's ids sit at run[position][row], positions lengths .. lengths +
    // steps - 1 of its requests.
    int lo[kLanes] = {}, hi[kLanes] = {};
    for (int l = 0; l < parts; ++l) {
      lo[l] = INT_MAX;
      for (int j = 0; j < count[l]; ++j) {
        lo[l] = std::min(lo[l], lengths[s[first[l] + j]]);
        hi[l] = std::max(hi[l], lengths[s[first[l] + j]] + steps);
      }
      select_lane(l);
      ck(hipMemcpyAsync(lanes[l].h_run, lanes[l].d_run + size_t(lo[l]) * count[l],
                        size_t(hi[l] - lo[l]) * count[l] * sizeof(int32_t), hipMemcpyDeviceToHost, stream));
    }
    select_lane(0);
    for (int l = 0; l < parts; ++l) ck(hipStreamSynchronize(lanes[l].stream));
    int valid = steps;
    for (int l = 0; l < parts; ++l)
      for (int j = 0; j < count[l]; ++j) {
        const int i = first[l] + j, base = lengths[s[i]] - lo[l];
        for (int t = 0; t < steps; ++t) {
          const int32_t id = lanes[l].h_run[size_t(base + t) * count[l] + j];
          tokens[size_t(t) * b + i] = id;
          if ((id < 0 || id >= V) && t + 1 < valid) valid = t + 1;
        }
      }
    for (int t = 0; t < valid; ++t) count_forward(true, true);
    for (int i = 0; i < b; ++i) lengths[s[i]] += valid;
    return valid;
  }

  // reference runtime.cu:204-211
  void score(const int32_t* tokens, const uint8_t* mask, int length, double* nll, uint64_t* count, double* positions) {
    check();
    if (!tokens || !mask || !nll || !count || length < 2 || length > opt.capacity || mask[0])
      throw Invalid("invalid score window");
    uint64_t targets = 0;
    for (int i = 0; i < length; ++i) {
      if (tokens[i] < 0 || tokens[i] >= V || mask[i] > 1) throw Invalid("invalid score token/mask");
      targets += mask[i];
    }
    if (!targets) throw Invalid("no shifted targets selected");
    const int slot = opt.cache_slots, q = length - 1;
    lengths[slot] = 0;
    std::copy(tokens, tokens + q, h_ids);
    h_slots[0] = slot;
    h_qlens[0] = q;
    h_offsets[0] = 0;
    upload_meta(size_t(q));
    layers(1, q);  // leaves ln_f of every row in norm
    ++trace.forward_calls;
    ++trace.embedding;
    trace.layernorm += 2 * L + 1;
    (quantized ? trace.gemm_int8 : trace.gemm_fp16) += 4 * L;
    trace.kv_scatter_gather += L;
    trace.attention += L;
    trace.residual += 2 * L;
    trace.gelu += L;
    ck(hipMemcpyAsync(d_score_tokens, tokens, size_t(length) * sizeof(int32_t), hipMemcpyHostToDevice, stream));
    ck(hipMemcpyAsync(d_score_mask, mask, size_t(length), hipMemcpyHostToDevice, stream));
    zero_f64_kernel<<<blocks_for(length), 256, 0, stream>>>(d_loss, length);
    ck(hipGetLastError());
    for (int row = 0; row < q; row += kScoreRows) {
      const int rows = std::min(kScoreRows, q - row);
      ++trace.lm_head;
      (quantized ? trace.gemm_int8 : trace.gemm_fp16) += 1;
      tia::Epilogue e;
      e.kind = tia::EPI_F32;
      e.y = logits;
      e.ldy = head.ldw;
      // (a one-token pass leaves norm P32-packed: then q == 1 and row == 0)
      gemm(norm_p32 ? norm : norm + int64_t(row) * H, rows, head, e, nullptr, nullptr, nullptr, norm_p32);
      ++trace.nll;
      nll_kernel<<<rows, 256, 0, stream>>>(logits, d_score_tokens, d_score_mask, d_loss, row + 1, V, head.ldw);
      ck(hipGetLastError());
    }
    sum_kernel<<<1, 256, 0, stream>>>(d_loss, d_loss_sum, length);
    ck(hipGetLastError());
    ck(hipMemcpyAsync(nll, d_loss_sum, sizeof(double), hipMemcpyDeviceToHost, stream));
    if (positions) ck(hipMemcpyAsync(positions, d_loss, size_t(length) * sizeof(double), hipMemcpyDeviceToHost, stream));
    ck(hipStreamSynchronize(stream));
    if (!std::isfinite(*nll) || *nll < 0) throw GpuError("non-finite or negative NLL");
    *count = targets;
  }
};

namespace {
template <class F>
int api(ti_llm_model* m, F&& fn) {
  error_text.clear();
  try {
    if (!m) throw Invalid("null model");
    DeviceScope scope(m->opt.device);
    m->check();
    fn();
    return TI_LLM_OK;
  } catch (const Invalid& e) {
    error_text = e.what();
    return TI_LLM_INVALID;
  } catch (const IOError& e) {
    error_text = e.what();
    return TI_LLM_IO;
  } catch (const GpuError& e) {
    if (m) m->poisoned = true;
    error_text = e.what();
    return TI_LLM_CUDA;
  } catch (const std::exception& e) {
    if (m) m->poisoned = true;
    error_text = e.what();
    return TI_LLM_INTERNAL;
  } catch (...) {
    if (m) m->poisoned = true;
    error_text = "unknown native failure";
    return TI_LLM_INTERNAL;
  }
}
}  // namespace

extern "C" int ti_llm_abi_version(void) { return 1; }
extern "C" const char* ti_llm_last_error(void) { return error_text.c_str(); }

extern "C" int ti_llm_create(const char* path, const ti_llm_options* o, ti_llm_model** out) {
  error_text.clear();
  if (out) *out = nullptr;
  try {
    if (!path || !o || !out || o->struct_size != sizeof(ti_llm_options) || o->device < 0 || o->max_batch < 1 ||
        o->max_batch > 32 || o->cache_slots < o->max_batch || o->cache_slots > 1024 || o->capacity < 2 ||
        o->capacity > 1024 || o->gemm_config < 0 || o->gemm_config > 11 || o->attention_config < 0 ||
        o->attention_config > 1)
      throw Invalid("invalid options/ABI size");
    if (ti_v2_abi_version() != 2) throw Invalid("v2 kernel ABI required");
    const tia::art::Artifact artifact = tia::art::load_artifact(path);
    DeviceScope scope(o->device);
    auto model = std::make_unique<ti_llm_model>();
    model->opt = *o;
    ck(hipStreamCreateWithFlags(&model->stream, hipStreamNonBlocking));
    model->init(artifact);
    *out = model.release();
    return TI_LLM_OK;
  } catch (const Invalid& e) {
    error_text = e.what();
    return TI_LLM_INVALID;
  } catch (const IOError& e) {
    error_text = e.what();
    return TI_LLM_IO;
  } catch (const GpuError& e) {
    error_text = e.what();
    return TI_LLM_CUDA;
  } catch (const std::exception& e) {
    error_text = e.what();
    return TI_LLM_INTERNAL;
  } catch (...) {
    error_text = "unknown create failure";
    return TI_LLM_INTERNAL;
  }
}

extern "C" int ti_llm_destroy(ti_llm_model* m) {
  error_text.clear();
  if (!m) {
    error_text = "null model";
    return TI_LLM_INVALID;
  }
  delete m;
  return TI_LLM_OK;
}

extern "C" int ti_llm_reset(ti_llm_model* m, int32_t slot) {
  return api(m, [&] {
    if (slot < 0 || slot >= m->opt.cache_slots) throw Invalid("invalid public slot");
    m->lengths[slot] = 0;
  });
}

extern "C" int ti_llm_lengths(ti_llm_model* m, int32_t* out, int32_t count) {
  return api(m, [&] {
    if (!out || count != m->opt.cache_slots) throw Invalid("wrong lengths output extent");
    std::copy(m->lengths.begin(), m->lengths.begin() + count, out);
  });
}

extern "C" int ti_llm_get_trace(ti_llm_model* m, ti_llm_trace* out) {
  return api(m, [&] {
    if (!out) throw Invalid("null trace output");
    *out = m->trace;
  });
}

extern "C" int ti_llm_forward_batch(ti_llm_model* m, const int32_t* slots, const int32_t* tokens,
                                    const int32_t* lengths, int32_t batch, int32_t stride, float* out,
                                    int32_t* next) {
  return api(m, [&] { m->forward(slots, tokens, lengths, batch, stride, out, next); });
}

// reference runtime.cu:190-203
extern "C" int ti_llm_greedy_batch(ti_llm_model* m, const int32_t* slots, const int32_t* prompts,
                                   const int32_t* prompt_lengths, const int32_t* requested, int32_t batch,
                                   int32_t stride, int32_t* output, int32_t out_stride, int32_t* output_lengths,
                                   double* ttft, double* total) {
  return api(m, [&] {
    if (!slots || !prompts || !prompt_lengths || !requested || !output || batch < 1 || batch > m->opt.max_batch ||
        stride < 1 || stride > m->opt.capacity || out_stride < 1 || out_stride > m->opt.capacity)
      throw Invalid("invalid greedy arguments");
    std::set<int> seen;
    for (int i = 0; i < batch; ++i) {
      if (slots[i] < 0 || slots[i] >= m->opt.cache_slots || !seen.insert(slots[i]).second || m->lengths[slots[i]] ||
          prompt_lengths[i] < 1 || prompt_lengths[i] > stride || requested[i] < 1 || requested[i] > out_stride ||
          requested[i] + prompt_lengths[i] > m->opt.capacity)
        throw Invalid("greedy needs empty distinct slots and bounded positive lengths");
      for (int j = 0; j < prompt_lengths[i]; ++j)
        if (prompts[int64_t(i) * stride + j] < 0 || prompts[int64_t(i) * stride + j] >= m->V)
          throw Invalid("invalid prompt token");
    }
    std::fill(output, output + int64_t(batch) * out_stride, -1);
    if (output_lengths) std::fill(output_lengths, output_lengths + batch, 0);
    const auto start = Clock::now();
    std::vector<int32_t> next(batch);
    m->forward(slots, prompts, prompt_lengths, batch, stride, nullptr, next.data());
    const double first = ms_since(start);
    std::vector<int> done(batch, 1);
    for (int i = 0; i < batch; ++i) {
      output[int64_t(i) * out_stride] = next[i];
      if (ttft) ttft[i] = first;
      if (total && requested[i] == 1) total[i] = first;
    }
    // Decode in runs: each run advances every unfinished request by the
    // fewest tokens any of them still needs, so the active set is fixed
    // within a run and at least one request finishes at its end.
    for (;;) {
      std::vector<int32_t> active, ids;
      std::vector<int> owner;
      int steps = 0;
      for (int i = 0; i < batch; ++i)
        if (done[i] < requested[i]) {
          active.push_back(slots[i]);
          ids.push_back(next[i]);
          owner.push_back(i);
          steps = steps ? std::min(steps, requested[i] - done[i]) : requested[i] - done[i];
        }
      if (active.empty()) break;
      const int n = int(active.size());
      std::vector<int32_t> generated(size_t(steps) * n);
      const int valid = m->decode_run(active.data(), ids.data(), n, steps, generated.data());
      const double elapsed = ms_since(start);
      for (int j = 0; j < n; ++j) {
        const int i = owner[j];
        for (int t = 0; t < valid; ++t) output[int64_t(i) * out_stride + done[i] + t] = generated[size_t(t) * n + j];
        done[i] += valid;
        next[i] = generated[size_t(valid - 1) * n + j];
        if (total && done[i] == requested[i]) total[i] = elapsed;
      }
      // An id outside the vocabulary ends the call as the reference's next
      // forward would: invalid, output so far kept, the model still usable.
      if (valid < steps) throw Invalid("token ID outside the model vocabulary");
    }
    if (output_lengths)
      for (int i = 0; i < batch; ++i) output_lengths[i] = done[i];
  });
}

extern "C" int ti_llm_score_window(ti_llm_model* m, const int32_t* tokens, const uint8_t* mask, int32_t length,
                                   double* nll, uint64_t* count, double* positions) {
  return api(m, [&] { m->score(tokens, mask, length, nll, count, positions); });
}

// Host-only self-test hooks for the artifact reader (no GPU needed): the
// reference checks these with llm/tests/test_artifact.cpp:7-15.
extern "C" int tia_llm_sha256_hex(const void* data, size_t n, char* out65) {
  const std::string h = tia::art::Sha256::of(data, n);
  std::memcpy(out65, h.c_str(), 65);
  return 0;
}
extern "C" int tia_llm_json_accepts(const char* text) {
  try {
    (void)tia::art::JsonReader(std::string(text)).parse();
    return 1;
  } catch (const Invalid&) {
    return 0;
  }
}
