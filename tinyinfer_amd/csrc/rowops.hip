// Row-wise LayerNorm and last-axis Softmax (fp16 and fp32) and elementwise
// tanh-GELU for gfx950.
//
// Rows up to 4096 columns take one wave per row: the row is read once into
// registers with 16-byte loads, reduced with wave64 butterflies (no LDS, no
// barriers), and written once — the HBM-minimal 2 x rows x cols x bytes.  Longer
// or unaligned rows fall back to a 256-thread block per row that re-reads the
// row from cache.  Semantics: LayerNorm y = (x - mean) * rsqrt(var + eps) * g + b
// with two-pass mean/variance in fp32 (reference
// kernels/src/cuda/tc/elementwise.cu:15-27, kernels/src/cuda/layernorm.cu:7-36);
// softmax y = exp(x - max) / sum with -inf entries exactly 0 (reference
// elementwise.cu:34-46, kernels/src/cuda/softmax.cu:19-53); fp16 storage rounds
// to nearest-even.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace tia {
namespace {

template <typename T>
struct Elem;
template <>
struct Elem<float> {
  static __device__ __forceinline__ float load(const float* p) { return *p; }
  static __device__ __forceinline__ void store(float* p, float v) { *p = v; }
};
template <>
struct Elem<uint16_t> {
  static __device__ __forceinline__ float load(const uint16_t* p) { return h2f(*p); }
  static __device__ __forceinline__ void store(uint16_t* p, float v) { *p = f2h(v); }
};

// VPL consecutive elements per lane per vector (16 bytes when VPL * sizeof(T) == 16).
// NT: a nontemporal (streaming) access, for row data touched once; the FP32
// row kernels stream x in and y out that way (measured at configs[2]: 12-24 %
// less time), while gamma and beta, read by every row, stay cached.
template <typename T, int VPL, bool NT = false>
__device__ __forceinline__ void load_vec(const T* p, float* out) {
  if constexpr (VPL * sizeof(T) == 16) {
    u32x4_t u;
    if constexpr (NT) u = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    else u = *reinterpret_cast<const u32x4_t*>(p);
    const uint32_t w[4] = {u[0], u[1], u[2], u[3]};
    if constexpr (sizeof(T) == 4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) out[i] = __builtin_bit_cast(float, w[i]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) out[i] = h2f(uint16_t(w[i >> 1] >> (16 * (i & 1))));
    }
  } else {
#pragma unroll
    for (int i = 0; i < VPL; ++i) out[i] = Elem<T>::load(p + i);
  }
}
template <typename T, int VPL, bool NT = false>
__device__ __forceinline__ void store_vec(T* p, const float* v) {
  if constexpr (VPL * sizeof(T) == 16) {
    uint32_t w[4];
    if constexpr (sizeof(T) == 4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = __builtin_bit_cast(uint32_t, v[i]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = uint32_t(f2h(v[2 * i])) | (uint32_t(f2h(v[2 * i + 1])) << 16);
    }
    if constexpr (NT) __builtin_nontemporal_store(u32x4_t{w[0], w[1], w[2], w[3]}, reinterpret_cast<u32x4_t*>(p));
    else *reinterpret_cast<u32x4_t*>(p) = u32x4_t{w[0], w[1], w[2], w[3]};
  } else {
#pragma unroll
    for (int i = 0; i < VPL; ++i) Elem<T>::store(p + i, v[i]);
  }
}

// One wave per row; lane l owns elements [VPL*l + 64*VPL*i, +VPL) for i < NV.
// gamma and beta are requested with the row (they do not depend on it), so the
// output pass needs no further round trip.
// P32: x and y are fragment-packed decode matrices (common.hpp p32_off; VPL 8).
template <typename T, int VPL, int NV, bool P32 = false, bool NT = false>
__device__ __forceinline__ void layernorm_row(const T* x, const T* g, const T* b, int row, int cols, float eps,
                                              float (&v)[NV][VPL]) {
  const int lane = threadIdx.x & 63;
  auto at = [&](int c) { return P32 ? p32_off(row, c) : int64_t(row) * cols + c; };
  float gv[NV][VPL], bv[NV][VPL];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = VPL * lane + 64 * VPL * i;
    if (c < cols) {
      load_vec<T, VPL, NT>(x + at(c), v[i]);
      load_vec<T, VPL>(g + c, gv[i]);
      load_vec<T, VPL>(b + c, bv[i]);
    } else {
#pragma unroll
      for (int e = 0; e < VPL; ++e) v[i][e] = gv[i][e] = bv[i][e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < VPL; ++e) s += v[i][e];
  }
  const float mean = wave_sum(s) / float(cols);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = VPL * lane + 64 * VPL * i;
    if (c < cols) {
#pragma unroll
      for (int e = 0; e < VPL; ++e) {
        const float d = v[i][e] - mean;
        ss += d * d;
      }
    }
  }
  const float inv = rsqrtf(wave_sum(ss) / float(cols) + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < VPL; ++e) v[i][e] = (v[i][e] - mean) * inv * gv[i][e] + bv[i][e];
}

template <typename T, int VPL, int NV, bool P32 = false, bool NT = false>
__global__ __launch_bounds__(256) void layernorm_wave(const T* x, const T* g, const T* b, T* y,
                                                      int rows, int cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  float v[NV][VPL];
  layernorm_row<T, VPL, NV, P32, NT>(x, g, b, row, cols, eps, v);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = VPL * lane + 64 * VPL * i;
    if (c < cols) store_vec<T, VPL, NT>(y + (P32 ? p32_off(row, c) : int64_t(row) * cols + c), v[i]);
  }
}

// Softmax of a row held as v (entries past cols are -inf): max, exp, sum, scale
// in place, in the order softmax_wave uses.
template <int VPL, int NV>
__device__ __forceinline__ void softmax_row(float (&v)[NV][VPL]) {
  float mx = -__builtin_huge_valf();
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < VPL; ++e) mx = fmaxf(mx, v[i][e]);
  mx = wave_max(mx);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < VPL; ++e) {
      v[i][e] = __expf(v[i][e] - mx);
      s += v[i][e];
    }
  const float inv = 1.f / wave_sum(s);
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < VPL; ++e) v[i][e] *= inv;
}

template <typename T, int VPL, int NV, bool NT = false>
__global__ __launch_bounds__(256) void softmax_wave(const T* x, T* y, int rows, int cols) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + int64_t(row) * cols;
  T* yr = y + int64_t(row) * cols;
  float v[NV][VPL];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = VPL * lane + 64 * VPL * i;
    if (c < cols) load_vec<T, VPL, NT>(xr + c, v[i]);
    else {
#pragma unroll
      for (int e = 0; e < VPL; ++e) v[i][e] = -__builtin_huge_valf();
    }
  }
  softmax_row<VPL, NV>(v);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = VPL * lane + 64 * VPL * i;
    if (c < cols) store_vec<T, VPL, NT>(yr + c, v[i]);
  }
}

// LayerNorm then last-axis softmax of each row in one pass: the graph that
// tinyc's norm_softmax issues as two calls, ti_*_layernorm then ti_*_softmax
// (reference bench/integrated.py:87-92).  The LayerNorm output stays in
// registers in the lane layout softmax_wave reads it with, so the values,
// maximum and sum are those of the two kernels through memory, for half the
// HBM traffic (x read once, y written once).
template <int VPL, int NV>
__global__ __launch_bounds__(256) void layernorm_softmax_wave(const float* x, const float* g, const float* b,
                                                              float* y, int rows, int cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  float v[NV][VPL];
  layernorm_row<float, VPL, NV, false, true>(x, g, b, row, cols, eps, v);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (VPL * lane + 64 * VPL * i >= cols) {
#pragma unroll
      for (int e = 0; e < VPL; ++e) v[i][e] = -__builtin_huge_valf();
    }
  }
  softmax_row<VPL, NV>(v);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = VPL * lane + 64 * VPL * i;
    if (c < cols) store_vec<float, VPL, true>(y + int64_t(row) * cols + c, v[i]);
  }
}

// Fallback: one 256-thread block per row, any width or alignment.
template <typename T>
__global__ __launch_bounds__(256) void layernorm_block(const T* x, const T* g, const T* b, T* y,
                                                       int cols, float eps) {
  __shared__ float lds[4];
  const T* xr = x + int64_t(blockIdx.x) * cols;
  T* yr = y + int64_t(blockIdx.x) * cols;
  float s = 0.f;
  for (int c = threadIdx.x; c < cols; c += 256) s += Elem<T>::load(xr + c);
  const float mean = block_sum<4>(s, lds) / float(cols);
  float ss = 0.f;
  for (int c = threadIdx.x; c < cols; c += 256) {
    const float d = Elem<T>::load(xr + c) - mean;
    ss += d * d;
  }
  const float inv = rsqrtf(block_sum<4>(ss, lds) / float(cols) + eps);
  for (int c = threadIdx.x; c < cols; c += 256)
    Elem<T>::store(yr + c, (Elem<T>::load(xr + c) - mean) * inv * Elem<T>::load(g + c) + Elem<T>::load(b + c));
}

template <typename T>
__global__ __launch_bounds__(256) void softmax_block(const T* x, T* y, int cols) {
  __shared__ float lds[4];
  const T* xr = x + int64_t(blockIdx.x) * cols;
  T* yr = y + int64_t(blockIdx.x) * cols;
  float mx = -__builtin_huge_valf();
  for (int c = threadIdx.x; c < cols; c += 256) mx = fmaxf(mx, Elem<T>::load(xr + c));
  mx = block_max<4>(mx, lds);
  float s = 0.f;
  for (int c = threadIdx.x; c < cols; c += 256) s += __expf(Elem<T>::load(xr + c) - mx);
  const float inv = 1.f / block_sum<4>(s, lds);
  for (int c = threadIdx.x; c < cols; c += 256) Elem<T>::store(yr + c, __expf(Elem<T>::load(xr + c) - mx) * inv);
}

__global__ void gelu_kernel(const uint16_t* x, uint16_t* y, int64_t count, bool vec) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (vec) {
    const int64_t nv = count / 8;
    for (int64_t i = t; i < nv; i += stride) {
      float v[8];
      load_vec<uint16_t, 8>(x + 8 * i, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = gelu_tanh(v[e]);
      store_vec<uint16_t, 8>(y + 8 * i, v);
    }
    for (int64_t i = nv * 8 + t; i < count; i += stride) y[i] = f2h(gelu_tanh(h2f(x[i])));
  } else {
    for (int64_t i = t; i < count; i += stride) y[i] = f2h(gelu_tanh(h2f(x[i])));
  }
}

// Deferred-GEMM finisher: split-K sum + bias + residual, then LayerNorm of the
// new row.  One workgroup of G waves per row: wave w sums splits w, w + G, ...
// for every column, the G partial rows meet in LDS and wave 0 adds them in
// group order, then does the residual and the LayerNorm with lane owning
// columns lane + 64 i.  NPL > 0 fixes cols = 64 * NPL so no load carries a
// bounds predicate (predicated loads are issued one round trip at a time);
// NPL = 0 is the predicated fallback for any cols <= 2048.  P32: x and norm are
// fragment-packed decode matrices (common.hpp p32_off), the partials row-major.
constexpr int kResLnMaxPerLane = 32;  // cols <= 2048
template <int G, int NPL, bool P32 = false>
__global__ __launch_bounds__(64 * G) void splitk_residual_ln_kernel(const float* partials, int splits, int rows,
                                                                    int cols, const uint16_t* bias, uint16_t* x,
                                                                    const uint16_t* g, const uint16_t* b,
                                                                    uint16_t* norm, float eps) {
  constexpr int N = NPL > 0 ? NPL : kResLnMaxPerLane;
  extern __shared__ float red[];  // [G][cols]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = blockIdx.x;
  const int64_t plane = int64_t(rows) * cols, base = int64_t(row) * cols;
  auto on = [&](int i) { return NPL > 0 || lane + 64 * i < cols; };
  auto xat = [&](int c) { return P32 ? p32_off(row, c) : base + c; };
  // Operands that do not depend on the partials are requested first, in one batch.
  // (A null bias reads gamma instead and is scaled to zero, so no load sits
  // behind a per-element branch.)
  float xv[N], bv[N], gv[N], btv[N];
  if (wave == 0) {
    const uint16_t* bp = bias ? bias : g;
    const float bscale = bias ? 1.f : 0.f;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int c = on(i) ? lane + 64 * i : 0;
      xv[i] = h2f(x[xat(c)]);
      gv[i] = h2f(g[c]);
      btv[i] = h2f(b[c]);
      bv[i] = h2f(bp[c]) * bscale;
    }
  }
  float v[N];
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = 0.f;
  for (int sp = wave; sp < splits; sp += G) {
    const float* p = partials + sp * plane + base + lane;
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (on(i)) v[i] += p[64 * i];
  }
#pragma unroll
  for (int i = 0; i < N; ++i)
    if (on(i)) red[wave * cols + lane + 64 * i] = v[i];
  __syncthreads();
  if (wave != 0) return;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int c = lane + 64 * i;
    if (on(i)) {
      float t = red[c];
#pragma unroll
      for (int w = 1; w < G; ++w) t += red[w * cols + c];
      const float h = rt16(t + bv[i]);
      v[i] = rt16(xv[i] + h);
      x[xat(c)] = f2h(v[i]);
      s += v[i];
    }
  }
  const float mean = wave_sum(s) / float(cols);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < N; ++i)
    if (on(i)) ss += (v[i] - mean) * (v[i] - mean);
  const float inv = rsqrtf(wave_sum(ss) / float(cols) + eps);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int c = lane + 64 * i;
    if (on(i)) norm[xat(c)] = f2h((v[i] - mean) * inv * gv[i] + btv[i]);
  }
}

// The same finisher with one wave per row and every load of the row in one
// round (no LDS, no barrier): lane l owns columns 8 l + 512 i (i < NV, cols % 8
// == 0); the S split partials are summed in split order, as the kernel above
// sums them for S <= G, then bias, residual and LayerNorm as there.  Columns
// past cols re-read the row's last 8 (clamped address) and are neither counted
// nor stored.  P32: x and norm are fragment-packed, the partials row-major.
template <int S, int NV, bool P32>
__global__ __launch_bounds__(256) void residual_ln_wave(const float* partials, int rows, int cols,
                                                        const uint16_t* bias, uint16_t* x, const uint16_t* g,
                                                        const uint16_t* b, uint16_t* norm, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t plane = int64_t(rows) * cols, base = int64_t(row) * cols;
  auto at = [&](int c) { return P32 ? p32_off(row, c) : base + c; };
  const uint16_t* bp = bias ? bias : g;  // a null bias reads gamma, scaled to zero
  const float bscale = bias ? 1.f : 0.f;
  u32x4_t xr[NV], gr[NV], br[NV], hr[NV];
  float4_t pr[S][NV][2];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = min(8 * lane + 512 * i, cols - 8);
    xr[i] = *reinterpret_cast<const u32x4_t*>(x + at(c));
    gr[i] = *reinterpret_cast<const u32x4_t*>(g + c);
    br[i] = *reinterpret_cast<const u32x4_t*>(b + c);
    hr[i] = *reinterpret_cast<const u32x4_t*>(bp + c);
#pragma unroll
    for (int sp = 0; sp < S; ++sp) {
      const float4_t* pp = reinterpret_cast<const float4_t*>(partials + sp * plane + base + c);
      pr[sp][i][0] = pp[0];
      pr[sp][i][1] = pp[1];
    }
  }
  auto half_at = [](const u32x4_t& u, int e) { return h2f(uint16_t(u[e >> 1] >> (16 * (e & 1)))); };
  float v[NV][8];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const bool on = 8 * lane + 512 * i < cols;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float t = pr[0][i][e >> 2][e & 3];
#pragma unroll
      for (int sp = 1; sp < S; ++sp) t += pr[sp][i][e >> 2][e & 3];
      const float h = rt16(t + half_at(hr[i], e) * bscale);
      v[i][e] = rt16(half_at(xr[i], e) + h);
      s += on ? v[i][e] : 0.f;
    }
  }
  const float mean = wave_sum(s) / float(cols);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const bool on = 8 * lane + 512 * i < cols;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += on ? (v[i][e] - mean) * (v[i][e] - mean) : 0.f;
  }
  const float inv = rsqrtf(wave_sum(ss) / float(cols) + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = 8 * lane + 512 * i;
    if (c >= cols) continue;
    uint32_t xo[4], no[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const float n0 = (v[i][e] - mean) * inv * half_at(gr[i], e) + half_at(br[i], e);
      const float n1 = (v[i][e + 1] - mean) * inv * half_at(gr[i], e + 1) + half_at(br[i], e + 1);
      xo[e >> 1] = uint32_t(f2h(v[i][e])) | (uint32_t(f2h(v[i][e + 1])) << 16);
      no[e >> 1] = uint32_t(f2h(n0)) | (uint32_t(f2h(n1)) << 16);
    }
    *reinterpret_cast<u32x4_t*>(x + at(c)) = u32x4_t{xo[0], xo[1], xo[2], xo[3]};
    *reinterpret_cast<u32x4_t*>(norm + at(c)) = u32x4_t{no[0], no[1], no[2], no[3]};
  }
}

bool al16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

template <typename T>
hipError_t layernorm_dispatch(const T* x, const T* g, const T* b, T* y, int rows, int cols,
                              float eps, hipStream_t st) {
  constexpr int VPL = 16 / sizeof(T);
  const bool vec = cols % VPL == 0 && al16(x) && al16(g) && al16(b) && al16(y);
  const dim3 grid(unsigned((rows + 3) / 4)), block(256);
  const int per = 64 * VPL;
  constexpr bool NT = sizeof(T) == 4;  // FP32 rows stream; fp16 outputs feed the next decode kernel
#define TIA_LN(V, NV) \
  hipLaunchKernelGGL((layernorm_wave<T, V, NV, false, NT>), grid, block, 0, st, x, g, b, y, rows, cols, eps)
  if (vec && cols <= per) TIA_LN(VPL, 1);
  else if (vec && cols <= 2 * per) TIA_LN(VPL, 2);
  else if (vec && cols <= 4 * per) TIA_LN(VPL, 4);
  else if (vec && cols <= 8 * per) TIA_LN(VPL, 8);
  else if (vec && VPL == 4 && cols <= 16 * per) TIA_LN(VPL, 16);
  else if (!vec && cols <= 64 * 16) TIA_LN(1, 16);
  else hipLaunchKernelGGL((layernorm_block<T>), dim3(unsigned(rows)), block, 0, st, x, g, b, y, cols, eps);
#undef TIA_LN
  return hipGetLastError();
}

template <typename T>
hipError_t softmax_dispatch(const T* x, T* y, int rows, int cols, hipStream_t st) {
  constexpr int VPL = 16 / sizeof(T);
  const bool vec = cols % VPL == 0 && al16(x) && al16(y);
  const dim3 grid(unsigned((rows + 3) / 4)), block(256);
  const int per = 64 * VPL;
  constexpr bool NT = sizeof(T) == 4;
#define TIA_SM(V, NV) hipLaunchKernelGGL((softmax_wave<T, V, NV, NT>), grid, block, 0, st, x, y, rows, cols)
  if (vec && cols <= per) TIA_SM(VPL, 1);
  else if (vec && cols <= 2 * per) TIA_SM(VPL, 2);
  else if (vec && cols <= 4 * per) TIA_SM(VPL, 4);
  else if (vec && cols <= 8 * per) TIA_SM(VPL, 8);
  else if (vec && VPL == 4 && cols <= 16 * per) TIA_SM(VPL, 16);
  else if (!vec && cols <= 64 * 16) TIA_SM(1, 16);
  else hipLaunchKernelGGL((softmax_block<T>), dim3(unsigned(rows)), block, 0, st, x, y, cols);
#undef TIA_SM
  return hipGetLastError();
}

}  // namespace

hipError_t layernorm_f16(const uint16_t* x, const uint16_t* g, const uint16_t* b, uint16_t* y,
                         int rows, int cols, float eps, hipStream_t st) {
  return layernorm_dispatch<uint16_t>(x, g, b, y, rows, cols, eps, st);
}
hipError_t layernorm_f16_p32(const uint16_t* x, const uint16_t* g, const uint16_t* b, uint16_t* y, int rows,
                             int cols, float eps, hipStream_t st) {
  if (rows < 1 || rows > 32 || cols % 64 != 0 || cols > 2048 || !al16(x) || !al16(g) || !al16(b) || !al16(y))
    return hipErrorInvalidValue;
  const dim3 grid(unsigned((rows + 3) / 4)), block(256);
#define TIA_LNP(NV) \
  hipLaunchKernelGGL((layernorm_wave<uint16_t, 8, NV, true>), grid, block, 0, st, x, g, b, y, rows, cols, eps)
  if (cols <= 512) TIA_LNP(1);
  else if (cols <= 1024) TIA_LNP(2);
  else TIA_LNP(4);
#undef TIA_LNP
  return hipGetLastError();
}
hipError_t softmax_f16(const uint16_t* x, uint16_t* y, int rows, int cols, hipStream_t st) {
  return softmax_dispatch<uint16_t>(x, y, rows, cols, st);
}
hipError_t layernorm_f32(const float* x, const float* g, const float* b, float* y, int rows,
                         int cols, float eps, hipStream_t st) {
  return layernorm_dispatch<float>(x, g, b, y, rows, cols, eps, st);
}
hipError_t softmax_f32(const float* x, float* y, int rows, int cols, hipStream_t st) {
  return softmax_dispatch<float>(x, y, rows, cols, st);
}
hipError_t layernorm_softmax_f32(const float* x, const float* g, const float* b, float* y, int rows, int cols,
                                float eps, hipStream_t st) {
  const bool vec = cols % 4 == 0 && al16(x) && al16(g) && al16(b) && al16(y);
  const dim3 grid(unsigned((rows + 3) / 4)), block(256);
#define TIA_LNSM(NV) \
  hipLaunchKernelGGL((layernorm_softmax_wave<4, NV>), grid, block, 0, st, x, g, b, y, rows, cols, eps)
  if (vec && cols <= 256) TIA_LNSM(1);
  else if (vec && cols <= 512) TIA_LNSM(2);
  else if (vec && cols <= 1024) TIA_LNSM(4);
  else if (vec && cols <= 2048) TIA_LNSM(8);
  else if (vec && cols <= 4096) TIA_LNSM(16);
  else {
    // Any other width or alignment: the two kernels, softmax in place on y.
    const hipError_t e = layernorm_dispatch<float>(x, g, b, y, rows, cols, eps, st);
    if (e != hipSuccess) return e;
    return softmax_dispatch<float>(y, y, rows, cols, st);
  }
#undef TIA_LNSM
  return hipGetLastError();
}
hipError_t splitk_residual_layernorm(const float* partials, int splits, int rows, int cols,
                                     const uint16_t* bias, uint16_t* x, const uint16_t* gamma,
                                     const uint16_t* beta, uint16_t* norm, float eps, hipStream_t st,
                                     bool p32) {
  if (cols > 64 * kResLnMaxPerLane || splits < 1) return hipErrorInvalidValue;
  if (p32 && (rows < 1 || rows > 32 || cols % 64 != 0)) return hipErrorInvalidValue;
  // Up to 4 splits: one wave per row, all loads in one round.
  if (splits <= 4 && cols % 8 == 0 && cols >= 8 && al16(partials) && al16(x) && al16(gamma) && al16(beta) && al16(norm) &&
      (!bias || al16(bias))) {
    const dim3 grid(unsigned((rows + 3) / 4)), block(256);
#define TIA_RLW(S_, NV_)                                                                                   \
  if (splits == S_) {                                                                                      \
    if (p32) hipLaunchKernelGGL((residual_ln_wave<S_, NV_, true>), grid, block, 0, st, partials, rows, cols, \
                                bias, x, gamma, beta, norm, eps);                                           \
    else hipLaunchKernelGGL((residual_ln_wave<S_, NV_, false>), grid, block, 0, st, partials, rows, cols,    \
                            bias, x, gamma, beta, norm, eps);                                               \
    return hipGetLastError();                                                                              \
  }
    if (cols <= 1024) {
      TIA_RLW(1, 2) TIA_RLW(2, 2) TIA_RLW(3, 2) TIA_RLW(4, 2)
    } else {
      TIA_RLW(1, 4) TIA_RLW(2, 4) TIA_RLW(3, 4) TIA_RLW(4, 4)
    }
#undef TIA_RLW
  }
  // LDS holds G rows of partial sums: keep it within 64 KiB.
  const size_t lds16 = 16 * cols * sizeof(float), lds8 = 8 * cols * sizeof(float);
  if (p32) {
#define TIA_RLNP(G, NPL, LDS)                                                                     \
  hipLaunchKernelGGL((splitk_residual_ln_kernel<G, NPL, true>), dim3(unsigned(rows)), dim3(64 * G), LDS, st, \
                     partials, splits, rows, cols, bias, x, gamma, beta, norm, eps)
    if (cols == 768) TIA_RLNP(16, 12, lds16);
    else if (cols == 1600) TIA_RLNP(8, 25, lds8);
    else if (cols <= 1024) TIA_RLNP(16, 0, lds16);
    else TIA_RLNP(8, 0, lds8);
#undef TIA_RLNP
    return hipGetLastError();
  }
#define TIA_RLN(G, NPL, LDS)                                                                              \
  hipLaunchKernelGGL((splitk_residual_ln_kernel<G, NPL>), dim3(unsigned(rows)), dim3(64 * G), LDS, st, partials, \
                     splits, rows, cols, bias, x, gamma, beta, norm, eps)
  if (cols == 768) TIA_RLN(16, 12, lds16);
  else if (cols == 1024) TIA_RLN(16, 16, lds16);
  else if (cols == 1600) TIA_RLN(8, 25, lds8);
  else if (cols == 2048) TIA_RLN(8, 32, lds8);
  else if (cols <= 1024) TIA_RLN(16, 0, lds16);
  else TIA_RLN(8, 0, lds8);
#undef TIA_RLN
  return hipGetLastError();
}
hipError_t gelu_f16(const uint16_t* x, uint16_t* y, int64_t count, hipStream_t st) {
  const bool vec = al16(x) && al16(y);
  const int64_t work = vec ? std::max<int64_t>(1, count / 8) : count;
  const int64_t blocks = std::min<int64_t>((work + 255) / 256, 8192);
  hipLaunchKernelGGL(gelu_kernel, dim3(unsigned(blocks)), dim3(256), 0, st, x, y, count, vec);
  return hipGetLastError();
}

}  // namespace tia
