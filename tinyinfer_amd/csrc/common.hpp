// Shared device helpers for the gfx950 (CDNA4, wave64) kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tia {

typedef _Float16 f16;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Fragment-packed activations ("P32") for decode matrices of at most 32 rows
// and K % 64 == 0: the 1 KiB MFMA A operand of rows 16t..16t+15, K columns
// 64c + 32s .. +31 (lane j + 16g holding row 16t + j, columns +8g .. +8g+7) is
// contiguous at element ((c * 2 + t) * 2 + s) * 512, so a wave loads it with
// one fully used 16-byte-per-lane instruction (row-major A would touch 16 rows
// with half-used cache lines per instruction).  A [32, K] matrix takes 32 * K
// elements; 8 consecutive columns k..k+7 (k % 8 == 0) of a row are contiguous.
__host__ __device__ __forceinline__ int64_t p32_off(int m, int k) {
  return ((int64_t(k >> 6) * 2 + (m >> 4)) * 2 + ((k >> 5) & 1)) * 512 + ((m & 15) + 16 * ((k >> 3) & 3)) * 8 +
         (k & 7);
}

// fp16_rn of an fp32 value: the value is first rounded to fp32 as its own
// step.  Without the opaque copy the compiler may fuse the operation that
// produced it (a multiply, add or fma) with the conversion into one
// mixed-precision fma that rounds the exact result straight to fp16 -- one
// rounding where the reference's fp32 arithmetic followed by __float2half_rn
// has two, so 1-ulp differences in rare cases.  The conversion itself is
// v_cvt_f16_f32 (nearest-even under the default mode register).
__device__ __forceinline__ f16 f16r(float v) {
  asm volatile("" : "+v"(v));
  return f16(v);
}
// fp16 bits <-> fp32.
__device__ __forceinline__ float h2f(uint16_t bits) { return float(__builtin_bit_cast(f16, bits)); }
__device__ __forceinline__ uint16_t f2h(float v) { return __builtin_bit_cast(uint16_t, f16r(v)); }
__device__ __forceinline__ float rt16(float v) { return float(f16r(v)); }

// tanh(x) = sign(x) (1 - 2 / (exp(2 |x|) + 1)) on the hardware exp2 and
// reciprocal (about 2e-7 absolute error; exp overflows to +inf for large |x|,
// giving exactly +-1).  Against the device libm's tanhf: fewer instructions
// and no branches, in the configs[1] GEMM epilogue M = 512,
// 768 -> 3072 12.76 -> 11.53 us, and over all 63 488 finite fp16 inputs the
// fp16 GELU below differs from the CPU oracle's (std::tanh) in 5 values by
// one ulp (1 with tanhf).
__device__ __forceinline__ float tanh_exp(float x) {
  const float e = __builtin_amdgcn_exp2f(fabsf(x) * 2.8853900817779268f);  // exp(2|x|) = 2^(2 log2(e) |x|)
  return copysignf(1.f - 2.f * __builtin_amdgcn_rcpf(e + 1.f), x);
}
// tanh-approximated GELU (GPT-2 "gelu_new"): 0.5 z (1 + tanh(sqrt(2/pi) (z + 0.044715 z^3))),
// the reference's expression (reference kernels/src/cuda/tc/elementwise.cu:29-31).
__device__ __forceinline__ float gelu_tanh(float z) {
  return 0.5f * z * (1.f + tanh_exp(0.7978845608028654f * (z + 0.044715f * z * z * z)));
}

// Workgroup barrier that orders LDS accesses only: outstanding global loads
// stay in flight across it (__syncthreads would wait for them).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Running argmax step: largest value, lowest index on ties; NaN never wins
// (reference llm/src/runtime.cu:59-66).
__device__ __forceinline__ void amax_merge(float& bv, int& bi, float v, int i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

// Butterfly reductions across the 64 lanes of a wave.  Every lane ends with the
// full result.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Reduction across a whole workgroup of NW waves through a small LDS array of
// at least NW floats.  All threads return the total.
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* lds) {
  v = wave_sum(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) lds[w] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < NW; ++i) t += lds[i];
  return t;
}
template <int NW>
__device__ __forceinline__ float block_max(float v, float* lds) {
  v = wave_max(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) lds[w] = v;
  __syncthreads();
  float t = lds[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) t = fmaxf(t, lds[i]);
  return t;
}

}  // namespace tia
