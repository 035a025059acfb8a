// benchlib/liblimits.so: machine-limit probes for bench.py only (not part of
// the product libraries or headers; no reference counterpart).  They measure
// what the roofline figures are compared against on this MI355X:
//  * tia_diag_empty: an empty kernel; back-to-back graph replays of it give the
//    per-launch floor that every kernel of the path pays.
//  * tia_diag_stream: a pure streaming read, `wgs` workgroups each reading
//    `per_wg` contiguous bytes with 16-byte nontemporal loads, UNROLL 1 KiB
//    wave-loads in flight per wave (reduced into one dword per lane so no load
//    is dead); the best a kernel of that shape can do against HBM.
#include <hip/hip_runtime.h>
#include <stdint.h>


// Entry points (C ABI, loaded by bench.py through ctypes):
//   int tia_diag_empty(uintptr_t stream): enqueue one empty kernel.
//   int tia_diag_stream(const void* src, unsigned* out, int64_t out_dwords,
//                       int64_t per_wg, int wgs, int threads, uintptr_t stream):
//     enqueue a streaming read of wgs * per_wg bytes from 16-byte aligned `src`,
//     workgroup w reading [w * per_wg, (w + 1) * per_wg) with `threads` threads
//     (a multiple of 64, at most 1024); `out` (out_dwords long) receives
//     wgs * threads dwords; per_wg a positive multiple of 1024.  Both return 0,
//     or 1 on invalid arguments (an `out` too short included) or a launch error.

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__global__ void empty_kernel() {}

template <int UNROLL>
__global__ void stream_kernel(const u32x4* __restrict__ src, unsigned* __restrict__ out, int64_t per_wg) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const u32x4* base = src + int64_t(blockIdx.x) * (per_wg / 16);
  const int64_t records = per_wg / 1024;
  unsigned acc = 0;
  for (int64_t i = wave; i < records; i += int64_t(nw) * UNROLL) {
    u32x4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int64_t r = min(i + int64_t(u) * nw, records - 1);
      v[u] = __builtin_nontemporal_load(base + r * 64 + lane);
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) acc += v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  out[int64_t(blockIdx.x) * blockDim.x + threadIdx.x] = acc;
}

}  // namespace

extern "C" int tia_diag_empty(uintptr_t stream) {
  hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, reinterpret_cast<hipStream_t>(stream));
  return hipGetLastError() == hipSuccess ? 0 : 1;
}

extern "C" int tia_diag_stream(const void* src, unsigned* out, int64_t out_dwords, int64_t per_wg, int wgs,
                               int threads, uintptr_t stream) {
  if (!src || !out || per_wg < 1024 || per_wg % 1024 != 0 || wgs < 1 || threads < 64 || threads > 1024 ||
      threads % 64 != 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0 || int64_t(wgs) * threads > out_dwords)
    return 1;
  hipLaunchKernelGGL(stream_kernel<8>, dim3(wgs), dim3(threads), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(src), out, per_wg);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}
