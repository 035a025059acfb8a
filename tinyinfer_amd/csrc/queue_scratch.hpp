// Scratch for kernels that finish their own split work inside one launch
// (split-K GEMMs, split-key decode attention) without any allocation: static
// device arrays, one slot per hardware queue.
//
// Why per queue: HIP enqueues every kernel dispatch with the AQL barrier bit
// set, so dispatches on one hardware queue never overlap in time; kernels that
// run at the same time come from different queues.  A kernel finds its queue's
// slot through the queue address (__builtin_amdgcn_queue_ptr), which every
// workgroup of a dispatch sees alike.  Streams share hardware queues (HIP maps
// them round-robin onto GPU_MAX_HW_QUEUES queues, 4 by default), so a slot is
// only ever used within one dispatch: split work is finished by the last
// workgroup of the same launch, never by a later one.
//
// Slots are claimed once per queue with a compare-and-swap on the key table and
// never released (a process uses a handful of queues per device), so a key
// once seen is final; a stale cached read can only show a free entry, which the
// compare-and-swap then resolves.  With more than kQueueSlots queues in use on
// one device, further queues share slot (queue address / 4096) mod kQueueSlots
// and calls that overlap on two such queues race.
//
// Each translation unit that includes this header and expands
// TIA_QUEUE_POOL(prefix, floats, counters) holds its own pool; counters are
// zero at load and every kernel leaves them zero.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tia {

constexpr int kQueueSlots = 32;
// Counters sit 32 apart (one 128-byte line each).
constexpr int kCounterStride = 32;

// A pool of `slots` (at most kQueueSlots) slots whose dispatches, when every
// slot is taken by other queues, get no slot (queue_slot_claim returns -1) and
// must then run a plan that needs none.
#define TIA_QUEUE_POOL_N(prefix, slots, data_floats, counter_count)                                 \
  static __device__ __align__(256) unsigned long long prefix##_keys[(slots)];                      \
  static __device__ __align__(256) float prefix##_data[(slots)][(data_floats)];                    \
  static __device__ __align__(256) unsigned prefix##_ctr[(slots)][(counter_count) * ::tia::kCounterStride];

#define TIA_QUEUE_POOL(prefix, data_floats, counter_count)                                          \
  static __device__ __align__(256) unsigned long long prefix##_keys[::tia::kQueueSlots];            \
  static __device__ __align__(256) float prefix##_data[::tia::kQueueSlots][(data_floats)];          \
  static __device__ __align__(256) unsigned prefix##_ctr[::tia::kQueueSlots][(counter_count) * ::tia::kCounterStride];

// The slot of the calling dispatch's queue.  Called by a whole wave (every lane
// gets the same answer); `key` is keys[lane] for lanes < kQueueSlots, read
// earlier with a plain load (it may be stale: see above).
__device__ __forceinline__ int queue_slot_resolve(unsigned long long* keys, unsigned long long key) {
  const unsigned long long me = reinterpret_cast<unsigned long long>(__builtin_amdgcn_queue_ptr());
  const int lane = int(threadIdx.x & 63);
  const unsigned long long hit = __ballot(lane < kQueueSlots && key == me);
  if (hit) return __builtin_ffsll(static_cast<long long>(hit)) - 1;
  // Entries that read as free, in index order: claim the first that is free,
  // or find this queue's key in it (a claim another workgroup made since).
  unsigned long long cand = __ballot(lane < kQueueSlots && key == 0);
  while (cand) {
    const int e = __builtin_ffsll(static_cast<long long>(cand)) - 1;
    cand &= cand - 1;
    unsigned long long prev = 0;  // the entry's value before the exchange
    if (lane == 0)
      __hip_atomic_compare_exchange_strong(keys + e, &prev, me, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
    prev = __shfl(prev, 0, 64);
    if (prev == 0 || prev == me) return e;
  }
  return int((me >> 12) % kQueueSlots);
}

// The slot of the calling dispatch's queue in a pool of `slots` entries, or
// -1 when every entry belongs to another queue.  Called by a whole wave;
// every wave of a dispatch gets the same answer (a key once claimed is final).
__device__ __forceinline__ int queue_slot_claim(unsigned long long* keys, int slots) {
  const unsigned long long me = reinterpret_cast<unsigned long long>(__builtin_amdgcn_queue_ptr());
  const int lane = int(threadIdx.x & 63);
  const unsigned long long key = lane < slots ? keys[lane] : ~0ull;
  const unsigned long long hit = __ballot(lane < slots && key == me);
  if (hit) return __builtin_ffsll(static_cast<long long>(hit)) - 1;
  unsigned long long cand = __ballot(lane < slots && key == 0);
  while (cand) {
    const int e = __builtin_ffsll(static_cast<long long>(cand)) - 1;
    cand &= cand - 1;
    unsigned long long prev = 0;
    if (lane == 0)
      __hip_atomic_compare_exchange_strong(keys + e, &prev, me, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
    prev = __shfl(prev, 0, 64);
    if (prev == 0 || prev == me) return e;
  }
  // Entries read as taken may have been claimed by this queue since: one
  // more look at the whole table.
  const unsigned long long again = lane < slots ? __hip_atomic_load(keys + lane, __ATOMIC_RELAXED,
                                                                     __HIP_MEMORY_SCOPE_AGENT) : 0ull;
  const unsigned long long hit2 = __ballot(lane < slots && again == me);
  return hit2 ? __builtin_ffsll(static_cast<long long>(hit2)) - 1 : -1;
}

// Relaxed agent-scope accesses: visible to every XCD (the hardware writes these
// stores through the XCD's L2 and reads these loads coherently).
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16-byte versions through a buffer resource: the same agent scope as the
// accesses above (cache policy SC1 = 0x10 on gfx950, which the relaxed
// agent-scope atomics above also carry).
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4q_t __attribute__((ext_vector_type(4)));
constexpr int kAgentScopePolicy = 0x10;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t agent_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, int(bytes), 0x00020000);
}
__device__ __forceinline__ void st_agent4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, f32x4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4q_t, v), r, int(byte_off), 0, kAgentScopePolicy);
}
__device__ __forceinline__ f32x4_t ld_agent4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, int(byte_off), 0, kAgentScopePolicy));
}

// Arrival of one of `parties` workgroups at `counter` after it stored its
// share with st_agent; called by a whole wave.  Returns true in the last
// workgroup to arrive, which then reads every share with ld_agent and must
// call depart().  The wait makes this wave's stores complete (acknowledged at
// the coherence point) before the counter moves; the last arriver's loads
// follow the counter's value.
__device__ __forceinline__ bool arrive_last(unsigned* counter, int parties) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  unsigned old = 0;
  if ((threadIdx.x & 63) == 0)
    old = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __builtin_amdgcn_readfirstlane(old);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return old == unsigned(parties - 1);
}
// The same for a whole workgroup whose waves all stored shares: each wave
// waits for its own stores, the workgroup meets, one thread moves the counter,
// and every thread learns whether this workgroup arrived last.
// `flag` is an int of LDS the workgroup no longer reads (the overload without
// it declares one: a kernel sized to fill LDS exactly passes its own).
__device__ __forceinline__ bool wg_arrive_last(unsigned* counter, int parties, int* flag) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    *flag = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == unsigned(parties - 1);
  __syncthreads();
  return *flag != 0;
}
__device__ __forceinline__ bool wg_arrive_last(unsigned* counter, int parties) {
  __shared__ int last;
  return wg_arrive_last(counter, parties, &last);
}
// Leaves the counter at zero for the next dispatch on this queue (called by
// the last arriver once; any thread of it).
__device__ __forceinline__ void depart(unsigned* counter) {
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace tia
