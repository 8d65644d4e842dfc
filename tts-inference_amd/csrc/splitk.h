// Split-K across workgroups without a second launch and without cache-wide fences.
//
// The S workgroups that share one output tile each publish their fp32 partial into
// their own slot of the workspace and bump the tile's counter; the workgroup that
// draws S-1 from the counter sums every slot in split order (so the result does not
// depend on arrival order) and runs the epilogue, then resets the counter to zero.
//
// Ordering uses only per-access coherence: slots are written and read with
// agent-scope atomic stores and loads (write-through / coherent loads, sc1), and an
// explicit vmcnt(0) wait makes the slot stores complete before the counter update.
// No buffer_wbl2 / buffer_inv, which write back or invalidate a whole L2 and cost
// more than the split saves.  decode_wg additionally places all splits of a tile on
// the same XCD, so every access of one meeting goes through one L2.
#pragma once

#include "common.h"

namespace qtts {

// Workgroup id -> (tile, split): all splits of a tile share wg % 8, i.e. run on the
// same XCD (the dispatcher deals consecutive workgroups to the 8 XCDs round-robin).
__device__ __forceinline__ void decode_wg(int wg, int S, int& tile, int& split) {
  const int group = wg / (8 * S), within = wg - group * 8 * S;
  split = within >> 3;
  tile = group * 8 + (within & 7);
}

// Wait until every outstanding vector-memory operation of this wave has completed
// (s_waitcnt vmcnt(0); expcnt and lgkmcnt left at their maxima).  The signal fences
// keep the compiler from moving memory operations across the wait.
__device__ __forceinline__ void wait_vmem() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <typename T> __device__ __forceinline__ void store_coherent(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T> __device__ __forceinline__ T load_coherent(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Partial-sum addition: fp32 for the float GEMMs; int32 for the int8 GEMM, wrapping
// modulo 2^32 like the matrix cores' own accumulation (so the split order cannot
// change an integer result).
__device__ __forceinline__ float meet_add(float a, float b) { return a + b; }
__device__ __forceinline__ int meet_add(int a, int b) { return (int)((unsigned)a + (unsigned)b); }

// One meeting.  `slots` points at the tile's S slots of nthreads * NV values each,
// stored value-major (value v of thread t at v * nthreads + t) so that each store or
// load instruction of a wave covers 64 consecutive values; every participating
// thread calls this with its NV accumulator values.  Returns
// true in the last-arriving workgroup, whose threads then hold the full sums.
// `flag` is a __shared__ word (used when nthreads > 64).
template <int NV, typename T>
__device__ __forceinline__ bool splitk_meet(T (&acc)[NV], T* __restrict__ slots,
                                            unsigned* __restrict__ counter, int S, int split, int tid,
                                            int nthreads, unsigned* flag) {
  T* mine = slots + (int64_t)split * nthreads * NV + tid;
#pragma unroll
  for (int v = 0; v < NV; ++v) store_coherent(mine + (int64_t)v * nthreads, acc[v]);
  wait_vmem();
  unsigned prev = 0;
  if (nthreads > 64) {
    __syncthreads();  // every wave's stores have completed (each waited above)
    if (tid == 0) *flag = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    prev = *flag;
  } else {
    if (tid == 0) prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = __shfl(prev, 0, 64);
  }
  if (prev != (unsigned)(S - 1)) return false;
#pragma unroll
  for (int v = 0; v < NV; ++v) acc[v] = T(0);
  for (int s = 0; s < S; ++s) {
    // All of a slot's loads go out before any is consumed: the scheduler keeps atomic
    // loads in order and would otherwise wait for each one before the next.
    const T* src = slots + (int64_t)s * nthreads * NV + tid;
    T part[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) part[v] = load_coherent(src + (int64_t)v * nthreads);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int v = 0; v < NV; ++v) acc[v] = meet_add(acc[v], part[v]);
  }
  if (tid == 0) reset_counter(counter);
  return true;
}

}  // namespace qtts
