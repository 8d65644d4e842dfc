// Building blocks of the LDS-pipelined GEMM kernels (tile.hip, tile_fp8.hip): direct
// global -> LDS loads, vmcnt waits by stage, and a fence-free workgroup barrier.
#pragma once

#include "common.h"

namespace qtts {

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void gbl_void_t;

// One 16-byte-per-lane direct load: lane l's 16 bytes land at lds_wave + 16 l.
__device__ __forceinline__ void load_to_lds16(const void* src, void* lds_wave) {
  __builtin_amdgcn_global_load_lds((gbl_void_t*)src, (lds_void_t*)lds_wave, 16, 0, 0);
}

// s_waitcnt vmcnt(N), expcnt and lgkmcnt left at their maxima.
template <int N> __device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// s_waitcnt lgkmcnt(0), vmcnt and expcnt left at their maxima: this wave's LDS
// accesses are complete (before a barrier that publishes them to other waves).
__device__ __forceinline__ void wait_lgkmcnt0() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Workgroup barrier without a memory fence: stage visibility is established by each
// wave's own vmcnt wait before it; the signal fences keep the compiler from moving
// LDS accesses across it.
__device__ __forceinline__ void barrier_only() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// vmcnt(A * FPW) for the largest A <= min(ahead, AMAX): wait until at most `ahead`
// stages of this wave's loads are still in flight.
template <int FPW, int AMAX> __device__ __forceinline__ void wait_stages(int ahead) {
  if constexpr (AMAX > 0) {
    if (ahead >= AMAX) {
      wait_vmcnt<AMAX * FPW>();
      return;
    }
    wait_stages<FPW, AMAX - 1>(ahead);
  } else {
    wait_vmcnt<0>();
  }
}

constexpr int kLdsBytes = 160 * 1024;  // LDS per workgroup on gfx950

}  // namespace qtts
