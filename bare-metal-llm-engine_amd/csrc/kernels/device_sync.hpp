// device_sync.hpp -- waits and barriers shared by the pipelined kernels.
//
// Vector-memory loads complete in issue order, so a kernel that issues its
// own loads in a known order can wait for an earlier one with
// `s_waitcnt vmcnt(<loads issued after it>)` and leave the later ones in
// flight; the compiler's own waits (and the fence __syncthreads() carries)
// wait for all of them.
#pragma once

#include <hip/hip_runtime.h>

namespace eng {

// s_waitcnt immediate waiting for vmcnt <= n only (expcnt 7 and lgkmcnt 15
// are the "don't wait" values).
constexpr int vmcnt_le(int n) { return (n & 15) | (7 << 4) | (15 << 8) | (((n >> 4) & 3) << 14); }
// s_waitcnt immediate waiting for lgkmcnt == 0 only (LDS accesses done).
constexpr int lgkmcnt_zero() { return 15 | (7 << 4) | (3 << 14); }

// Workgroup barrier without a memory fence: __syncthreads()'s fence compiles
// to a wait for every load in flight. The memory clobber keeps the compiler
// from moving LDS accesses across it; a caller that wrote LDS waits for
// lgkmcnt(0) first.
__device__ __forceinline__ void barrier_no_fence() { asm volatile("s_barrier" ::: "memory"); }

// LDS writes of this wave done, then the fence-free barrier, with scheduling
// barriers so the compiler moves nothing across it.
__device__ __forceinline__ void lds_barrier() {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_s_waitcnt(lgkmcnt_zero());
#endif
  __builtin_amdgcn_sched_barrier(0);
  barrier_no_fence();
  __builtin_amdgcn_sched_barrier(0);
}

// 16-byte direct global -> LDS load: lane l's 16 bytes land at lds + 16 l
// bytes (lds the same in every lane of the wave), from any address the lane
// names. The builtin is device-only.
template <typename T>
__device__ __forceinline__ void dma16(const T* src, T* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 0);
#endif
}

}  // namespace eng
