// wp_sync.h -- the workgroup barrier the gfx950 kernels use for LDS data.
#pragma once

#include <hip/hip_runtime.h>

namespace wp {

// Workgroup barrier for LDS data only: waits for this wave's LDS accesses
// (and scalar loads: both count on lgkmcnt) but not for its global loads and
// stores in flight, which __syncthreads (a workgroup-scope fence plus
// s_barrier) would drain with s_waitcnt vmcnt(0).  Every LDS write a wave
// issued before the barrier is visible to every wave of the workgroup after
// it.  A value that reached LDS from a global load was waited for (vmcnt)
// before the LDS write that stores it could issue, so the pattern "global
// load -> LDS write -> lds_barrier -> LDS read by another wave" is ordered.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

}  // namespace wp
