// wp_apply.h -- launch interface of the gfx950 plan / shrink / expand kernels.
#pragma once

#include <hip/hip_runtime.h>

#include "wp_types.h"

namespace wp {

// Kernel arguments of one shrink or expand launch (passed by value).
struct ApplyArgs {
  const void* x;   // X [T, ldx]
  int64_t ldx;
  void* h;         // H [T, ldh] (I/O dtype)
  int64_t ldh;
  void* y;         // Y [T, ldy]
  int64_t ldy;
  int32_t d_model;
  int32_t rank;      // 8/16/32/64, or 0 for mixed ranks (per adapter)
  int32_t dc;        // shrink d-range per workgroup, multiple of 128
  int32_t n_chunks;  // ceil(d_model / dc)
  int32_t n_ochunks; // expand workgroups per block (all slices)
  int32_t ptok;      // rows per chunk in `partials` (>= tokens in the plan)
  int32_t pstride;   // floats per partial row (rank, or 64 when mixed)
  float* partials;   // fp32 [n_chunks][ptok][pstride]
  PlanView plan;
  Weights w;
};

// Builds the step plan from token_lora_indices (wp_plan.hip).
hipError_t launch_plan(const void* idx, int idx_is_int64, int T, uint32_t* header, Segment* segments, Block* blocks,
                       int32_t* perm, int seg_cap, int block_cap, hipStream_t stream);

hipError_t launch_shrink(int dtype_bf16, const ApplyArgs& a, int max_blocks, hipStream_t stream);
hipError_t launch_expand(int dtype_bf16, const ApplyArgs& a, int max_blocks, hipStream_t stream);

// Output columns one expand workgroup produces.
int expand_cols_per_workgroup();

}  // namespace wp
