// wp_apply.h -- launch interface of the gfx950 plan / shrink / expand kernels.
#pragma once

#include <hip/hip_runtime.h>

#include "wp_types.h"

namespace wp {

// Loads the first dword of every 64-byte line of a kernel's first `BYTES`
// bytes of arguments at once (scalar loads, all in flight together) and
// waits for them once.  A kernel's argument reads further down, which the
// compiler issues one dependent branch at a time, then hit the scalar cache
// instead of missing line after line: measured on MI355X, the cfg2 decode
// step 1219 -> 1189 us and cfg5's 44-launch step 465 -> 425 us.  BYTES must
// not exceed the kernel's explicit arguments.
template <int BYTES>
__device__ __forceinline__ void touch_kernel_args() {
  const uint32_t* ka = (const uint32_t*)__builtin_amdgcn_kernarg_segment_ptr();
  uint32_t t = 0;
#pragma unroll
  for (int i = 0; i < BYTES / 4; i += 16) t ^= ka[i];
  asm volatile("" ::"s"(t));
}
// The same in two steps: the loads where touch_kernel_args_issue is called,
// the wait where its result is passed to touch_kernel_args_wait.
template <int BYTES>
__device__ __forceinline__ uint32_t touch_kernel_args_issue() {
  const uint32_t* ka = (const uint32_t*)__builtin_amdgcn_kernarg_segment_ptr();
  uint32_t t = 0;
#pragma unroll
  for (int i = 0; i < BYTES / 4; i += 16) t ^= ka[i];
  return t;
}
__device__ __forceinline__ void touch_kernel_args_wait(uint32_t t) { asm volatile("" ::"s"(t)); }

// Kernel arguments of one shrink or expand launch (passed by value).
struct ApplyArgs {
  const void* x;   // X [T, ldx]
  int64_t ldx;
  void* h;         // H [T, ldh] (I/O dtype)
  int64_t ldh;
  void* y;         // Y [T, ldy]
  int64_t ldy;
  int32_t d_model;
  int32_t rank;       // 8/16/32/64, or 0 for mixed ranks (per adapter)
  int32_t dc;         // shrink d-range per workgroup, multiple of 128
  int32_t n_chunks;   // ceil(d_model / dc): d-ranges, i.e. partials per H value
  int32_t srows;      // rank rows per shrink workgroup: kShrinkRows, or kShrinkRowsFused (fused roles only)
  int32_t n_rgroups;  // rank groups of srows rows; n_chunks * n_rgroups shrink workgroups per block
  int32_t n_ochunks;  // 256-column output chunks per block (all slices)
  int32_t n_sub;      // output chunks per expand workgroup (fused), else 1
  int32_t tiles;      // most 16-token tiles per block of the plan (1 or 4)
  int32_t n_slots;    // block slots of the grid (>= the plan's block count)
  int32_t hs;         // elements per H / partial row: n_a x hs1
  int32_t hs1;        // elements of one A slice's H in a row: rank, or 64 for mixed ranks
  int32_t pad_rank;   // 1: the shrink side writes all hs1 rows of a slice, zeros past the adapter's rank
                      // (table mode with one A per slice and mixed ranks: every slice's partial has one width)
  int32_t ptok;       // rows per chunk of `part` (plan positions)
  int32_t red_first;  // shrink() of decode-sized plans: 1 = the block reducers are dispatched before the
                      // shrink workgroups they wait for (only when they take at most half of the resident
                      // workgroups, so that those always find room)
  float* part;        // fp32 partial H by plan position: [n_chunks][ptok][hs], kPartialEmpty between calls
  uint32_t* consumed; // per block (stride kCounterStride): fused calls count expand workgroups done reading,
                      // shrink() counts d-range workgroups done; zero between calls
  uint32_t spin_limit; // polls before a wait on partials gives up (kDefaultSpinLimit)
  uint64_t* trace;     // traced builds (WP_TRACE) only: kTraceWords timestamps per workgroup, or null
  int64_t trace_words; // capacity of `trace` (a launch whose grid does not fit is not traced)
  PlanView plan;
  Weights w;
  // shrink() only: 1 = H is fp32 and the call adds alpha * sum to it,
  // unrounded (vLLM's lora_shrink buffer); 0 = H = rn(alpha * sum) in the
  // I/O type.  At the end of the arguments: fields placed before the hot
  // kernels' argument reads measured up to 0.3 us more per launch.
  int32_t h_f32;
  int32_t pad_end;
};

// Words per workgroup of a traced build's timestamp buffer: stamps 0..6 and
// a tag (role and block) in word 7.
constexpr int kTraceWords = 8;
// 1 in a library built with WP_TRACE.
int traced_build();

// Bound of a wait on partials: polls of ~1 us each, so about 0.1 s.
constexpr uint32_t kDefaultSpinLimit = 1u << 17;

// Builds the step plan from token_lora_indices (wp_plan.hip).
// Blocks hold at most bt (<= kBlockTokens) tokens.  The same launch first
// does what `m` asks (publications into the adapter table; the partial
// buffer's repair after a give-up); m may be null.
// bentries (may be null): each block's adapter-table entry at the table
// version left in header[kHdrPlanVer] (Weights::a_base in table mode).
hipError_t launch_plan(const void* idx, int idx_is_int64, int T, uint32_t* header, Segment* segments, Block* blocks,
                       int32_t* perm, int32_t* bperm, Entry* bentries, int seg_cap, int block_cap, int bt,
                       const Maint* m, hipStream_t stream);
// The plan build's maintenance alone (one workgroup), for eager calls that
// run between plan builds.
hipError_t launch_maintain(uint32_t* header, const Maint& m, hipStream_t stream);

// Tiny writes of adapter-table entries and of one slot publication, in stream
// order (one wave): pub (if not null) gets (pub_id, pub_gen, pub_entry) under
// its sequence lock, the retired generations are raised, then dst[i] =
// val[i] for i < n.
constexpr int kMaxEntryWrites = 16;
struct EntryWrites {
  int32_t n;
  int32_t pub_id;
  uint32_t pub_gen;
  SlotPub* pub;
  Entry pub_entry;
  Entry* dst[kMaxEntryWrites];
  Entry val[kMaxEntryWrites];
  // Slot generations released: *retire[i] = max(*retire[i], retire_gen[i]).
  int32_t n_retire;
  uint32_t* retire[kMaxEntryWrites];
  uint32_t retire_gen[kMaxEntryWrites];
  // Plan header whose table version (kHdrTableVer) is raised once the
  // writes are done, or null.
  uint32_t* header;
};
hipError_t launch_entry_writes(const EntryWrites& w, hipStream_t stream);

// Staging copies: job j copies a_bytes from src_a to dst_a and b_bytes from
// src_b to dst_b (sources in device memory or in pinned host memory the
// device reads directly), over kStageWorkgroups workgroups; the job's last
// workgroup to finish then publishes (pub_id, pub_gen, pub_entry) into *pub
// under its sequence lock.  pub->copies counts the job's finished workgroups
// (zero between jobs).
constexpr int kMaxStageJobs = 8;
constexpr int kStageWorkgroups = 8;
struct StageJob {
  const void* src_a;
  void* dst_a;
  uint64_t a_bytes;  // multiple of 16
  const void* src_b;
  void* dst_b;
  uint64_t b_bytes;  // multiple of 16
  SlotPub* pub;
  int32_t pub_id;
  uint32_t pub_gen;
  int32_t pad;
  Entry pub_entry;
};
struct StageJobs {
  int32_t n;
  int32_t pad;
  StageJob job[kMaxStageJobs];
};
hipError_t launch_stage_copies(const StageJobs& jobs, hipStream_t stream);

// shrink(): a workgroup streams its d-range (a.dc, a multiple of
// kShrinkSlices * 128 columns) in groups of kShrinkSlices 128-column slices.
constexpr int kShrinkSlices = 8;

// One launch: shrink + expand of a whole add_lora call (partials, counters).
hipError_t launch_fused(int dtype_bf16, const ApplyArgs& a, hipStream_t stream);
// shrink(): one workgroup per (block, d-range) computes every rank row; the
// block's last workgroup to finish sums the d-ranges into H[token].
hipError_t launch_shrink(int dtype_bf16, const ApplyArgs& a, hipStream_t stream);
// shrink() of decode-sized plans: the fused kernel's shrink workgroups
// (kShrinkRowsFused rows x d-range) and one reducer per block writing H;
// a.part is the fused calls' partial buffer (kPartialEmpty between calls).
hipError_t launch_shrink_small(int dtype_bf16, const ApplyArgs& a, hipStream_t stream);
// expand(): expand from a caller-provided token-indexed H.
hipError_t launch_expand(int dtype_bf16, const ApplyArgs& a, hipStream_t stream);

// Sets n 32-bit words at p to v (vector stores; a kernel, so that a caller
// may capture it in a graph).
hipError_t launch_fill_u32(uint32_t* p, uint32_t v, size_t n, hipStream_t stream);

// The base linear plus its per-token LoRA delta in one launch (see
// linear_kernel): a is an add_lora call's arguments (stacked weights, the
// kShrinkOnly split, a.h the token-indexed H rows, a.y the output), l the
// GEMM's.
struct LinearArgs {
  const void* w;        // [n_out, ldw] base weight (the I/O type)
  int64_t ldw;
  const void* bias;     // [n_out] or null
  int32_t n_out;        // multiple of 16
  int32_t tokens;       // rows of x and y
  int32_t groups;       // token groups of 128
  int32_t splits;       // K-ranges per column tile
  int32_t k_range;      // columns of x per K-range (multiple of 128)
  int32_t pad;
  float* gpart;         // [groups][n_out / 16][splits][128][16] fp32 partials
  uint32_t* tile_cnt;   // [groups * n_out / 16] counters (zero between calls)
  uint32_t* hflag;      // [n_slots] H-ready flags (zero between calls)
  uint32_t* hcnt;       // [n_slots] readers counted on each flag (zero between calls)
};
hipError_t launch_linear(int dtype_bf16, const ApplyArgs& a, const LinearArgs& l, hipStream_t stream);

// Streams `bytes` (a multiple of 16) from p with 16-byte non-temporal loads
// over `workgroups` workgroups of 512 threads and stores nothing but an
// improbable fold into sink (512 x 16 bytes); bytes == 0 launches one
// workgroup that does nothing.  A measurement of the device's read rate and
// launch cost, not part of any call.
hipError_t launch_read_probe(const void* p, size_t bytes, void* sink, int workgroups, hipStream_t stream);

// *out = *word and *word = 0, as one device-scope atomic exchange (one
// thread, in stream order).
hipError_t launch_take_word(uint32_t* word, uint32_t* out, hipStream_t stream);

// The per-token work of vLLM V1's LoRA op surface around the grouped kernels
// (wp_aux.hip prep_kernel), one workgroup per block slot of the plan:
//   * h_src != null: the rank columns of slice s of token t's H,
//     h_src[s * h_slice_stride + t * h_row_stride + k] (fp32 if h_f32, else
//     the I/O type), rounded into h_dst[t * ldh_dst + s * rank + k];
//   * zero_y: y[t, y_off[s] .. + o_size[s]) = 0 for every slice;
//   * otherwise, for each slice with bias[s]: y = rn(y + bias[s][id]) over
//     the window (bias rows bias_stride[s] elements apart; ids >= num_ids
//     flagged kErrIdRange).
struct PrepArgs {
  PlanView plan;
  int32_t n_slots;
  int32_t n_slices;
  int32_t num_ids;
  int32_t rank;
  const void* h_src;
  int64_t h_slice_stride;
  int64_t h_row_stride;
  void* h_dst;
  int32_t ldh_dst;
  int32_t h_f32;
  void* y;
  int64_t ldy;
  int32_t zero_y;
  int32_t pad;
  int32_t o_size[kMaxSlices];
  int32_t y_off[kMaxSlices];
  const void* bias[kMaxSlices];
  int64_t bias_stride[kMaxSlices];
};
hipError_t launch_prep(int dtype_bf16, const PrepArgs& p, hipStream_t stream);

// Barrier probe: `workgroups` workgroups of `threads` (256 or 1024) run
// `rounds` rounds of LDS writes, lds_barrier(), and reads of every slot;
// slots that did not hold the round's value are added to *mismatches.
hipError_t launch_barrier_probe(const uint32_t* salts, int rounds, int threads, int workgroups, uint32_t* mismatches,
                                hipStream_t stream);

// Handoff probe (a measurement, not part of any call): see wp_aux.hip.
struct HandoffProbe {
  const void* a;     // streamed before the count (a call's A and X bytes)
  uint64_t a16;      // 16-byte words
  const void* b;     // streamed around the wait (B, and Y read)
  uint64_t b16;
  void* y;           // written last (Y)
  uint64_t y16;
  uint32_t* counters;  // 2 x kCounterStride words per group, zero between launches
  uint32_t* err;       // bit 0: a wait gave up
  int32_t group;       // workgroups that wait for each other
  int32_t mode;        // 0 no wait, 1 first b batch before the wait, 2 all of b after it
  uint32_t spin_limit;
  int32_t pad;
};
hipError_t launch_handoff_probe(const HandoffProbe& p, int workgroups, hipStream_t stream);

// Output columns one expand workgroup produces.
int expand_cols_per_workgroup();
// Waves per SIMD the fused kernel for `rank` (0: mixed) runs at, single- or
// multi-chunk: with the CU count, how many of its workgroups are resident.
int fused_waves_per_simd(int rank, int multi);
// Waves per SIMD of shrink() on decode-sized plans (its resident workgroups
// per compute unit).
int shrink_small_waves_per_simd();

}  // namespace wp
