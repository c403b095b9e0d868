// wp_plan.hip -- once-per-step segment plan, built on the GPU (gfx950).
//
// Input: token_lora_indices[T] (int64 or int32) in HBM.  One workgroup builds,
// with every intermediate held in LDS (gfx950: 160 KB per workgroup):
//
//   1. the exported segment table, bit-exact with the reference's
//      build_seg_bounds_kernel (csrc/kernels/warp_pipe_r32.cu:461-512):
//      maximal runs of equal ids in token order, ids < 0 skipped, every run
//      split into pieces of 32 tokens (the last one takes the remainder),
//      slots assigned in token-start order by an exclusive scan;
//   2. the grouping the apply kernels run on (no reference counterpart): the
//      runs are sorted by adapter id (bitonic sort of 64-bit (id, run) keys, so
//      token order is kept inside an adapter), concatenated into `perm`, and
//      each adapter's tokens are cut into blocks of `bt` tokens.  Every touched
//      adapter's weights are then streamed once per block instead of once per
//      run (about 232 runs vs 49 adapters for 256 Zipf-routed decode tokens).
//
// The reference uses one 256-thread block with a serial per-run scan and a
// Hillis-Steele scan over shared memory, writing over PCIe into mapped host
// memory.  Here: wave64 shuffle scans, LDS-resident arrays, HBM outputs written
// by all threads in parallel (each output slot finds its run by binary search
// over the scanned offsets), and capacities of 256 / 2048 / 8192 tokens.
#include <hip/hip_runtime.h>

#include "wp_apply.h"
#include "wp_sync.h"

namespace wp {
namespace {


// Exclusive scan of one int per thread across the workgroup.  `scratch` holds
// NT/64 ints.  Returns the thread's exclusive prefix; *total gets the sum.
// Begins and ends with a workgroup barrier.
template <int NT>
__device__ __forceinline__ int block_exclusive_scan(int v, int* scratch, int* total) {
  constexpr int kWaves = NT / 64;
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  lds_barrier();
  if (lane == 63) scratch[wid] = x;
  lds_barrier();
  if (wid == 0) {
    int w = lane < kWaves ? scratch[lane] : 0;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(w, off, 64);
      if (lane >= off) w += y;
    }
    if (lane < kWaves) scratch[lane] = w;
  }
  lds_barrier();
  const int base = wid > 0 ? scratch[wid - 1] : 0;
  *total = scratch[kWaves - 1];
  lds_barrier();
  return base + x - v;
}

// Largest i in [0, n) with a[i] <= q, for non-decreasing a and a[0] <= q.
__device__ __forceinline__ int upper_index(const int* a, int n, int q) {
  int lo = 0;
  int hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a[mid] <= q) {
      lo = mid;
    } else {
      hi = mid - 1;
    }
  }
  return lo;
}

// Traced builds (-DWP_TRACE): thread 0 records the 100 MHz real-time counter
// at the plan build's phase boundaries into m.trace[0..7], after waiting for
// its memory operations: 0 entry, 1 ids in LDS (maintenance done), 2 run
// starts, 3 segment table stored, 4 runs sorted, 5 perm stored, 6 block
// table stored, 7 block token lists and header stored.
#ifdef WP_TRACE
__device__ __forceinline__ void plan_stamp(const Maint& m, int i) {
  if (m.trace != nullptr && threadIdx.x == 0) {
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    m.trace[i] = wall_clock64();
  }
}
#else
__device__ __forceinline__ void plan_stamp(const Maint&, int) {}
#endif

// ---------------------------------------------------------- maintenance ----

__device__ __forceinline__ uint64_t agent_load64(const void* p) {
  return __hip_atomic_load(static_cast<const uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void agent_store64(void* p, uint64_t v) {
  __hip_atomic_store(static_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// What a plan build does first (every thread of the workgroup takes part):
//   * each ready staging-slot publication is written into the adapter table,
//     so that every kernel of the step that follows sees the same table (a
//     publication read while its writer is at work -- odd or changed sequence
//     -- is left for the next build);
//   * after a give-up (kHdrPoison), the partial buffer is refilled with
//     kPartialEmpty and the per-block counters cleared, then the word reset.
// Ends with a workgroup barrier.
__device__ void maintain(uint32_t* header, const Maint& m, int* s_flag) {
  const int tid = threadIdx.x;
  if (m.table != nullptr && tid < m.n_pubs) {
    const SlotPub* p = m.pubs + tid;
    const uint32_t s1 = __hip_atomic_load(&p->seq, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
    if ((s1 & 1u) == 0u) {
      const int32_t id = __hip_atomic_load(&p->id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t gen = __hip_atomic_load(&p->gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t retired = __hip_atomic_load(m.retired + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      uint64_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = agent_load64(reinterpret_cast<const uint64_t*>(&p->entry) + i);
      // The payload loads complete before the sequence is read again.
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      const uint32_t s2 = __hip_atomic_load(&p->seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // A fill whose release has been enqueued before this build is not
      // installed again, whichever landed first.
      if (s1 == s2 && id >= 0 && id < m.table_cap && gen > retired) {
        uint64_t* dst = reinterpret_cast<uint64_t*>(m.table + id);
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = w[i];
        __hip_atomic_fetch_add(&header[kHdrTableVer], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if (tid == 0) *s_flag = m.part != nullptr ? static_cast<int>(
                              __hip_atomic_load(&header[kHdrPoison], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) : 0;
  __syncthreads();
  if (*s_flag != 0) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 e = u32x4{kPartialEmpty, kPartialEmpty, kPartialEmpty, kPartialEmpty};
    u32x4* part4 = reinterpret_cast<u32x4*>(m.part);
    for (uint64_t i = tid; i < m.part_words / 4; i += blockDim.x) part4[i] = e;
    for (uint64_t i = tid; i < m.consumed_words; i += blockDim.x) m.consumed[i] = 0u;
    __syncthreads();
    if (tid == 0) __hip_atomic_store(&header[kHdrPoison], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

__global__ __launch_bounds__(256) void maintain_kernel(uint32_t* header, Maint m) {
  __shared__ int s_flag;
  maintain(header, m, &s_flag);
}

// A publication under its sequence lock: odd sequence, payload, even
// sequence, with agent-scope release fences between, so a reader that saw
// the same even value before and after its payload loads has a whole payload.
// One thread.
__device__ void publish(SlotPub* pub, int32_t id, uint32_t gen, const Entry& en) {
  const uint32_t base = __hip_atomic_load(&pub->seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & ~1u;
  __hip_atomic_store(&pub->seq, base + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __hip_atomic_store(&pub->id, id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(&pub->gen, gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    agent_store64(reinterpret_cast<uint64_t*>(&pub->entry) + i, reinterpret_cast<const uint64_t*>(&en)[i]);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __hip_atomic_store(&pub->seq, base + 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One wave; thread 0 writes.
__global__ __launch_bounds__(64) void entry_writes_kernel(EntryWrites w) {
  if (threadIdx.x != 0) return;
  if (w.pub != nullptr) publish(w.pub, w.pub_id, w.pub_gen, w.pub_entry);
  for (int i = 0; i < w.n_retire; ++i)
    __hip_atomic_fetch_max(w.retire[i], w.retire_gen[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (int i = 0; i < w.n; ++i) *w.dst[i] = w.val[i];
  if (w.header != nullptr && w.n > 0)
    __hip_atomic_fetch_add(&w.header[kHdrTableVer], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroup (job, part) copies its share of the job's A and B in 16-byte
// units; every workgroup's stores complete before it counts itself done, and
// the job's last workgroup publishes the slot.
__global__ __launch_bounds__(256) void stage_copy_kernel(StageJobs jobs) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const int j = blockIdx.x / kStageWorkgroups;
  const int part = blockIdx.x - j * kStageWorkgroups;
  const StageJob& job = jobs.job[j];
  const uint64_t stride = static_cast<uint64_t>(kStageWorkgroups) * blockDim.x;
  const uint64_t first = static_cast<uint64_t>(part) * blockDim.x + threadIdx.x;
  for (int m = 0; m < 2; ++m) {
    const u32x4* src = static_cast<const u32x4*>(m == 0 ? job.src_a : job.src_b);
    u32x4* dst = static_cast<u32x4*>(m == 0 ? job.dst_a : job.dst_b);
    const uint64_t n = (m == 0 ? job.a_bytes : job.b_bytes) / 16;
    // Four loads in flight per thread.
    uint64_t i = first;
    for (; i + 3 * stride < n; i += 4 * stride) {
      const u32x4 v0 = src[i], v1 = src[i + stride], v2 = src[i + 2 * stride], v3 = src[i + 3 * stride];
      dst[i] = v0;
      dst[i + stride] = v1;
      dst[i + 2 * stride] = v2;
      dst[i + 3 * stride] = v3;
    }
    for (; i < n; i += stride) dst[i] = src[i];
  }
  __shared__ int s_last;
  // Release: this workgroup's stores are visible device-wide before its count.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t done = __hip_atomic_fetch_add(&job.pub->copies, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    s_last = done == kStageWorkgroups - 1 ? 1 : 0;
  }
  __syncthreads();
  if (s_last != 0 && threadIdx.x == 0) {
    __hip_atomic_store(&job.pub->copies, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    publish(job.pub, job.pub_id, job.pub_gen, job.pub_entry);
  }
}

// Runs sorted by counting (below) when there are at most kRankMax of them and
// the waves' broadcast reads (keys x keys per thread x waves) stay within
// kRankWork; past that, a bitonic sort.  Measured on MI355X: 256-token plans
// 15.8 -> 12.7 us per build_seg_bounds; at 1024 threads the waves' reads
// queue on the CU's LDS (2048 Zipf-routed tokens: 42 us bitonic, 96 us by
// counting).
constexpr int kRankMax = 1024;
constexpr int kRankWork = 4096;

// plan_kernel's explicit arguments, as laid out in its kernel-argument
// segment: touch_kernel_args reads below this size only.
struct PlanKernelArgs {
  const void* idx;
  int idx_is_int64, T;
  uint32_t* header;
  Segment* segments;
  Block* blocks;
  int32_t* perm;
  int32_t* bperm;
  Entry* bentries;
  int seg_cap, block_cap, bt;
  Maint m;
};
static_assert(offsetof(PlanKernelArgs, m) == 80 && sizeof(PlanKernelArgs) == 80 + sizeof(Maint),
              "plan_kernel's argument size as passed to touch_kernel_args");

template <int NT, int E>
__global__ __launch_bounds__(NT) void plan_kernel(const void* __restrict__ idx, int idx_is_int64, int T,
                                                  uint32_t* __restrict__ header, Segment* __restrict__ segments,
                                                  Block* __restrict__ blocks, int32_t* __restrict__ perm,
                                                  int32_t* __restrict__ bperm, Entry* __restrict__ bentries,
                                                  int seg_cap, int block_cap, int bt, Maint m) {
  touch_kernel_args<static_cast<int>(sizeof(PlanKernelArgs))>();
  constexpr int CAP = NT * E;
  // s_big: the ids (int64) first, then the sort keys, then per-run offsets.
  __shared__ unsigned long long s_big[CAP];
  __shared__ int s_a[CAP + 1];  // run starts, later group adapter ids
  __shared__ int s_b[CAP + 1];  // per-run segment bases, later group offsets
  __shared__ int s_scan[NT / 64];
  __shared__ unsigned long long s_sorted[kRankMax];  // sorted keys (counting path)
  long long* s_id = reinterpret_cast<long long*>(s_big);

  const int tid = threadIdx.x;
  const int e0 = tid * E;
  plan_stamp(m, 0);

  // 1. ids, loaded first so that their latency overlaps the maintenance's
  //    (the routing does not depend on the adapter table).
  long long ids[E];
#pragma unroll
  for (int k = 0; k < E; ++k) {
    const int i = tid + k * NT;
    ids[k] = 0;
    if (i < T)
      ids[k] = idx_is_int64 ? static_cast<const long long*>(idx)[i]
                            : static_cast<long long>(static_cast<const int*>(idx)[i]);
  }

  // 0. Publications into the adapter table; the partial buffer's repair.
  maintain(header, m, s_scan);
  // The table version the block entry copies below are taken at (every
  // install above has raised it before maintain's closing barrier).
  // A build without copies records a version that no table write produces
  // (the complement of the current one), so copies left by an earlier build
  // can never pass for current ones.
  const uint32_t table_ver =
      tid == 0 ? __hip_atomic_load(&header[kHdrTableVer], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;

  // ids -> LDS.
#pragma unroll
  for (int k = 0; k < E; ++k) s_id[tid + k * NT] = ids[k];
  lds_barrier();
  plan_stamp(m, 1);

  // 2. Run starts in token order (reference :484): s_a[r] = first token of run r.
  bool is_start[E];
  int nstart = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = e0 + e;
    is_start[e] = i < T && (i == 0 || s_id[i - 1] != s_id[i]);
    nstart += is_start[e] ? 1 : 0;
  }
  int n_runs = 0;
  int rb = block_exclusive_scan<NT>(nstart, s_scan, &n_runs);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    if (is_start[e]) s_a[rb++] = e0 + e;
  }
  if (tid == 0) s_a[n_runs] = T;
  lds_barrier();
  plan_stamp(m, 2);

  // 3. Exported table.  Pieces per run: ceil(len/32) when id >= 0 (reference
  //    :485-489); slot bases by exclusive scan in token-start order (:494-503).
  int pieces[E];
  int psum = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int r = e0 + e;
    pieces[e] = 0;
    if (r < n_runs) {
      const int st = s_a[r];
      if (s_id[st] >= 0) pieces[e] = (s_a[r + 1] - st + kMaxSegmentTokens - 1) / kMaxSegmentTokens;
    }
    psum += pieces[e];
  }
  int n_segs = 0;
  int sb = block_exclusive_scan<NT>(psum, s_scan, &n_segs);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int r = e0 + e;
    if (r < n_runs) s_b[r] = sb;
    sb += pieces[e];
  }
  if (tid == 0) s_b[n_runs] = n_segs;
  lds_barrier();
  const int seg_out = n_segs < seg_cap ? n_segs : seg_cap;
  for (int q = tid; q < seg_out; q += NT) {
    const int r = upper_index(s_b, n_runs, q);
    const int st = s_a[r];
    const int len = s_a[r + 1] - st;
    const int p = q - s_b[r];
    const int rem = len - p * kMaxSegmentTokens;
    Segment s;
    s.adapter_id = static_cast<int>(s_id[st]);
    s.token_start = st + p * kMaxSegmentTokens;
    s.token_count = rem < kMaxSegmentTokens ? rem : kMaxSegmentTokens;
    s.pad = 0;
    segments[q] = s;
  }
  plan_stamp(m, 3);

  // 4. Sort the runs with id >= 0 by (adapter id, run index).
  unsigned long long key[E];
  int nvalid = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int r = e0 + e;
    key[e] = ~0ull;
    if (r < n_runs) {
      const long long id = s_id[s_a[r]];
      if (id >= 0) {
        key[e] = (static_cast<unsigned long long>(static_cast<unsigned>(static_cast<int>(id))) << 32) |
                 static_cast<unsigned>(r);
        ++nvalid;
      }
    }
  }
  int n_vruns = 0;
  int vb = block_exclusive_scan<NT>(nvalid, s_scan, &n_vruns);  // ends every read of s_id
#pragma unroll
  for (int e = 0; e < E; ++e) {
    if (key[e] != ~0ull) s_big[vb++] = key[e];
  }
  const unsigned long long* skey = s_big;  // the sorted keys
  if (n_vruns <= kRankMax && n_vruns * E * (NT / 64) <= kRankWork) {
    // Keys are distinct (the run index is in them): a key's position is
    // the number of keys below it.  Every lane reads the same key at once
    // (an LDS broadcast), with no barrier per step, unlike a bitonic sort's
    // log^2 rounds (7 of the 16 us of a 256-token plan).
    lds_barrier();
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if (key[e] == ~0ull) continue;
      int below = 0;
#pragma unroll 8
      for (int i = 0; i < n_vruns; ++i) below += s_big[i] < key[e] ? 1 : 0;
      s_sorted[below] = key[e];
    }
    lds_barrier();
    skey = s_sorted;
  } else {
    int P = 1;
    while (P < n_vruns) P <<= 1;
    for (int i = n_vruns + tid; i < P; i += NT) s_big[i] = ~0ull;
    lds_barrier();
    for (int k = 2; k <= P; k <<= 1) {
      for (int j = k >> 1; j > 0; j >>= 1) {
        for (int i = tid; i < P; i += NT) {
          const int ixj = i ^ j;
          if (ixj > i) {
            const unsigned long long a = s_big[i];
            const unsigned long long b = s_big[ixj];
            const bool ascending = (i & k) == 0;
            if ((a > b) == ascending) {
              s_big[i] = b;
              s_big[ixj] = a;
            }
          }
        }
        lds_barrier();
      }
    }
  }

  plan_stamp(m, 4);
  // 5. perm: the tokens of the sorted runs, concatenated.
  int len_e[E];
  int start_e[E];
  int gid_e[E];
  bool gstart[E];
  int lsum = 0;
  int gcount = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int p = e0 + e;
    len_e[e] = 0;
    start_e[e] = 0;
    gid_e[e] = 0;
    gstart[e] = false;
    if (p < n_vruns) {
      const unsigned long long kk = skey[p];
      const int r = static_cast<int>(kk & 0xffffffffull);
      start_e[e] = s_a[r];
      len_e[e] = s_a[r + 1] - s_a[r];
      gid_e[e] = static_cast<int>(kk >> 32);
      gstart[e] = p == 0 || (skey[p - 1] >> 32) != (kk >> 32);
    }
    lsum += len_e[e];
    gcount += gstart[e] ? 1 : 0;
  }
  int n_tok = 0;
  int ob = block_exclusive_scan<NT>(lsum, s_scan, &n_tok);  // ends every read of s_big keys and s_a
  int off_e[E];
  int* s_roff = reinterpret_cast<int*>(s_big);           // [CAP] run offsets into perm
  int* s_rstart = reinterpret_cast<int*>(s_big) + CAP;   // [CAP] run first tokens
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int p = e0 + e;
    off_e[e] = ob;
    if (p < n_vruns) {
      s_roff[p] = ob;
      s_rstart[p] = start_e[e];
    }
    ob += len_e[e];
  }
  lds_barrier();
  // perm[q] for q = tid + e*NT, kept in registers until the run tables are
  // free, then in LDS for the block lists below.
  int pv[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int q = tid + e * NT;
    pv[e] = 0;
    if (q < n_tok) {
      const int p = upper_index(s_roff, n_vruns, q);
      pv[e] = s_rstart[p] + (q - s_roff[p]);
      perm[q] = pv[e];
    }
  }

  plan_stamp(m, 5);
  // 6. Groups (one per adapter) and their blocks of bt tokens.
  int n_groups = 0;
  int gb = block_exclusive_scan<NT>(gcount, s_scan, &n_groups);  // ends every read of s_roff / s_rstart
  int* s_perm = reinterpret_cast<int*>(s_big) + CAP;             // [CAP] perm (over s_rstart)
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int q = tid + e * NT;
    if (q < n_tok) s_perm[q] = pv[e];
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    if (gstart[e]) {
      s_b[gb] = off_e[e];
      s_a[gb] = gid_e[e];
      ++gb;
    }
  }
  if (tid == 0) s_b[n_groups] = n_tok;
  lds_barrier();
  int nb[E];
  int bsum = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int g = e0 + e;
    nb[e] = g < n_groups ? (s_b[g + 1] - s_b[g] + bt - 1) / bt : 0;
    bsum += nb[e];
  }
  int n_blocks = 0;
  int bb = block_exclusive_scan<NT>(bsum, s_scan, &n_blocks);
  int* s_bbase = reinterpret_cast<int*>(s_big);  // [CAP] first block of each group
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int g = e0 + e;
    if (g < n_groups) s_bbase[g] = bb;
    bb += nb[e];
  }
  lds_barrier();
  const int blk_out = n_blocks < block_cap ? n_blocks : block_cap;
  for (int q = tid; q < blk_out; q += NT) {
    const int g = upper_index(s_bbase, n_groups, q);
    const int j = q - s_bbase[g];
    const int n = s_b[g + 1] - s_b[g];
    Block b;
    b.adapter_id = s_a[g];
    b.first = s_b[g] + j * bt;
    b.count = n - j * bt < bt ? n - j * bt : bt;
    b.entry = s_a[g];
    blocks[q] = b;
    if (bentries != nullptr) {
      // The block's adapter-table entry (agent-scope loads: the maintenance
      // above may have installed it from another wave), or an empty one.
      uint64_t w[4] = {0, 0, 0, 0};
      if (m.table != nullptr && b.entry >= 0 && b.entry < m.table_cap) {
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = agent_load64(reinterpret_cast<const uint64_t*>(m.table + b.entry) + i);
      }
      uint64_t* dst = reinterpret_cast<uint64_t*>(bentries + q);
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[i] = w[i];
    }
  }
  plan_stamp(m, 6);
  // Block-padded token lists, from the LDS copy of perm.
  for (int u = tid; u < blk_out * bt; u += NT) {
    const int q = u / bt;
    const int j = u - q * bt;
    const int g = upper_index(s_bbase, n_groups, q);
    const int n = s_b[g + 1] - s_b[g];
    const int jj = (q - s_bbase[g]) * bt + j;  // position inside the group
    if (jj < n) bperm[static_cast<int64_t>(q) * kBlockTokens + j] = s_perm[s_b[g] + jj];
  }

  if (tid == 0) {
    header[kHdrNumSegments] = static_cast<uint32_t>(n_segs);
    header[kHdrNumBlocks] = static_cast<uint32_t>(blk_out);
    header[kHdrNumGroups] = static_cast<uint32_t>(n_groups);
    header[kHdrNumValid] = static_cast<uint32_t>(n_tok);
    header[kHdrT] = static_cast<uint32_t>(T);
    header[kHdrBlockTokens] = static_cast<uint32_t>(bt);
    header[kHdrPlanVer] = bentries != nullptr ? table_ver : ~table_ver;
  }
  plan_stamp(m, 7);
}

}  // namespace

// Host launcher: the smallest capacity variant that holds T.
hipError_t launch_plan(const void* idx, int idx_is_int64, int T, uint32_t* header, Segment* segments, Block* blocks,
                       int32_t* perm, int32_t* bperm, Entry* bentries, int seg_cap, int block_cap, int bt,
                       const Maint* m, hipStream_t stream) {
  if (T < 0 || bt < 1 || bt > kBlockTokens) return hipErrorInvalidValue;
  Maint mm{};
  if (m != nullptr) mm = *m;
  // Publications are applied by threads 0..n_pubs-1 of the smallest variant.
  if (mm.n_pubs < 0 || mm.n_pubs > 256) return hipErrorInvalidValue;
  if (T <= 256) {
    plan_kernel<256, 1><<<1, 256, 0, stream>>>(idx, idx_is_int64, T, header, segments, blocks, perm, bperm,
                                               bentries, seg_cap, block_cap, bt, mm);
  } else if (T <= 2048) {
    plan_kernel<1024, 2><<<1, 1024, 0, stream>>>(idx, idx_is_int64, T, header, segments, blocks, perm, bperm,
                                                 bentries, seg_cap, block_cap, bt, mm);
  } else if (T <= kPlanMaxTokens) {
    plan_kernel<1024, 8><<<1, 1024, 0, stream>>>(idx, idx_is_int64, T, header, segments, blocks, perm, bperm,
                                                 bentries, seg_cap, block_cap, bt, mm);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_maintain(uint32_t* header, const Maint& m, hipStream_t stream) {
  if (m.n_pubs < 0 || m.n_pubs > 256) return hipErrorInvalidValue;
  maintain_kernel<<<1, 256, 0, stream>>>(header, m);
  return hipGetLastError();
}

hipError_t launch_entry_writes(const EntryWrites& w, hipStream_t stream) {
  if (w.n < 0 || w.n > kMaxEntryWrites || w.n_retire < 0 || w.n_retire > kMaxEntryWrites) return hipErrorInvalidValue;
  entry_writes_kernel<<<1, 64, 0, stream>>>(w);
  return hipGetLastError();
}

hipError_t launch_stage_copies(const StageJobs& jobs, hipStream_t stream) {
  if (jobs.n < 0 || jobs.n > kMaxStageJobs) return hipErrorInvalidValue;
  for (int j = 0; j < jobs.n; ++j)
    if (jobs.job[j].pub == nullptr || jobs.job[j].a_bytes % 16 != 0 || jobs.job[j].b_bytes % 16 != 0)
      return hipErrorInvalidValue;
  if (jobs.n == 0) return hipSuccess;
  stage_copy_kernel<<<jobs.n * kStageWorkgroups, 256, 0, stream>>>(jobs);
  return hipGetLastError();
}

}  // namespace wp
