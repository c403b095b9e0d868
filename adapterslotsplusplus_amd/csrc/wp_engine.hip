// wp_engine.hip -- host side of the C ABI declared in include/warppipe_mi355x.h.
//
// Replaces the reference's pybind11 WarpPipeExtension (csrc/pybind/warp_pipe_bindings.cpp),
// AdapterStore (csrc/memory/adapter_store.h), StagingBufferPool
// (csrc/memory/staging_buffer.h), build_segment_table (csrc/dispatch/segment_builder.cpp)
// and the rank dispatcher (csrc/dispatch/warp_pipe_dispatcher.cpp).
//
// Design points that differ from the reference, each fixing a behaviour it
// documents as a defect or limit:
//   * The segment table and the by-adapter plan live in HBM, written by the
//     plan kernel or by a stream-ordered upload from pinned memory (the
//     reference writes mapped host memory from the CPU, unordered with in-flight
//     kernels, and every kernel block reads it over PCIe).
//   * Registered weights are copied into engine-owned memory from a stream-ordered
//     pool (hipMallocFromPoolAsync / hipFreeAsync), so eviction can never free
//     memory a queued kernel still reads.  Cold adapters live in a pinned host
//     store and become usable through prefetch (H2D on the prefetch stream).
//   * Staging slots are sized per adapter (the reference's fixed 512 KiB slots
//     overflow for rank 64 x 13824), eviction releases the id's slot, and a slot
//     is never overwritten before the kernels that read it have finished.
//   * Every scratch buffer (fp32 partials, counters, plan arrays) is
//     allocated at engine creation, so calls allocate nothing and graph
//     replays keep valid pointers.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/warppipe_mi355x.h"
#include "wp_apply.h"

using namespace wp;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

#define WP_HIP(expr)                                                                           \
  do {                                                                                         \
    const hipError_t wp_e_ = (expr);                                                           \
    if (wp_e_ != hipSuccess) return fail(WP_ERR_HIP, "%s: %s", #expr, hipGetErrorString(wp_e_)); \
  } while (0)

struct DeviceGuard {
  int prev = -1;
  bool changed = false;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) == hipSuccess && prev != dev) {
      changed = hipSetDevice(dev) == hipSuccess;
    }
  }
  ~DeviceGuard() {
    if (changed) (void)hipSetDevice(prev);
  }
};

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline bool aligned(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }
inline bool rank_ok(int r) { return r == 8 || r == 16 || r == 32 || r == 64; }

struct Adapter {
  int32_t rank = 0, d = 0, o = 0, dtype = 0;
  float alpha = 0.f;
  void* dA = nullptr;    // device copies (pool)
  void* dB = nullptr;
  void* host = nullptr;  // host-resident adapters: one pinned allocation, A then B
  void* hA = nullptr;    // ... and its A and B as the device addresses them
  void* hB = nullptr;
  size_t a_bytes = 0, b_bytes = 0;
  hipEvent_t copied = nullptr;  // recorded after the registration copy
  bool borrowed = false;        // dA/dB are the caller's (registered by reference): never freed here
};

// A staging slot.  Kernels reach its buffers only through the adapter table:
// once the copy has landed, the prefetch stream publishes the slot's entry
// (SlotPub); the next plan build -- or an eager call that finds the slot ready
// -- writes it into the table; a release writes the adapter's registered
// entry back on the caller's stream and hands the buffers to the engine's
// free list behind an event recorded there.  A prefetch takes a free buffer
// whose event has completed (a host query) or a new one from the pool, so a
// copy never waits for the caller's stream: that wait -- a side stream
// waiting on an event of the stream that replays the step -- measured ~70 us
// per step on MI355X, and a stream-ordered free ~170 us of host time.
struct Slot {
  int32_t adapter = -1;
  void* A = nullptr;
  void* B = nullptr;
  size_t a_bytes = 0, b_bytes = 0;  // sizes of A and B
  hipEvent_t ready = nullptr;     // prefetch stream: copy and publication done
  uint32_t gen = 0;               // generation of the slot's current (or last) fill
  bool issued = false;
  bool applied = false;           // an eager call has enqueued the table write of the publication
};

// Expand workgroups per block a fused call aims for.
constexpr int kExpandWorkgroups = 16;

// Shrink split of a fused call with `rows`-row rank groups: the groups, then
// shrink_workgroups(rows) / groups d-ranges (at least 8), each a multiple of
// 128 (four waves x 32).  Workgroup ids map to the 8 XCDs round-robin, so
// with a multiple of 8 d-ranges every rank group of one d-range runs on the
// same XCD and its X rows are fetched once into that XCD's L2.  The count is
// then halved (down to 4) while
//   - a wave's share of a d-range is under one full batch of K-steps
//     (4 x 32 columns: fewer columns leave loads of the batch unused), or
//   - the grid (block bound x (shrink + expand workgroups)) exceeds the
//     workgroups the device holds at the kernel's occupancy (`resident`,
//     0 to skip this test): workgroups that start late issue their loads
//     during the partials exchange.
// Measured on MI355X: cfg2 o_proj 14.3 -> 14.1 us, cfg5 step 836 -> 797 us,
// cfg1 9.2 -> 8.8 us.  Multi-slice calls skip the residency test: their grid
// does not fit at either count, and the halved one only adds a load round
// (qkv 20.6 -> 20.8 us).  It is also halved while the d-ranges' partial rows
// (nc x hs fp32 per plan position, hs = the A slices' H columns side by side)
// exceed the partial buffer's kMaxChunks x kMaxRank; four d-ranges of four
// 64-column slices fill it exactly.
inline void shrink_split(int d, int rank, int rows, int n_a, int hs, int64_t slots, int64_t expand_per_block,
                         int64_t resident, ApplyArgs* a) {
  const int g = shrink_rank_groups(rank, rows);
  int nc = static_cast<int>(std::min<int64_t>(std::max(8, shrink_workgroups(rows) / g), ceil_div(d, 128)));
  while (nc > 4 && (d < nc * 512 || nc * hs > kMaxChunks * kMaxRank ||
                    (resident > 0 && slots * (nc * g * n_a + expand_per_block) > resident)))
    nc /= 2;
  const int c = static_cast<int>(ceil_div(ceil_div(d, nc), 128) * 128);
  a->dc = c;
  a->n_chunks = static_cast<int>(ceil_div(d, c));
  a->srows = rows;
  a->n_rgroups = g;
}

// Split of a decode-sized shrink() launch: 32-row rank groups x d-ranges of
// about 512 columns (each wave's share one batch of loads), or 1024 columns
// past eight ranges (fewer workgroups than residency rounds; measured on
// MI355X at d = 13824, and at d = 5120: cfg3 gate/up 42.8 -> 42.2 us per
// call), at most kMaxChunks; one reducer workgroup per block.
inline void shrink_small_split(int d, int rank, ApplyArgs* a) {
  int64_t n = std::max<int64_t>(ceil_div(d, 512), 1);
  if (n > 8) n = std::min<int64_t>(ceil_div(d, 1024), kMaxChunks);
  a->dc = static_cast<int>(ceil_div(ceil_div(d, n), 128) * 128);
  a->n_chunks = static_cast<int>(ceil_div(d, a->dc));
  a->srows = kShrinkRowsFused;
  a->n_rgroups = shrink_rank_groups(rank, kShrinkRowsFused);
  a->n_ochunks = 1;
  a->n_sub = 1;
}

// d-ranges of a shrink() launch: one workgroup per block and d-range, every
// rank row; a d-range is kShrinkSlices x 128 columns (a multiple of that
// past kMaxChunks ranges).
inline void shrink_range_split(int d, ApplyArgs* a) {
  const int group = kShrinkSlices * 128;
  const int64_t n = std::min<int64_t>(ceil_div(d, group), kMaxChunks);
  a->dc = static_cast<int>(ceil_div(ceil_div(d, n), group) * group);
  a->n_chunks = static_cast<int>(ceil_div(d, a->dc));
  a->srows = 0;
  a->n_rgroups = 1;
}

}  // namespace

// Pinned upload buffers of host-built plans, used in turn: a plan upload
// waits (on the host) only for the one issued kUploadRing builds before it.
constexpr int kUploadRing = 4;
// Adapter-table size when the configuration gives none.
constexpr int32_t kDefaultTableIds = 1 << 16;
constexpr int32_t kMaxTableIds = 1 << 22;
// Column-tile counters of linear_lora: (token groups x output columns / 16)
// of one call at most.
constexpr int kLinCounters = 1 << 16;
// Staging slots an engine may have (publications are applied by one thread each).
constexpr int kMaxStagingSlots = 256;

struct wp_engine {
  int device = 0;
  wp_config cfg{};
  hipStream_t pstream = nullptr;
  hipMemPool_t pool = nullptr;
  std::unordered_map<int32_t, Adapter> adapters;
  std::vector<Slot> slots;
  // Pinned host copies of evicted adapters, freed once the prefetch stream
  // has passed the recorded event (a copy may still read them).
  std::vector<std::pair<void*, hipEvent_t>> host_graveyard;
  // Released slot buffers: reusable once `after` (recorded on the releasing
  // stream behind the release) has completed.  Events are shared by the
  // buffers of one release batch (event_refs) and recycled.
  struct FreeBuf {
    void* ptr;
    size_t bytes;
    hipEvent_t after;
  };
  std::vector<FreeBuf> free_bufs;
  std::vector<hipEvent_t> spare_events;
  std::unordered_map<hipEvent_t, int> event_refs;

  // Workspace (one allocation).
  char* ws = nullptr;
  uint32_t* header = nullptr;
  Segment* segs = nullptr;
  Block* blocks = nullptr;
  int32_t* perm = nullptr;
  int32_t* bperm = nullptr;     // [block_cap][kBlockTokens]
  uint32_t* consumed = nullptr; // [block_cap][kCounterStride]
  Entry* plan_entries = nullptr;
  float* part = nullptr;        // [kMaxChunks][ptok][kMaxRank] fp32 partial H of fused calls (kPartialEmpty between calls)
  float* spart = nullptr;       // [kMaxChunks][tok_cap][kMaxRank] d-range partials of shrink() launches (no invariant)
  void* hbuf = nullptr;         // [tok_cap][kMaxSlices x kMaxRank] 2-byte H of large-plan add_lora calls
  SlotPub* pubs = nullptr;      // [num_staging_slots] staging publications
  uint32_t* retired = nullptr;  // [num_staging_slots] highest released generation per slot
  uint32_t* lin_cnt = nullptr;  // [kLinCounters] column-tile counters of linear_lora (zero between calls)
  uint32_t* lin_flag = nullptr; // [2][block_cap] H flags and their reader counts (zero between calls)
  Entry* dtable = nullptr;      // [table_cap] id-indexed adapter table of build_seg_bounds plans
  Entry* bentries = nullptr;    // [block_cap] a build_seg_bounds plan's copy of each block's table entry
  bool plan_bentries = false;   // the last build_seg_bounds plan wrote bentries
  int table_cap = 0;
  int seg_cap = 0, block_cap = 0, tok_cap = 0, entry_cap = 0;
  int ptok = 0;                 // plan positions of `part`: fused calls run on plans of <= kSmallPlanTokens
  uint64_t part_words = 0, consumed_words = 0;
  int n_cu = 256;  // compute units of the device
  int32_t entry_offset = 0;  // table-mode calls on device-built plans read dtable + entry_offset
  int32_t entry_count = 0;   // ... and at most this many entries (0: to the table's end)
  int64_t max_adapters = 0;  // declared most registered adapters (wp_set_max_adapters), 0: none declared
  // wp_poll_device_errors: the error word is moved (and cleared) by a kernel
  // into a pinned, device-mapped host word; `err_ready` is recorded behind
  // it, and the host reads the word once the event has completed.
  uint32_t* err_host = nullptr;   // host address
  uint32_t* err_hdev = nullptr;   // its device address
  hipEvent_t err_ready = nullptr;
  bool err_pending = false;
  uint32_t spin_limit = kDefaultSpinLimit;
  uint64_t* trace = nullptr;  // traced builds: per-workgroup timestamps of fused launches
  int64_t trace_words = 0;

  char* pinned[kUploadRing] = {};
  hipEvent_t upload_done[kUploadRing] = {};
  bool upload_pending[kUploadRing] = {};
  int upload_next = 0;
  size_t pinned_bytes = 0;

  // Host view of the current plan.
  int plan_kind = 0;          // 0 none, 1 host-built (build_segments), 2 device-built (build_seg_bounds)
  int64_t plan_T = 0;         // device: T of build_seg_bounds; host: max token end
  int plan_bt = kBlockTokens; // most tokens per block of the current plan
  int plan_blocks = 0;        // host: exact block count
  int plan_valid = 0;         // host: exact token count in perm
  std::vector<int32_t> plan_entry_ids;  // host: adapter id per entry
  std::vector<int> plan_entry_slot;     // host: staging slot read by the entry, or -1
};

namespace {

int find_slot(const wp_engine* e, int32_t id) {
  for (size_t i = 0; i < e->slots.size(); ++i)
    if (e->slots[i].adapter == id) return static_cast<int>(i);
  return -1;
}

bool slot_ready(const Slot& s) { return s.adapter >= 0 && s.issued && hipEventQuery(s.ready) == hipSuccess; }

bool stream_capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess) return false;
  return st != hipStreamCaptureStatusNone;
}

// The adapter's table entry as registered: its device copies, or no weights
// (a host-resident adapter is usable only through a staging slot).
Entry registered_entry(const Adapter& ad) {
  Entry en{};
  en.a_ptr = reinterpret_cast<uint64_t>(ad.dA);
  en.b_ptr = reinterpret_cast<uint64_t>(ad.dB);
  en.alpha = ad.alpha;
  en.rank_dtype = pack_rank_dtype(ad.rank, ad.dtype);
  en.d_model = ad.d;
  en.out_features = ad.o;
  return en;
}

Entry staged_entry(const Adapter& ad, const Slot& sl) {
  Entry en = registered_entry(ad);
  en.a_ptr = reinterpret_cast<uint64_t>(sl.A);
  en.b_ptr = reinterpret_cast<uint64_t>(sl.B);
  return en;
}

// Entry of a host-built plan: the staged copy once its slot is ready, else
// the registered one.
Entry entry_for(const wp_engine* e, int32_t id, const Adapter& ad, int* slot_used) {
  *slot_used = -1;
  const int s = find_slot(e, id);
  if (s >= 0 && slot_ready(e->slots[s])) {
    *slot_used = s;
    return staged_entry(ad, e->slots[s]);
  }
  return registered_entry(ad);
}

Maint maint_view(const wp_engine* e) {
  Maint m{};
  m.part = e->part;
  m.part_words = e->part_words;
  m.consumed = e->consumed;
  m.consumed_words = e->consumed_words;
  m.pubs = e->pubs;
  m.retired = e->retired;
  m.n_pubs = static_cast<int32_t>(e->slots.size());
  m.table_cap = e->table_cap;
  m.table = e->dtable;
  return m;
}

// Table entry `id` = en, in stream order (ids outside the table are reached
// through build_segments tables only).
int table_write(wp_engine* e, int32_t id, const Entry& en, hipStream_t stream) {
  if (id < 0 || id >= e->table_cap) return WP_OK;
  EntryWrites w{};
  w.header = e->header;
  w.n = 1;
  w.dst[0] = e->dtable + id;
  w.val[0] = en;
  WP_HIP(launch_entry_writes(w, stream));
  return WP_OK;
}

// Eager calls on a build_seg_bounds plan: a slot whose copy has landed since
// the plan was built is written into the table before the call (the plan
// build writes every ready publication, so captured steps need no such launch).
int apply_ready_slots(wp_engine* e, hipStream_t stream) {
  bool any = false;
  for (auto& sl : e->slots)
    if (sl.issued && !sl.applied && hipEventQuery(sl.ready) == hipSuccess) {
      sl.applied = true;
      any = true;
    }
  if (any) WP_HIP(launch_maintain(e->header, maint_view(e), stream));
  return WP_OK;
}

void sweep_graveyard(wp_engine* e, bool wait) {
  for (size_t i = 0; i < e->host_graveyard.size();) {
    auto& g = e->host_graveyard[i];
    if (wait || hipEventQuery(g.second) == hipSuccess) {
      if (wait) (void)hipEventSynchronize(g.second);
      (void)hipHostFree(g.first);
      (void)hipEventDestroy(g.second);
      g = e->host_graveyard.back();
      e->host_graveyard.pop_back();
    } else {
      ++i;
    }
  }
}

void invalidate_host_plan_for(wp_engine* e, int32_t id) {
  if (e->plan_kind != 1) return;
  for (int32_t pid : e->plan_entry_ids)
    if (pid == id) {
      e->plan_kind = 0;
      return;
    }
}

// Frees slots, on `stream`: the fill's generation is retired (no plan build
// after this installs its publication, whether the copy lands before or
// after) and the adapter's registered entry written back into the table and
// into the current host-built plan, so kernels enqueued after this never
// read the slot; its buffers go to the free list behind an event recorded
// after these writes.  Kernels enqueued before it on `stream` (graph replays
// included) finish first.  The slot index is free again at once: its next
// fill publishes a higher generation.  One entry-write launch for up to
// kMaxEntryWrites / 2 slots.
int release_slots_on(wp_engine* e, const int* slot_ids, int n, hipStream_t stream) {
  int done = 0;
  while (done < n) {
    EntryWrites w{};
    w.header = e->header;
    std::vector<int> batch;
    for (; done < n && w.n + 2 <= kMaxEntryWrites; ++done) {
      const int s = slot_ids[done];
      if (s < 0 || e->slots[s].adapter < 0) continue;
      Slot& sl = e->slots[s];
      // The fill's generation is retired in this stream's order; its
      // publication may land before or after (the copy is not waited for),
      // and a later fill of the slot publishes a higher generation.
      w.retire[w.n_retire] = e->retired + s;
      w.retire_gen[w.n_retire++] = sl.gen;
      Entry reg{};
      auto it = e->adapters.find(sl.adapter);
      if (it != e->adapters.end()) reg = registered_entry(it->second);
      if (sl.adapter < e->table_cap) {
        w.dst[w.n] = e->dtable + sl.adapter;
        w.val[w.n++] = reg;
      }
      if (e->plan_kind == 1)
        for (size_t k = 0; k < e->plan_entry_slot.size(); ++k)
          if (e->plan_entry_slot[k] == s) {
            // A slot holds one adapter, which a host-built plan lists once.
            w.dst[w.n] = e->plan_entries + k;
            w.val[w.n++] = reg;
            e->plan_entry_slot[k] = -1;
          }
      sl.adapter = -1;
      sl.issued = false;
      sl.applied = false;
      batch.push_back(s);
    }
    if (batch.empty()) continue;
    WP_HIP(launch_entry_writes(w, stream));
    // The batch's buffers go to the free list behind one event.
    hipEvent_t ev = nullptr;
    if (!e->spare_events.empty()) {
      ev = e->spare_events.back();
      e->spare_events.pop_back();
    } else {
      WP_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    }
    WP_HIP(hipEventRecord(ev, stream));
    int refs = 0;
    for (int s : batch) {
      Slot& sl = e->slots[s];
      if (sl.A) e->free_bufs.push_back({sl.A, sl.a_bytes, ev}), ++refs;
      if (sl.B) e->free_bufs.push_back({sl.B, sl.b_bytes, ev}), ++refs;
      sl.A = sl.B = nullptr;
    }
    if (refs > 0) e->event_refs[ev] = refs;
    else e->spare_events.push_back(ev);
  }
  return WP_OK;
}

int release_slot_on(wp_engine* e, int s, hipStream_t stream) { return release_slots_on(e, &s, 1, stream); }

// A slot buffer of at least `bytes`: the smallest free one whose release has
// completed, else a new pool allocation on the prefetch stream.
int take_slot_buffer(wp_engine* e, size_t bytes, void** out) {
  int best = -1;
  for (size_t i = 0; i < e->free_bufs.size(); ++i) {
    const auto& f = e->free_bufs[i];
    if (f.bytes < bytes || (best >= 0 && f.bytes >= e->free_bufs[best].bytes)) continue;
    if (hipEventQuery(f.after) != hipSuccess) continue;
    best = static_cast<int>(i);
  }
  if (best < 0) {
    WP_HIP(hipMallocFromPoolAsync(out, bytes, e->pool, e->pstream));
    return WP_OK;
  }
  *out = e->free_bufs[best].ptr;
  hipEvent_t ev = e->free_bufs[best].after;
  e->free_bufs[best] = e->free_bufs.back();
  e->free_bufs.pop_back();
  if (--e->event_refs[ev] == 0) {
    e->event_refs.erase(ev);
    e->spare_events.push_back(ev);
  }
  return WP_OK;
}

int evict_impl(wp_engine* e, int32_t id, hipStream_t stream) {
  auto it = e->adapters.find(id);
  if (it == e->adapters.end()) return WP_OK;
  int rc = release_slot_on(e, find_slot(e, id), stream);
  if (rc != WP_OK) return rc;
  Adapter& ad = it->second;
  // Kernels enqueued from here on find no weights for the id; those enqueued
  // before finish before the stream-ordered frees.
  if ((rc = table_write(e, id, Entry{}, stream)) != WP_OK) return rc;
  if (ad.dA && !ad.borrowed) WP_HIP(hipFreeAsync(ad.dA, stream));
  if (ad.dB && !ad.borrowed) WP_HIP(hipFreeAsync(ad.dB, stream));
  if (ad.host) {
    hipEvent_t ev = nullptr;
    WP_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    WP_HIP(hipEventRecord(ev, e->pstream));
    e->host_graveyard.emplace_back(ad.host, ev);
  }
  if (ad.copied) WP_HIP(hipEventDestroy(ad.copied));
  e->adapters.erase(it);
  invalidate_host_plan_for(e, id);
  sweep_graveyard(e, false);
  return WP_OK;
}

PlanView plan_view(const wp_engine* e) {
  PlanView v;
  v.header = e->header;
  v.segments = e->segs;
  v.blocks = e->blocks;
  v.perm = e->perm;
  v.bperm = e->bperm;
  return v;
}

// Fields every apply launch shares.
ApplyArgs base_args(const wp_engine* e, int rank) {
  ApplyArgs a{};
  a.rank = rank;
  a.n_sub = 1;
  a.tiles = (e->plan_bt + 15) / 16;
  a.hs = rank == 0 ? kMaxRank : rank;
  a.hs1 = a.hs;
  a.w.n_a = 1;
  a.ptok = e->ptok;
  a.part = e->part;
  a.consumed = e->consumed;
  a.spin_limit = e->spin_limit;
  a.trace = e->trace;
  a.trace_words = e->trace_words;
  a.plan = plan_view(e);
  return a;
}

// Upper bound on the block count of the current plan, given at most `groups`
// distinct adapters: sum_g ceil(n_g / TB) <= floor(T / TB) + G, and <= T.
// shrink() / expand() on a device-built plan pass the number of registered
// adapters: a routing that only names registered adapters stays within the
// bound, and the kernels flag kErrCapacity when it does not (ids that are
// not registered sort among the others and can push blocks past it).
// Bounding by T alone would launch mostly empty workgroups on large plans
// (8192 tokens: 8192 slots x 48 chunks for 144 real blocks, ~150 us of
// dispatch), and a loop over items in the kernels costs their registers.
int block_bound(const wp_engine* e, int64_t groups) {
  if (e->plan_kind == 1) return e->plan_blocks;
  const int64_t T = e->plan_T;
  const int64_t g = std::min<int64_t>(T, std::max<int64_t>(groups, 1));
  return static_cast<int>(std::min<int64_t>(T, T / e->plan_bt + g));
}

// Distinct ids an adapter-store call on a device-built plan can resolve,
// given `registered` adapters and a table window of `window` ids (the
// selected layer's: a multi-layer store is not bounded by every layer's
// adapters).  An eager call counts the adapters registered now: a routing
// that names only registered ids stays within it.  A call being captured
// into a graph is replayed after later registrations, so it counts every id
// of the window (its grid then holds up to T block slots, most of them empty
// at decode sizes), unless the caller declared the most adapters it will
// register (wp_set_max_adapters), which registration then enforces.
int64_t call_ids(const wp_engine* e, hipStream_t stream, int64_t registered, int64_t window) {
  if (e->max_adapters > 0) return std::min<int64_t>(window, e->max_adapters);
  if (stream_capturing(stream)) return window;
  return std::min<int64_t>(window, registered);
}

int64_t resolvable_ids(const wp_engine* e, hipStream_t stream) {
  const int64_t window =
      e->entry_count > 0 ? e->entry_count : std::max<int64_t>(0, static_cast<int64_t>(e->table_cap) - e->entry_offset);
  return call_ids(e, stream, static_cast<int64_t>(e->adapters.size()), window);
}

// Registration past the declared maximum (wp_set_max_adapters) is refused:
// grids sized by it would drop the extra adapters' blocks.
int check_max_adapters(const wp_engine* e, int32_t adapter_id) {
  if (e->max_adapters > 0 && e->adapters.count(adapter_id) == 0 &&
      static_cast<int64_t>(e->adapters.size()) >= e->max_adapters)
    return fail(WP_ERR_CAPACITY, "register_adapter: %lld adapters are registered, the declared maximum "
                                 "(set_max_adapters)", (long long)e->max_adapters);
  return WP_OK;
}


}  // namespace

// ============================================================================
// C ABI
// ============================================================================

extern "C" {

const char* wp_last_error(void) { return g_last_error.c_str(); }

int wp_abi_version(void) { return WP_ABI_VERSION; }

int wp_rank_supported(int32_t rank) { return rank_ok(rank) ? 1 : 0; }

int wp_block_tokens(int64_t T) { return plan_block_tokens(T); }

int wp_create(const wp_config* cfg_in, wp_engine** out) {
  if (out == nullptr) return fail(WP_ERR_INVALID, "wp_create: out is NULL");
  *out = nullptr;
  wp_config cfg{};
  cfg.device = 0;
  cfg.num_staging_slots = 8;
  cfg.max_tokens = kPlanMaxTokens;
  cfg.max_rank = kMaxRank;
  cfg.max_adapter_ids = kDefaultTableIds;
  if (cfg_in) cfg = *cfg_in;
  if (cfg.max_adapter_ids == 0) cfg.max_adapter_ids = kDefaultTableIds;
  if (cfg.max_tokens <= 0 || cfg.max_tokens > kPlanMaxTokens)
    return fail(WP_ERR_INVALID, "wp_create: max_tokens must be in [1, %d]", kPlanMaxTokens);
  if (cfg.num_staging_slots < 0 || cfg.num_staging_slots > kMaxStagingSlots)
    return fail(WP_ERR_INVALID, "wp_create: num_staging_slots must be in [0, %d]", kMaxStagingSlots);
  if (cfg.max_adapter_ids < 0 || cfg.max_adapter_ids > kMaxTableIds)
    return fail(WP_ERR_INVALID, "wp_create: max_adapter_ids must be in [0, %d]", kMaxTableIds);
  int ndev = 0;
  const hipError_t ce = hipGetDeviceCount(&ndev);
  if (ce != hipSuccess || ndev <= 0)
    return fail(WP_ERR_NO_DEVICE, "wp_create: no HIP device available (%s)", hipGetErrorString(ce));
  if (cfg.device < 0 || cfg.device >= ndev) return fail(WP_ERR_INVALID, "wp_create: device %d out of range", cfg.device);
  DeviceGuard g(cfg.device);

  wp_engine* e = new wp_engine();
  e->device = cfg.device;
  // Four SIMDs per CU and four waves per workgroup: a CU holds as many
  // workgroups as a SIMD holds waves.
  if (hipDeviceGetAttribute(&e->n_cu, hipDeviceAttributeMultiprocessorCount, cfg.device) != hipSuccess || e->n_cu <= 0)
    e->n_cu = 256;
  e->cfg = cfg;
  auto bail = [&](int rc) {
    wp_destroy(e);
    return rc;
  };

  hipMemPoolProps props{};
  props.allocType = hipMemAllocationTypePinned;
  props.location.type = hipMemLocationTypeDevice;
  props.location.id = cfg.device;
  if (hipMemPoolCreate(&e->pool, &props) != hipSuccess)
    return bail(fail(WP_ERR_HIP, "wp_create: hipMemPoolCreate failed"));
  uint64_t keep = ~0ull;
  (void)hipMemPoolSetAttribute(e->pool, hipMemPoolAttrReleaseThreshold, &keep);
  // A block freed on one stream is reused by another only once the free has
  // completed; the pool never makes a stream wait for another's frees.
  int no = 0, yes = 1;
  (void)hipMemPoolSetAttribute(e->pool, hipMemPoolReuseAllowInternalDependencies, &no);
  (void)hipMemPoolSetAttribute(e->pool, hipMemPoolReuseFollowEventDependencies, &no);
  (void)hipMemPoolSetAttribute(e->pool, hipMemPoolReuseAllowOpportunistic, &yes);

  e->tok_cap = cfg.max_tokens;
  e->seg_cap = std::max(cfg.max_tokens, kRefMaxSegments);
  e->block_cap = cfg.max_tokens + kRefMaxSegments;
  e->entry_cap = kRefMaxSegments;
  e->table_cap = cfg.max_adapter_ids;
  e->ptok = std::min(cfg.max_tokens, kSmallPlanTokens);
  e->part_words = static_cast<uint64_t>(kMaxChunks) * e->ptok * kMaxRank;
  e->consumed_words = static_cast<uint64_t>(e->block_cap) * kCounterStride;
  size_t off = 0;
  auto carve = [&](size_t bytes) {
    const size_t at = off;
    off += (bytes + 255) & ~size_t(255);
    return at;
  };
  const size_t o_hdr = carve(sizeof(uint32_t) * kHdrWords);
  const size_t o_seg = carve(sizeof(Segment) * e->seg_cap);
  const size_t o_blk = carve(sizeof(Block) * e->block_cap);
  const size_t o_perm = carve(sizeof(int32_t) * e->tok_cap);
  const size_t o_bperm = carve(sizeof(int32_t) * static_cast<size_t>(e->block_cap) * kBlockTokens);
  const size_t o_cons = carve(sizeof(uint32_t) * e->consumed_words);
  const size_t o_ent = carve(sizeof(Entry) * e->entry_cap);
  const size_t o_pub = carve(sizeof(SlotPub) * std::max(cfg.num_staging_slots, 1));
  const size_t o_ret = carve(sizeof(uint32_t) * std::max(cfg.num_staging_slots, 1));
  const size_t o_lin = carve(sizeof(uint32_t) * (kLinCounters + 2 * static_cast<size_t>(e->block_cap)));
  const size_t o_tab = carve(sizeof(Entry) * std::max(e->table_cap, 1));
  const size_t o_bent = carve(sizeof(Entry) * e->block_cap);
  const size_t o_spart = carve(sizeof(float) * kMaxChunks * static_cast<size_t>(e->tok_cap) * kMaxRank);
  const size_t hbuf_bytes = sizeof(uint16_t) * static_cast<size_t>(e->tok_cap) * kMaxSlices * kMaxRank;
  const size_t o_hbuf = carve(hbuf_bytes);
  const size_t o_part = carve(sizeof(float) * e->part_words);
  if (hipMalloc(reinterpret_cast<void**>(&e->ws), off) != hipSuccess)
    return bail(fail(WP_ERR_HIP, "wp_create: workspace allocation (%zu bytes) failed", off));
  e->header = reinterpret_cast<uint32_t*>(e->ws + o_hdr);
  e->segs = reinterpret_cast<Segment*>(e->ws + o_seg);
  e->blocks = reinterpret_cast<Block*>(e->ws + o_blk);
  e->perm = reinterpret_cast<int32_t*>(e->ws + o_perm);
  e->bperm = reinterpret_cast<int32_t*>(e->ws + o_bperm);
  e->consumed = reinterpret_cast<uint32_t*>(e->ws + o_cons);
  e->plan_entries = reinterpret_cast<Entry*>(e->ws + o_ent);
  e->pubs = reinterpret_cast<SlotPub*>(e->ws + o_pub);
  e->retired = reinterpret_cast<uint32_t*>(e->ws + o_ret);
  e->lin_cnt = reinterpret_cast<uint32_t*>(e->ws + o_lin);
  e->lin_flag = e->lin_cnt + kLinCounters;
  e->dtable = reinterpret_cast<Entry*>(e->ws + o_tab);
  e->bentries = reinterpret_cast<Entry*>(e->ws + o_bent);
  e->spart = reinterpret_cast<float*>(e->ws + o_spart);
  e->hbuf = e->ws + o_hbuf;
  e->part = reinterpret_cast<float*>(e->ws + o_part);
  // Everything starts at zero except the partials (kPartialEmpty) and the
  // publications' ids (-1: nothing published); filled by kernels, then waited for.
  if (launch_fill_u32(reinterpret_cast<uint32_t*>(e->ws), 0u, o_part / 4, nullptr) != hipSuccess ||
      launch_fill_u32(reinterpret_cast<uint32_t*>(e->part), kPartialEmpty, e->part_words, nullptr) != hipSuccess)
    return bail(fail(WP_ERR_HIP, "wp_create: workspace fill failed"));
  for (int i = 0; i < cfg.num_staging_slots; ++i) {
    EntryWrites w{};
    w.pub = e->pubs + i;
    w.pub_id = -1;
    if (launch_entry_writes(w, nullptr) != hipSuccess) return bail(fail(WP_ERR_HIP, "wp_create: slot setup failed"));
  }
  if (hipDeviceSynchronize() != hipSuccess) return bail(fail(WP_ERR_HIP, "wp_create: workspace setup failed"));

  e->pinned_bytes = sizeof(uint32_t) * kHdrWords + sizeof(Segment) * e->seg_cap + sizeof(Block) * e->block_cap +
                    sizeof(int32_t) * e->tok_cap + sizeof(int32_t) * static_cast<size_t>(e->block_cap) * kBlockTokens +
                    sizeof(Entry) * e->entry_cap + 1024;
  for (int i = 0; i < kUploadRing; ++i) {
    if (hipHostMalloc(reinterpret_cast<void**>(&e->pinned[i]), e->pinned_bytes, hipHostMallocDefault) != hipSuccess)
      return bail(fail(WP_ERR_HIP, "wp_create: pinned upload buffer failed"));
    if (hipEventCreateWithFlags(&e->upload_done[i], hipEventDisableTiming) != hipSuccess)
      return bail(fail(WP_ERR_HIP, "wp_create: event creation failed"));
  }
  // The prefetch engine's own stream, default priority, never synchronising
  // with the null stream (reference: bindings:32).
  if (hipStreamCreateWithFlags(&e->pstream, hipStreamNonBlocking) != hipSuccess)
    return bail(fail(WP_ERR_HIP, "wp_create: prefetch stream creation failed"));
  // The first host-to-device copy on a new stream sets up its copy queue
  // (~5 ms on MI355X, with the host blocked): pay it here, not in the first
  // prefetch_adapter of a serving loop.  hbuf is scratch with no contents yet.
  if (hipMemcpyAsync(e->hbuf, e->pinned[0], std::min(e->pinned_bytes, hbuf_bytes), hipMemcpyHostToDevice,
                     e->pstream) != hipSuccess ||
      hipStreamSynchronize(e->pstream) != hipSuccess)
    return bail(fail(WP_ERR_HIP, "wp_create: prefetch stream warm-up copy failed"));
  e->slots.resize(cfg.num_staging_slots);
  for (auto& s : e->slots) {
    if (hipEventCreateWithFlags(&s.ready, hipEventDisableTiming) != hipSuccess)
      return bail(fail(WP_ERR_HIP, "wp_create: slot event creation failed"));
  }
  void* eh = nullptr;
  void* ed = nullptr;
  if (hipHostMalloc(&eh, 256, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess ||
      hipHostGetDevicePointer(&ed, eh, 0) != hipSuccess ||
      hipEventCreateWithFlags(&e->err_ready, hipEventDisableTiming) != hipSuccess) {
    if (eh) (void)hipHostFree(eh);
    return bail(fail(WP_ERR_HIP, "wp_create: error word setup failed"));
  }
  e->err_host = static_cast<uint32_t*>(eh);
  e->err_hdev = static_cast<uint32_t*>(ed);
  *e->err_host = 0;
  *out = e;
  return WP_OK;
}

int wp_destroy(wp_engine* e) {
  if (e == nullptr) return WP_OK;
  DeviceGuard g(e->device);
  (void)hipDeviceSynchronize();
  for (auto& kv : e->adapters) {
    Adapter& ad = kv.second;
    if (ad.dA && !ad.borrowed) (void)hipFree(ad.dA);
    if (ad.dB && !ad.borrowed) (void)hipFree(ad.dB);
    if (ad.host) (void)hipHostFree(ad.host);
    if (ad.copied) (void)hipEventDestroy(ad.copied);
  }
  sweep_graveyard(e, true);
  for (auto& f : e->free_bufs) (void)hipFree(f.ptr);
  for (auto& kv : e->event_refs) (void)hipEventDestroy(kv.first);
  for (hipEvent_t ev : e->spare_events) (void)hipEventDestroy(ev);
  for (auto& s : e->slots) {
    if (s.A) (void)hipFree(s.A);
    if (s.B) (void)hipFree(s.B);
    if (s.ready) (void)hipEventDestroy(s.ready);
  }
  if (e->ws) (void)hipFree(e->ws);
  for (int i = 0; i < kUploadRing; ++i) {
    if (e->pinned[i]) (void)hipHostFree(e->pinned[i]);
    if (e->upload_done[i]) (void)hipEventDestroy(e->upload_done[i]);
  }
  if (e->err_host) (void)hipHostFree(e->err_host);
  if (e->err_ready) (void)hipEventDestroy(e->err_ready);
  if (e->pstream) (void)hipStreamDestroy(e->pstream);
  if (e->pool) (void)hipMemPoolDestroy(e->pool);
  delete e;
  return WP_OK;
}

int wp_register_adapter(wp_engine* e, int32_t adapter_id, const void* A, const void* B, int32_t rank, int32_t d_model,
                        int32_t out_features, float alpha_scale, int32_t dtype, int32_t host_resident, void* stream_) {
  if (!e) return fail(WP_ERR_INVALID, "register_adapter: engine is NULL");
  if (!rank_ok(rank)) return fail(WP_ERR_INVALID, "register_adapter: unsupported rank %d (only 8/16/32/64)", rank);
  if (dtype != WP_DTYPE_F16 && dtype != WP_DTYPE_BF16) return fail(WP_ERR_INVALID, "register_adapter: bad dtype");
  if (d_model <= 0 || d_model % 8 != 0) return fail(WP_ERR_INVALID, "register_adapter: d_model must be a positive multiple of 8");
  if (out_features <= 0 || out_features % 4 != 0)
    return fail(WP_ERR_INVALID, "register_adapter: out_features must be a positive multiple of 4");
  if (!A || !B) return fail(WP_ERR_INVALID, "register_adapter: null weights");
  // Reference: AdapterStore::register_adapter rejects pointers that are not
  // 16-byte aligned (adapter_store.h:23-25).
  if (!aligned(A, 16) || !aligned(B, 16))
    return fail(WP_ERR_INVALID, "AdapterStore::register_adapter: A/B pointer not 16-byte aligned");
  DeviceGuard g(e->device);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (stream_capturing(stream)) return fail(WP_ERR_STATE, "register_adapter cannot run during graph capture");
  int rc = check_max_adapters(e, adapter_id);
  if (rc != WP_OK) return rc;
  if ((rc = evict_impl(e, adapter_id, stream)) != WP_OK) return rc;
  Adapter ad;
  ad.rank = rank;
  ad.d = d_model;
  ad.o = out_features;
  ad.dtype = dtype;
  ad.alpha = alpha_scale;
  ad.a_bytes = sizeof(uint16_t) * static_cast<size_t>(rank) * d_model;
  ad.b_bytes = sizeof(uint16_t) * static_cast<size_t>(out_features) * rank;
  if (host_resident) {
    // Pinned and mapped: the staging copy kernel reads it directly.
    const size_t a_span = (ad.a_bytes + 255) & ~size_t(255);
    WP_HIP(hipHostMalloc(&ad.host, a_span + ad.b_bytes, hipHostMallocMapped));
    std::memcpy(ad.host, A, ad.a_bytes);
    std::memcpy(static_cast<char*>(ad.host) + a_span, B, ad.b_bytes);
    void* dev = nullptr;
    WP_HIP(hipHostGetDevicePointer(&dev, ad.host, 0));
    ad.hA = dev;
    ad.hB = static_cast<char*>(dev) + a_span;
  } else {
    WP_HIP(hipMallocFromPoolAsync(&ad.dA, ad.a_bytes, e->pool, stream));
    WP_HIP(hipMallocFromPoolAsync(&ad.dB, ad.b_bytes, e->pool, stream));
    WP_HIP(hipMemcpyAsync(ad.dA, A, ad.a_bytes, hipMemcpyDefault, stream));
    WP_HIP(hipMemcpyAsync(ad.dB, B, ad.b_bytes, hipMemcpyDefault, stream));
    WP_HIP(hipEventCreateWithFlags(&ad.copied, hipEventDisableTiming));
    WP_HIP(hipEventRecord(ad.copied, stream));
  }
  e->adapters[adapter_id] = ad;
  return table_write(e, adapter_id, registered_entry(ad), stream);
}

int wp_register_adapter_ref(wp_engine* e, int32_t adapter_id, const void* A, const void* B, int32_t rank,
                            int32_t d_model, int32_t out_features, float alpha_scale, int32_t dtype, void* stream_) {
  if (!e) return fail(WP_ERR_INVALID, "register_adapter_ref: engine is NULL");
  if (!rank_ok(rank)) return fail(WP_ERR_INVALID, "register_adapter: unsupported rank %d (only 8/16/32/64)", rank);
  if (dtype != WP_DTYPE_F16 && dtype != WP_DTYPE_BF16) return fail(WP_ERR_INVALID, "register_adapter: bad dtype");
  if (d_model <= 0 || d_model % 8 != 0) return fail(WP_ERR_INVALID, "register_adapter: d_model must be a positive multiple of 8");
  if (out_features <= 0 || out_features % 4 != 0)
    return fail(WP_ERR_INVALID, "register_adapter: out_features must be a positive multiple of 4");
  if (!A || !B) return fail(WP_ERR_INVALID, "register_adapter: null weights");
  if (!aligned(A, 16) || !aligned(B, 16))
    return fail(WP_ERR_INVALID, "AdapterStore::register_adapter: A/B pointer not 16-byte aligned");
  DeviceGuard g(e->device);
  // The kernels read the pointers directly: they must be device memory of
  // this engine's device.
  for (const void* p : {A, B}) {
    hipPointerAttribute_t at{};
    if (hipPointerGetAttributes(&at, p) != hipSuccess || at.type != hipMemoryTypeDevice || at.device != e->device) {
      (void)hipGetLastError();
      return fail(WP_ERR_INVALID, "register_adapter_ref: A/B must be device memory of device %d", e->device);
    }
  }
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (stream_capturing(stream)) return fail(WP_ERR_STATE, "register_adapter cannot run during graph capture");
  int rc = check_max_adapters(e, adapter_id);
  if (rc != WP_OK) return rc;
  if ((rc = evict_impl(e, adapter_id, stream)) != WP_OK) return rc;
  Adapter ad;
  ad.rank = rank;
  ad.d = d_model;
  ad.o = out_features;
  ad.dtype = dtype;
  ad.alpha = alpha_scale;
  ad.a_bytes = sizeof(uint16_t) * static_cast<size_t>(rank) * d_model;
  ad.b_bytes = sizeof(uint16_t) * static_cast<size_t>(out_features) * rank;
  ad.dA = const_cast<void*>(A);
  ad.dB = const_cast<void*>(B);
  ad.borrowed = true;
  e->adapters[adapter_id] = ad;
  return table_write(e, adapter_id, registered_entry(ad), stream);
}

int wp_evict_adapter(wp_engine* e, int32_t adapter_id, void* stream) {
  if (!e) return fail(WP_ERR_INVALID, "evict_adapter: engine is NULL");
  DeviceGuard g(e->device);
  if (stream_capturing(static_cast<hipStream_t>(stream)))
    return fail(WP_ERR_STATE, "evict_adapter cannot run during graph capture");
  return evict_impl(e, adapter_id, static_cast<hipStream_t>(stream));
}

int wp_has_adapter(wp_engine* e, int32_t adapter_id) { return (e && e->adapters.count(adapter_id)) ? 1 : 0; }

int wp_set_max_adapters(wp_engine* e, int64_t n) {
  if (!e) return fail(WP_ERR_INVALID, "set_max_adapters: engine is NULL");
  if (n < 0) return fail(WP_ERR_INVALID, "set_max_adapters: negative count");
  if (n > 0 && static_cast<int64_t>(e->adapters.size()) > n)
    return fail(WP_ERR_STATE, "set_max_adapters: %zu adapters are registered already", e->adapters.size());
  e->max_adapters = n;
  return WP_OK;
}

int wp_set_entry_offset(wp_engine* e, int32_t offset, int32_t count) {
  if (!e) return fail(WP_ERR_INVALID, "set_entry_offset: engine is NULL");
  if (offset < 0 || count < 0) return fail(WP_ERR_INVALID, "set_entry_offset: negative offset %d / count %d", offset, count);
  e->entry_offset = offset;
  e->entry_count = count;
  return WP_OK;
}

int wp_build_segments(wp_engine* e, const int32_t* ids, int32_t K, const int32_t* offsets, int32_t n_offsets,
                      void* stream_) {
  if (!e) return fail(WP_ERR_INVALID, "build_segments: engine is NULL");
  if (K < 0 || n_offsets != K + 1)
    return fail(WP_ERR_INVALID, "build_segment_table: seg_offsets must have K+1 entries");
  if (K > kRefMaxSegments) return fail(WP_ERR_CAPACITY, "build_segment_table: K exceeds WP_MAX_SEGMENTS");
  DeviceGuard g(e->device);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (stream_capturing(stream)) return fail(WP_ERR_STATE, "build_segments cannot run during graph capture");

  // Entries (one per distinct adapter, first-appearance order) and groups.
  std::vector<int32_t> entry_ids;
  std::vector<int> entry_slot;
  std::vector<Entry> entries;
  std::unordered_map<int32_t, int> entry_of;
  std::vector<std::vector<int>> group_segs;
  std::vector<std::pair<int32_t, int32_t>> ranges;
  int64_t max_end = 0;
  for (int k = 0; k < K; ++k) {
    const int32_t id = ids[k];
    const int32_t st = offsets[k];
    const int32_t cnt = offsets[k + 1] - offsets[k];
    auto it = e->adapters.find(id);
    if (it == e->adapters.end()) return fail(WP_ERR_UNKNOWN_ADAPTER, "AdapterStore::lookup: unknown adapter_id %d", id);
    if (st < 0 || cnt < 0) return fail(WP_ERR_INVALID, "build_segments: segment %d has a negative start or count", k);
    auto ei = entry_of.find(id);
    int ent;
    if (ei == entry_of.end()) {
      int su = -1;
      Entry en = entry_for(e, id, it->second, &su);
      if (en.a_ptr == 0)
        return fail(WP_ERR_STATE, "build_segments: adapter %d is host-resident and not staged (prefetch it first)", id);
      ent = static_cast<int>(entries.size());
      entry_of[id] = ent;
      entries.push_back(en);
      entry_ids.push_back(id);
      entry_slot.push_back(su);
      group_segs.emplace_back();
    } else {
      ent = ei->second;
    }
    if (cnt > 0) {
      group_segs[ent].push_back(k);
      ranges.emplace_back(st, cnt);
      max_end = std::max<int64_t>(max_end, static_cast<int64_t>(st) + cnt);
    }
  }
  std::sort(ranges.begin(), ranges.end());
  for (size_t i = 1; i < ranges.size(); ++i)
    if (static_cast<int64_t>(ranges[i - 1].first) + ranges[i - 1].second > ranges[i].first)
      return fail(WP_ERR_INVALID, "build_segments: segments overlap at token %d", ranges[i].first);
  int64_t n_tok = 0;
  for (auto& r : ranges) n_tok += r.second;
  if (n_tok > e->tok_cap)
    return fail(WP_ERR_CAPACITY, "build_segments: %lld tokens exceed max_tokens %d", (long long)n_tok, e->tok_cap);
  // Large-plan calls keep H in the engine's [max_tokens, 64] buffer by token
  // row, so the last token row bounds the table as much as the token count.
  if (max_end > e->tok_cap)
    return fail(WP_ERR_CAPACITY, "build_segments: segments reach token %lld, beyond max_tokens %d",
                (long long)max_end, e->tok_cap);

  // The ring's next pinned buffer: only the upload issued kUploadRing builds
  // ago can still be reading it.
  const int ring = e->upload_next;
  e->upload_next = (ring + 1) % kUploadRing;
  if (e->upload_pending[ring]) {
    WP_HIP(hipEventSynchronize(e->upload_done[ring]));
    e->upload_pending[ring] = false;
  }
  char* p = e->pinned[ring];
  uint32_t* hdr = reinterpret_cast<uint32_t*>(p);
  Segment* hsegs = reinterpret_cast<Segment*>(p + 256);
  Block* hblocks = reinterpret_cast<Block*>(reinterpret_cast<char*>(hsegs) + sizeof(Segment) * std::max(K, 1));
  int32_t* hperm = nullptr;
  Entry* hent = nullptr;
  for (int k = 0; k < K; ++k) {
    hsegs[k].adapter_id = ids[k];
    hsegs[k].token_start = offsets[k];
    hsegs[k].token_count = offsets[k + 1] - offsets[k];
    hsegs[k].pad = 0;
  }
  // perm: each adapter's segments concatenated; blocks of bt tokens.
  const int bt = plan_block_tokens(max_end);
  std::vector<int32_t> perm_v;
  perm_v.reserve(static_cast<size_t>(n_tok));
  std::vector<Block> blocks_v;
  for (size_t ent = 0; ent < group_segs.size(); ++ent) {
    const int first = static_cast<int>(perm_v.size());
    for (int k : group_segs[ent])
      for (int32_t t = offsets[k]; t < offsets[k + 1]; ++t) perm_v.push_back(t);
    const int n = static_cast<int>(perm_v.size()) - first;
    for (int j = 0; j < n; j += bt) {
      Block b;
      b.adapter_id = entry_ids[ent];
      b.first = first + j;
      b.count = std::min(bt, n - j);
      b.entry = static_cast<int>(ent);
      blocks_v.push_back(b);
    }
  }
  if (static_cast<int>(blocks_v.size()) > e->block_cap) return fail(WP_ERR_CAPACITY, "build_segments: too many blocks");
  std::memcpy(hblocks, blocks_v.data(), sizeof(Block) * blocks_v.size());
  hperm = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(hblocks) + sizeof(Block) * std::max<size_t>(blocks_v.size(), 1));
  std::memcpy(hperm, perm_v.data(), sizeof(int32_t) * perm_v.size());
  int32_t* hbperm = hperm + std::max<size_t>(perm_v.size(), 1);
  for (size_t q = 0; q < blocks_v.size(); ++q)
    for (int j = 0; j < kBlockTokens; ++j)
      hbperm[q * kBlockTokens + j] = j < blocks_v[q].count ? perm_v[blocks_v[q].first + j] : -1;
  char* pe = reinterpret_cast<char*>(hbperm + std::max<size_t>(blocks_v.size(), 1) * kBlockTokens);
  pe = reinterpret_cast<char*>((reinterpret_cast<uintptr_t>(pe) + 63) & ~uintptr_t(63));
  hent = reinterpret_cast<Entry*>(pe);
  std::memcpy(hent, entries.data(), sizeof(Entry) * entries.size());
  hdr[kHdrNumSegments] = static_cast<uint32_t>(K);
  hdr[kHdrNumBlocks] = static_cast<uint32_t>(blocks_v.size());
  hdr[kHdrNumGroups] = static_cast<uint32_t>(entries.size());
  hdr[kHdrNumValid] = static_cast<uint32_t>(n_tok);
  hdr[kHdrT] = static_cast<uint32_t>(max_end);

  WP_HIP(hipMemcpyAsync(e->header, hdr, sizeof(uint32_t) * kHdrErrors, hipMemcpyHostToDevice, stream));
  if (K > 0) WP_HIP(hipMemcpyAsync(e->segs, hsegs, sizeof(Segment) * K, hipMemcpyHostToDevice, stream));
  if (!blocks_v.empty())
    WP_HIP(hipMemcpyAsync(e->blocks, hblocks, sizeof(Block) * blocks_v.size(), hipMemcpyHostToDevice, stream));
  if (!perm_v.empty())
    WP_HIP(hipMemcpyAsync(e->perm, hperm, sizeof(int32_t) * perm_v.size(), hipMemcpyHostToDevice, stream));
  if (!blocks_v.empty())
    WP_HIP(hipMemcpyAsync(e->bperm, hbperm, sizeof(int32_t) * blocks_v.size() * kBlockTokens, hipMemcpyHostToDevice,
                          stream));
  if (!entries.empty())
    WP_HIP(hipMemcpyAsync(e->plan_entries, hent, sizeof(Entry) * entries.size(), hipMemcpyHostToDevice, stream));
  WP_HIP(hipEventRecord(e->upload_done[ring], stream));
  e->upload_pending[ring] = true;
  // What a device plan build does first: ready publications into the table,
  // the partial buffer's repair after a give-up.
  WP_HIP(launch_maintain(e->header, maint_view(e), stream));

  e->plan_kind = 1;
  e->plan_T = max_end;
  e->plan_bt = bt;
  e->plan_blocks = static_cast<int>(blocks_v.size());
  e->plan_valid = static_cast<int>(n_tok);
  e->plan_entry_ids = entry_ids;
  e->plan_entry_slot = entry_slot;
  return WP_OK;
}

int wp_build_seg_bounds(wp_engine* e, const void* idx, int32_t idx_is_int64, int64_t T, void* stream_) {
  if (!e) return fail(WP_ERR_INVALID, "build_seg_bounds: engine is NULL");
  if (T < 0) return fail(WP_ERR_INVALID, "build_seg_bounds: negative token count");
  // Reference: returns False, and launches nothing, above its capacity (bindings:165-166).
  if (T > e->cfg.max_tokens) return WP_NOT_HANDLED;
  if (T > 0 && idx == nullptr) return fail(WP_ERR_INVALID, "build_seg_bounds: null indices");
  DeviceGuard g(e->device);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  const int bt = plan_block_tokens(T);
  Maint m = maint_view(e);
  m.trace = e->trace_words >= 8 ? e->trace : nullptr;
  // Engines with registered adapters (table-mode calls) get each block's
  // table entry copied by the plan build; stacked-weight engines skip it.
  Entry* bent = e->adapters.empty() ? nullptr : e->bentries;
  WP_HIP(launch_plan(idx, idx_is_int64 ? 1 : 0, static_cast<int>(T), e->header, e->segs, e->blocks, e->perm,
                     e->bperm, bent, e->seg_cap, e->block_cap, bt, &m, stream));
  e->plan_bentries = bent != nullptr;
  // Slots whose copy had landed are in the table once this build has run
  // (event queries are not allowed while a graph is being captured).
  if (!stream_capturing(stream))
    for (auto& sl : e->slots)
      if (sl.issued && !sl.applied && hipEventQuery(sl.ready) == hipSuccess) sl.applied = true;
  e->plan_kind = 2;
  e->plan_T = T;
  e->plan_bt = bt;
  e->plan_blocks = -1;
  e->plan_valid = -1;
  e->plan_entry_ids.clear();
  e->plan_entry_slot.clear();
  return WP_OK;
}

int wp_read_segments(wp_engine* e, int32_t* out, int64_t cap, int64_t* num_segments, void* stream_) {
  if (!e || !num_segments) return fail(WP_ERR_INVALID, "read_segments: null argument");
  DeviceGuard g(e->device);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  uint32_t hdr[kHdrWords];
  WP_HIP(hipMemcpyAsync(hdr, e->header, sizeof(hdr), hipMemcpyDeviceToHost, stream));
  WP_HIP(hipStreamSynchronize(stream));
  const int64_t n = e->plan_kind == 0 ? 0 : hdr[kHdrNumSegments];
  *num_segments = n;
  const int64_t m = std::min<int64_t>(std::min<int64_t>(n, cap), e->seg_cap);
  if (m > 0 && out) {
    std::vector<Segment> tmp(static_cast<size_t>(m));
    WP_HIP(hipMemcpyAsync(tmp.data(), e->segs, sizeof(Segment) * m, hipMemcpyDeviceToHost, stream));
    WP_HIP(hipStreamSynchronize(stream));
    for (int64_t i = 0; i < m; ++i) {
      out[3 * i + 0] = tmp[i].adapter_id;
      out[3 * i + 1] = tmp[i].token_start;
      out[3 * i + 2] = tmp[i].token_count;
    }
  }
  return WP_OK;
}

int wp_read_plan(wp_engine* e, int32_t* perm, int64_t perm_cap, int32_t* blocks, int64_t block_cap, int64_t* n_valid,
                 int64_t* n_blocks, void* stream_) {
  if (!e || !n_valid || !n_blocks) return fail(WP_ERR_INVALID, "read_plan: null argument");
  DeviceGuard g(e->device);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  uint32_t hdr[kHdrWords];
  WP_HIP(hipMemcpyAsync(hdr, e->header, sizeof(hdr), hipMemcpyDeviceToHost, stream));
  WP_HIP(hipStreamSynchronize(stream));
  *n_valid = hdr[kHdrNumValid];
  *n_blocks = hdr[kHdrNumBlocks];
  const int64_t np = std::min<int64_t>(*n_valid, perm_cap);
  const int64_t nb = std::min<int64_t>(*n_blocks, block_cap);
  if (np > 0 && perm) WP_HIP(hipMemcpyAsync(perm, e->perm, sizeof(int32_t) * np, hipMemcpyDeviceToHost, stream));
  if (nb > 0 && blocks) WP_HIP(hipMemcpyAsync(blocks, e->blocks, sizeof(Block) * nb, hipMemcpyDeviceToHost, stream));
  WP_HIP(hipStreamSynchronize(stream));
  return WP_OK;
}

int wp_read_device_errors(wp_engine* e, uint32_t* flags, void* stream_) {
  if (!e || !flags) return fail(WP_ERR_INVALID, "read_device_errors: null argument");
  DeviceGuard g(e->device);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (stream_capturing(stream)) return fail(WP_ERR_STATE, "read_device_errors cannot run during graph capture");
  uint32_t v = 0;
  // Bits a poll (wp_poll_device_errors) has already moved out of the word.
  if (e->err_pending) {
    WP_HIP(hipEventSynchronize(e->err_ready));
    v |= __atomic_load_n(e->err_host, __ATOMIC_ACQUIRE);
    e->err_pending = false;
  }
  uint32_t w = 0;
  WP_HIP(hipMemcpyAsync(&w, e->header + kHdrErrors, sizeof(w), hipMemcpyDeviceToHost, stream));
  WP_HIP(hipStreamSynchronize(stream));
  WP_HIP(launch_fill_u32(e->header + kHdrErrors, 0u, 1, stream));
  v |= w;
  // After a give-up the buffer is repaired here too, not only at the next plan build.
  if (v & kErrSpin) WP_HIP(launch_maintain(e->header, maint_view(e), stream));
  WP_HIP(hipStreamSynchronize(stream));
  *flags = v;
  return WP_OK;
}

int wp_poll_device_errors(wp_engine* e, uint32_t* flags, void* stream_) {
  if (!e || !flags) return fail(WP_ERR_INVALID, "poll_device_errors: null argument");
  *flags = 0;
  DeviceGuard g(e->device);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (stream_capturing(stream)) return WP_OK;
  if (e->err_pending) {
    const hipError_t q = hipEventQuery(e->err_ready);
    if (q == hipErrorNotReady) {
      (void)hipGetLastError();
      return WP_OK;  // the previous take is still in flight: its bits come with a later poll
    }
    WP_HIP(q);
    *flags = __atomic_load_n(e->err_host, __ATOMIC_ACQUIRE);
    e->err_pending = false;
  }
  // The word as of this point of the stream, moved to the host word and
  // cleared on the device in one exchange.
  WP_HIP(launch_take_word(e->header + kHdrErrors, e->err_hdev, stream));
  WP_HIP(hipEventRecord(e->err_ready, stream));
  e->err_pending = true;
  return WP_OK;
}

namespace {

int check_io(const char* who, int32_t dtype, const void* p16, const char* name) {
  if (dtype != WP_DTYPE_F16 && dtype != WP_DTYPE_BF16) return fail(WP_ERR_INVALID, "%s: dtype must be fp16 or bf16", who);
  if (p16 && !aligned(p16, 16)) return fail(WP_ERR_INVALID, "%s: %s must be 16-byte aligned", who, name);
  return WP_OK;
}

// Table-mode weights for the current plan.
int table_weights(wp_engine* e, hipStream_t stream, Weights* w) {
  w->mode = kTable;
  if (e->plan_kind == 1) {
    if (e->entry_offset != 0)
      return fail(WP_ERR_INVALID, "adapter layers other than 0 need a build_seg_bounds table (build_segments resolves "
                                  "its adapters when it is called)");
    w->entries = e->plan_entries;
    w->num_ids = static_cast<int32_t>(e->plan_entry_ids.size());
    return WP_OK;
  }
  if (!stream_capturing(stream)) {
    const int rc = apply_ready_slots(e, stream);
    if (rc != WP_OK) return rc;
  }
  // A layer's adapters sit at ids offset by layer * stride: the plan's
  // per-token ids index the table from that offset.
  w->entries = e->dtable + std::min(e->entry_offset, e->table_cap);
  w->num_ids = std::max(0, e->table_cap - e->entry_offset);
  if (e->entry_count > 0) w->num_ids = std::min(w->num_ids, e->entry_count);
  // The plan's copies are of entries at offset 0 (a block's entry is its id).
  w->a_base[0] = e->plan_bentries && e->entry_offset == 0 ? e->bentries : nullptr;
  return WP_OK;
}

// Validates an add_lora call on stacked weights (vLLM's wa_t_all /
// wb_t_all) and fills the launch fields that do not depend on the plan or on
// where the scratch buffers live.  WP_NOT_HANDLED for a rank without kernels
// (reference: add_lora_packed returns False, bindings:197-198).
int stacked_call_args(const char* who, void* y, const void* x, int32_t n_a, const void* const* wa,
                      const int64_t* wa_stride0, int32_t num_loras, int32_t n_slices, const void* const* wb,
                      const int64_t* wb_stride0, const int32_t* out_features, const int32_t* y_col_offsets, float scale,
                      int32_t rank, int32_t d_model, int64_t y_row_stride, int32_t dtype, ApplyArgs* a) {
  if (!rank_ok(rank)) return WP_NOT_HANDLED;
  int rc = check_io(who, dtype, x, "x");
  if (rc != WP_OK) return rc;
  if (n_a != 1 && n_a != n_slices) return fail(WP_ERR_INVALID, "%s: one A for all slices, or one per slice", who);
  if (!wa || !wa_stride0) return fail(WP_ERR_INVALID, "%s: null wa_t_all", who);
  for (int s = 0; s < n_a; ++s) {
    if ((rc = check_io(who, dtype, wa[s], "wa_t_all")) != WP_OK) return rc;
    if (!wa[s]) return fail(WP_ERR_INVALID, "%s: null wa_t_all", who);
    if (wa_stride0[s] % 8 != 0) return fail(WP_ERR_INVALID, "%s: wa_t_all stride must be a multiple of 8", who);
  }
  if (!y || !aligned(y, 8)) return fail(WP_ERR_INVALID, "%s: y must be 8-byte aligned", who);
  if (d_model <= 0 || d_model % 8 != 0) return fail(WP_ERR_INVALID, "%s: d_model must be a positive multiple of 8", who);
  if (num_loras <= 0) return fail(WP_ERR_INVALID, "%s: num_loras must be positive", who);
  if (n_slices < 1 || n_slices > kMaxSlices || !wb || !wb_stride0 || !out_features || !y_col_offsets)
    return fail(WP_ERR_INVALID, "%s: 1..%d output slices with their weights, strides, widths and offsets", who,
                kMaxSlices);
  if (y_row_stride % 4 != 0) return fail(WP_ERR_INVALID, "%s: y row stride must be a multiple of 4", who);
  for (int s = 0; s < n_slices; ++s) {
    if ((rc = check_io(who, dtype, wb[s], "wb_t_all")) != WP_OK) return rc;
    if (wb_stride0[s] % 8 != 0) return fail(WP_ERR_INVALID, "%s: wb_t_all stride must be a multiple of 8", who);
    if (out_features[s] <= 0 || out_features[s] % 4 != 0 || y_col_offsets[s] < 0 || y_col_offsets[s] % 4 != 0 ||
        y_col_offsets[s] + out_features[s] > y_row_stride)
      return fail(WP_ERR_INVALID, "%s: slice %d window [%d, %d) does not fit y (row stride %lld, 4-aligned)", who, s,
                  y_col_offsets[s], y_col_offsets[s] + out_features[s], (long long)y_row_stride);
  }
  a->rank = rank;
  a->n_sub = 1;
  a->hs1 = rank;
  a->hs = n_a * rank;
  a->x = x;
  a->ldx = d_model;
  a->y = y;
  a->ldy = y_row_stride;
  a->d_model = d_model;
  a->w.mode = kStacked;
  a->w.num_ids = num_loras;
  a->w.n_a = n_a;
  for (int s = 0; s < n_a; ++s) {
    a->w.a_base[s] = wa[s];
    a->w.a_stride[s] = wa_stride0[s];
  }
  a->w.scale = scale;
  a->w.n_slices = n_slices;
  const int cols = expand_cols_per_workgroup();
  int oc = 0;
  for (int s = 0; s < n_slices; ++s) {
    a->w.b_base[s] = wb[s];
    a->w.b_stride[s] = wb_stride0[s];
    a->w.o_size[s] = out_features[s];
    a->w.y_off[s] = y_col_offsets[s];
    a->w.oc_start[s] = oc;
    oc += static_cast<int>(ceil_div(out_features[s], cols));
  }
  a->w.oc_start[n_slices] = oc;
  a->n_ochunks = oc;
  a->spin_limit = kDefaultSpinLimit;
  return WP_OK;
}

// Work split of a fused call (a->n_slots, the output chunks and the rank set):
// about kExpandWorkgroups expand workgroups per block -- wider outputs (several
// slices) give each workgroup several chunks, so that the block's partials are
// summed fewer times -- and the shrink side in 32-row groups for those
// multi-chunk calls (half the shrink workgroups, so more of the expand side is
// resident from the start), 16-row groups otherwise; except that calls small
// enough run one chunk per expand workgroup (below).
void fused_split(ApplyArgs* a, int rank, int d_model, int n_cu) {
  const int64_t resident = static_cast<int64_t>(n_cu) * fused_waves_per_simd(rank, 0);
  a->n_sub = static_cast<int>(ceil_div(a->n_ochunks, kExpandWorkgroups));
  if (a->n_sub > 1) {
    // Several slices, but a grid small enough that the single-chunk kernel
    // (16-row shrink groups, one output chunk per expand workgroup, every
    // workgroup's B and Y loaded before the wait) needs at most twice the
    // workgroups the device holds at once: that kernel, not the multi-chunk
    // one that loads its later chunks only after the partials are in.
    // Measured on MI355X: cfg5's q/k/v (one A per slice) 44-launch step
    // 535 -> 462 us, cfg2 flatness at 1..16 resident adapters 183 -> 168 us
    // (N=1); allowing three times the residency slowed cfg2's qkv call
    // (18.0 -> 19.8 us).
    ApplyArgs one = *a;
    shrink_split(d_model, rank, kShrinkRows, a->w.n_a, a->hs, a->n_slots, a->n_ochunks, resident, &one);
    const int64_t per_block = static_cast<int64_t>(one.n_chunks) * one.n_rgroups * a->w.n_a + a->n_ochunks;
    if (a->n_slots * per_block <= 2 * resident) {
      one.n_sub = 1;
      *a = one;
      return;
    }
  }
  const int multi = a->n_sub > 1 ? 1 : 0;
  shrink_split(d_model, rank, multi ? kShrinkRowsFused : kShrinkRows, a->w.n_a, a->hs, a->n_slots,
               ceil_div(a->n_ochunks, a->n_sub), multi ? 0 : resident, a);
}

}  // namespace

int wp_shrink(wp_engine* e, const void* X, void* H, int32_t d_model, int32_t rank, int64_t T, int64_t h_row_stride,
              int32_t dtype, void* stream_) {
  if (!e) return fail(WP_ERR_INVALID, "shrink: engine is NULL");
  if (rank != 0 && !rank_ok(rank)) return fail(WP_ERR_INVALID, "dispatch_bgmv_shrink: unsupported rank (only 8/16/32/64)");
  int rc = check_io("shrink", dtype, X, "X");
  if (rc != WP_OK) return rc;
  if ((rc = check_io("shrink", dtype, H, "H")) != WP_OK) return rc;
  if (d_model <= 0 || d_model % 8 != 0) return fail(WP_ERR_INVALID, "shrink: d_model must be a positive multiple of 8");
  const int64_t need = rank == 0 ? kMaxRank : rank;
  if (h_row_stride < need || h_row_stride % 8 != 0)
    return fail(WP_ERR_INVALID, "shrink: H row stride %lld must be >= %lld and a multiple of 8", (long long)h_row_stride,
                (long long)need);
  if (e->plan_kind == 0) return fail(WP_ERR_STATE, "shrink: no segment table (call build_segments or build_seg_bounds)");
  if (e->plan_T > T) return fail(WP_ERR_INVALID, "shrink: segments reach token %lld but X has %lld rows", (long long)e->plan_T, (long long)T);
  if (e->plan_kind == 1) {
    for (size_t i = 0; i < e->plan_entry_ids.size(); ++i) {
      const Adapter& ad = e->adapters.at(e->plan_entry_ids[i]);
      if (ad.d != d_model)
        return fail(WP_ERR_INVALID, "shrink: adapter %d has d_model %d, call has %d", e->plan_entry_ids[i], ad.d, d_model);
      if (rank != 0 && ad.rank != rank)
        return fail(WP_ERR_INVALID, "shrink: adapter %d has rank %d, call has %d", e->plan_entry_ids[i], ad.rank, rank);
      if (ad.dtype != dtype) return fail(WP_ERR_INVALID, "shrink: adapter %d dtype differs from X", e->plan_entry_ids[i]);
    }
  }
  DeviceGuard g(e->device);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  ApplyArgs a = base_args(e, rank);
  a.x = X;
  a.ldx = d_model;
  a.h = H;
  a.ldh = h_row_stride;
  a.d_model = d_model;
  if ((rc = table_weights(e, stream, &a.w)) != WP_OK) return rc;
  a.w.n_slices = 1;
  a.n_slots = block_bound(e, resolvable_ids(e, stream));
  if (e->plan_T <= kSmallPlanTokens) {
    // Decode-sized plans: many small shrink workgroups and a reducer per
    // block (the fused calls' shrink side), not one workgroup per block and
    // d-range streaming every rank row.
    shrink_small_split(d_model, rank, &a);
    // The reducers first when they take at most half of the resident
    // workgroups: they then poll while the shrink workgroups stream instead
    // of being dispatched after them.
    a.red_first = 2 * static_cast<int64_t>(a.n_slots) <= static_cast<int64_t>(e->n_cu) * shrink_small_waves_per_simd() ? 1 : 0;
    WP_HIP(launch_shrink_small(dtype == WP_DTYPE_BF16, a, stream));
  } else {
    shrink_range_split(d_model, &a);
    a.part = e->spart;
    a.ptok = e->tok_cap;
    WP_HIP(launch_shrink(dtype == WP_DTYPE_BF16, a, stream));
  }
  return WP_OK;
}

int wp_expand(wp_engine* e, const void* H, void* Y, int32_t out_features, int32_t rank, int64_t T, int64_t h_row_stride,
              int64_t y_row_stride, int32_t y_col_offset, int32_t dtype, void* stream_) {
  if (!e) return fail(WP_ERR_INVALID, "expand: engine is NULL");
  if (rank != 0 && !rank_ok(rank)) return fail(WP_ERR_INVALID, "dispatch_bgmv_expand: unsupported rank (only 8/16/32/64)");
  int rc = check_io("expand", dtype, H, "H");
  if (rc != WP_OK) return rc;
  if (dtype != WP_DTYPE_F16 && dtype != WP_DTYPE_BF16) return fail(WP_ERR_INVALID, "expand: bad dtype");
  if (!aligned(Y, 8)) return fail(WP_ERR_INVALID, "expand: Y must be 8-byte aligned");
  if (out_features <= 0 || out_features % 4 != 0)
    return fail(WP_ERR_INVALID, "expand: out_features must be a positive multiple of 4");
  if (y_col_offset < 0 || y_col_offset % 4 != 0 || y_row_stride % 4 != 0 || y_row_stride < y_col_offset + out_features)
    return fail(WP_ERR_INVALID, "expand: Y window [%d, %d) does not fit row stride %lld with 4-element alignment",
                y_col_offset, y_col_offset + out_features, (long long)y_row_stride);
  const int64_t need = rank == 0 ? kMaxRank : rank;
  if (h_row_stride < need || h_row_stride % 8 != 0) return fail(WP_ERR_INVALID, "expand: bad H row stride");
  if (e->plan_kind == 0) return fail(WP_ERR_STATE, "expand: no segment table (call build_segments or build_seg_bounds)");
  if (e->plan_T > T) return fail(WP_ERR_INVALID, "expand: segments reach token %lld but Y has %lld rows", (long long)e->plan_T, (long long)T);
  if (e->plan_kind == 1) {
    for (size_t i = 0; i < e->plan_entry_ids.size(); ++i) {
      const Adapter& ad = e->adapters.at(e->plan_entry_ids[i]);
      if (ad.o != out_features)
        return fail(WP_ERR_INVALID, "expand: adapter %d has out_features %d, call has %d", e->plan_entry_ids[i], ad.o,
                    out_features);
      if (rank != 0 && ad.rank != rank)
        return fail(WP_ERR_INVALID, "expand: adapter %d has rank %d, call has %d", e->plan_entry_ids[i], ad.rank, rank);
      if (ad.dtype != dtype) return fail(WP_ERR_INVALID, "expand: adapter %d dtype differs from Y", e->plan_entry_ids[i]);
    }
  }
  DeviceGuard g(e->device);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  ApplyArgs a = base_args(e, rank);
  a.h = const_cast<void*>(H);
  a.ldh = h_row_stride;
  a.y = Y;
  a.ldy = y_row_stride;
  if ((rc = table_weights(e, stream, &a.w)) != WP_OK) return rc;
  const int cols = expand_cols_per_workgroup();
  a.w.n_slices = 1;
  a.w.o_size[0] = out_features;
  a.w.y_off[0] = y_col_offset;
  a.w.oc_start[0] = 0;
  a.w.oc_start[1] = static_cast<int32_t>(ceil_div(out_features, cols));
  a.n_ochunks = a.w.oc_start[1];
  a.n_slots = block_bound(e, resolvable_ids(e, stream));
  WP_HIP(launch_expand(dtype == WP_DTYPE_BF16, a, stream));
  return WP_OK;
}

}  // extern "C"

namespace {

// add_lora on stacked weights with one A shared by every slice (n_a = 1) or
// one A per slice (n_a = n_slices).
int add_lora_impl(wp_engine* e, const char* who, void* y, const void* x, int32_t n_a, const void* const* wa,
                  const int64_t* wa_stride0, int32_t num_loras, int32_t n_slices, const void* const* wb,
                  const int64_t* wb_stride0, const int32_t* out_features, const int32_t* y_col_offsets, float scale,
                  int32_t rank, int32_t d_model, int64_t T, int64_t y_row_stride, int32_t dtype, void* stream_) {
  if (!e) return fail(WP_ERR_INVALID, "%s: engine is NULL", who);
  ApplyArgs a{};
  int rc = stacked_call_args(who, y, x, n_a, wa, wa_stride0, num_loras, n_slices, wb, wb_stride0, out_features,
                             y_col_offsets, scale, rank, d_model, y_row_stride, dtype, &a);
  if (rc != WP_OK) return rc;
  if (e->plan_kind == 0) return fail(WP_ERR_STATE, "%s: no segment table (call build_seg_bounds first)", who);
  if (e->plan_T > T)
    return fail(WP_ERR_INVALID, "%s: segments reach token %lld but x has %lld rows", who, (long long)e->plan_T,
                (long long)T);
  DeviceGuard g(e->device);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  a.tiles = (e->plan_bt + 15) / 16;
  a.ptok = e->ptok;
  a.part = e->part;
  a.consumed = e->consumed;
  a.spin_limit = e->spin_limit;
  a.trace = e->trace;
  a.trace_words = e->trace_words;
  a.plan = plan_view(e);
  a.n_slots = block_bound(e, num_loras);
  fused_split(&a, rank, d_model, e->n_cu);
  if (e->plan_bt > 16) {
    // Large plans (prefill-sized, 64-token blocks): shrink into the engine's
    // H (one launch per A slice, each into its columns of an H row), then
    // expand from it.  Each launch keeps several token tiles in flight per
    // workgroup; the kernel boundary replaces the in-kernel wait.
    if (e->plan_T > e->tok_cap) return fail(WP_ERR_CAPACITY, "%s: table reaches past the engine's H rows", who);
    a.h = e->hbuf;
    a.ldh = a.hs;
    a.n_sub = 1;
    shrink_range_split(d_model, &a);
    a.part = e->spart;
    a.ptok = e->tok_cap;
    for (int sa = 0; sa < n_a; ++sa) {
      ApplyArgs as = a;
      as.w.n_a = 1;
      as.hs = as.hs1 = rank;  // the d-range partials' row (a single A slice)
      as.w.a_base[0] = a.w.a_base[sa];
      as.w.a_stride[0] = a.w.a_stride[sa];
      as.h = static_cast<char*>(e->hbuf) + sizeof(uint16_t) * static_cast<size_t>(sa) * rank;
      WP_HIP(launch_shrink(dtype == WP_DTYPE_BF16, as, stream));
    }
    WP_HIP(launch_expand(dtype == WP_DTYPE_BF16, a, stream));
    return WP_OK;
  }
  WP_HIP(launch_fused(dtype == WP_DTYPE_BF16, a, stream));
  return WP_OK;
}

}  // namespace

extern "C" {

int wp_add_lora(wp_engine* e, void* y, const void* x, const void* wa, int64_t wa_stride0, int32_t num_loras,
                int32_t n_slices, const void* const* wb, const int64_t* wb_stride0, const int32_t* out_features,
                const int32_t* y_col_offsets, float scale, int32_t rank, int32_t d_model, int64_t T,
                int64_t y_row_stride, int32_t dtype, void* stream) {
  return add_lora_impl(e, "add_lora", y, x, 1, &wa, &wa_stride0, num_loras, n_slices, wb, wb_stride0, out_features,
                       y_col_offsets, scale, rank, d_model, T, y_row_stride, dtype, stream);
}

int wp_linear_lora(wp_engine* e, void* y, const void* x, const void* w, int64_t w_row_stride, const void* bias,
                   const void* wa, int64_t wa_stride0, const void* wb, int64_t wb_stride0, int32_t num_loras,
                   float scale, int32_t rank, int32_t d_in, int32_t d_out, int64_t T, int32_t dtype, void* stream_) {
  const char* who = "linear_lora";
  if (!e) return fail(WP_ERR_INVALID, "%s: engine is NULL", who);
  ApplyArgs a{};
  const int32_t off0 = 0;
  int rc = stacked_call_args(who, y, x, 1, &wa, &wa_stride0, num_loras, 1, &wb, &wb_stride0, &d_out, &off0, scale,
                             rank, d_in, d_out, dtype, &a);
  if (rc != WP_OK) return rc;
  if ((rc = check_io(who, dtype, w, "w")) != WP_OK) return rc;
  if (!w) return fail(WP_ERR_INVALID, "%s: null weight", who);
  if (!aligned(y, 16)) return fail(WP_ERR_INVALID, "%s: y must be 16-byte aligned", who);
  if (bias && !aligned(bias, 2)) return fail(WP_ERR_INVALID, "%s: bias must be 2-byte aligned", who);
  if (w_row_stride < d_in || w_row_stride % 8 != 0)
    return fail(WP_ERR_INVALID, "%s: weight row stride %lld must be >= d_in and a multiple of 8", who,
                (long long)w_row_stride);
  if (T < 1) return fail(WP_ERR_INVALID, "%s: x has no rows", who);
  if (e->plan_kind == 0) return fail(WP_ERR_STATE, "%s: no segment table (call build_seg_bounds first)", who);
  if (e->plan_T > T)
    return fail(WP_ERR_INVALID, "%s: segments reach token %lld but x has %lld rows", who, (long long)e->plan_T,
                (long long)T);
  // Decode-sized plans (16-token blocks) and whole 128-column K-slices and
  // 16-column output tiles only; the caller runs the linear and add_lora
  // otherwise.
  if (e->plan_bt > 16 || d_in % 128 != 0 || d_out % 16 != 0 || T > kSmallPlanTokens) return WP_NOT_HANDLED;
  DeviceGuard g(e->device);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  a.tiles = 1;
  a.ptok = e->ptok;
  a.part = e->part;
  a.consumed = e->consumed;
  a.spin_limit = e->spin_limit;
  a.trace = e->trace;
  a.trace_words = e->trace_words;
  a.plan = plan_view(e);
  a.n_slots = block_bound(e, num_loras);
  a.h = e->hbuf;
  a.ldh = rank;
  shrink_small_split(d_in, rank, &a);
  LinearArgs l{};
  l.w = w;
  l.ldw = w_row_stride;
  l.bias = bias;
  l.n_out = d_out;
  l.tokens = static_cast<int32_t>(T);
  l.groups = static_cast<int32_t>(ceil_div(T, 128));
  // K-ranges: about two GEMM workgroups per compute unit, whole K-slices,
  // within the partial buffer.
  const int64_t tiles = static_cast<int64_t>(l.groups) * (d_out / 16);
  if (tiles > kLinCounters) return WP_NOT_HANDLED;
  const int64_t slices = d_in / 128;
  int64_t splits = std::max<int64_t>(1, std::min<int64_t>(slices, (2 * static_cast<int64_t>(e->n_cu) + tiles / 2) / tiles));
  const uint64_t part_floats = static_cast<uint64_t>(kMaxChunks) * e->tok_cap * kMaxRank;
  while (splits > 1 && static_cast<uint64_t>(tiles) * splits * 128 * 16 > part_floats) --splits;
  if (static_cast<uint64_t>(tiles) * splits * 128 * 16 > part_floats) return WP_NOT_HANDLED;
  l.k_range = static_cast<int32_t>(ceil_div(slices, splits) * 128);
  l.splits = static_cast<int32_t>(ceil_div(d_in, l.k_range));
  l.gpart = e->spart;
  l.tile_cnt = e->lin_cnt;
  l.hflag = e->lin_flag;
  l.hcnt = e->lin_flag + e->block_cap;
  if (a.n_slots > e->block_cap) return fail(WP_ERR_CAPACITY, "%s: more block slots than the engine holds", who);
  WP_HIP(launch_linear(dtype == WP_DTYPE_BF16, a, l, stream));
  return WP_OK;
}

int wp_add_lora_nslice(wp_engine* e, void* y, const void* x, int32_t n_slices, const void* const* wa,
                       const int64_t* wa_stride0, const void* const* wb, const int64_t* wb_stride0,
                       const int32_t* out_features, const int32_t* y_col_offsets, int32_t num_loras, float scale,
                       int32_t rank, int32_t d_model, int64_t T, int64_t y_row_stride, int32_t dtype, void* stream) {
  return add_lora_impl(e, "add_lora_nslice", y, x, n_slices, wa, wa_stride0, num_loras, n_slices, wb, wb_stride0,
                       out_features, y_col_offsets, scale, rank, d_model, T, y_row_stride, dtype, stream);
}

int wp_shrink_expand(wp_engine* e, const void* X, void* Y, int32_t d_model, int32_t out_features, int32_t rank,
                     int64_t T, int64_t y_row_stride, int32_t y_col_offset, int32_t dtype, void* stream_) {
  if (!e) return fail(WP_ERR_INVALID, "shrink_expand: engine is NULL");
  if (e->plan_kind == 0 || e->plan_T > kSmallPlanTokens) {
    // Large plans: shrink() into the engine's H, then expand() from it (the
    // same checks and errors as the two calls).
    const int64_t hs = rank == 0 ? kMaxRank : rank;
    int rc = wp_shrink(e, X, e->hbuf, d_model, rank, T, hs, dtype, stream_);
    if (rc != WP_OK) return rc;
    return wp_expand(e, e->hbuf, Y, out_features, rank, T, hs, y_row_stride, y_col_offset, dtype, stream_);
  }
  if (rank != 0 && !rank_ok(rank)) return fail(WP_ERR_INVALID, "shrink_expand: unsupported rank (only 8/16/32/64)");
  int rc = check_io("shrink_expand", dtype, X, "X");
  if (rc != WP_OK) return rc;
  if (!aligned(Y, 8)) return fail(WP_ERR_INVALID, "shrink_expand: Y must be 8-byte aligned");
  if (d_model <= 0 || d_model % 8 != 0) return fail(WP_ERR_INVALID, "shrink_expand: d_model must be a positive multiple of 8");
  if (out_features <= 0 || out_features % 4 != 0)
    return fail(WP_ERR_INVALID, "shrink_expand: out_features must be a positive multiple of 4");
  if (y_col_offset < 0 || y_col_offset % 4 != 0 || y_row_stride % 4 != 0 || y_row_stride < y_col_offset + out_features)
    return fail(WP_ERR_INVALID, "shrink_expand: Y window [%d, %d) does not fit row stride %lld with 4-element alignment",
                y_col_offset, y_col_offset + out_features, (long long)y_row_stride);
  if (e->plan_T > T)
    return fail(WP_ERR_INVALID, "shrink_expand: segments reach token %lld but X has %lld rows", (long long)e->plan_T,
                (long long)T);
  if (e->plan_kind == 1) {
    for (size_t i = 0; i < e->plan_entry_ids.size(); ++i) {
      const Adapter& ad = e->adapters.at(e->plan_entry_ids[i]);
      if (ad.d != d_model || ad.o != out_features || (rank != 0 && ad.rank != rank) || ad.dtype != dtype)
        return fail(WP_ERR_INVALID, "shrink_expand: adapter %d is %d x %d, rank %d; the call is %d x %d, rank %d",
                    e->plan_entry_ids[i], ad.d, ad.o, ad.rank, d_model, out_features, rank);
    }
  }
  DeviceGuard g(e->device);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  ApplyArgs a = base_args(e, rank);
  a.x = X;
  a.ldx = d_model;
  a.y = Y;
  a.ldy = y_row_stride;
  a.d_model = d_model;
  if ((rc = table_weights(e, stream, &a.w)) != WP_OK) return rc;
  const int cols = expand_cols_per_workgroup();
  a.w.n_slices = 1;
  a.w.o_size[0] = out_features;
  a.w.y_off[0] = y_col_offset;
  a.w.oc_start[0] = 0;
  a.w.oc_start[1] = static_cast<int32_t>(ceil_div(out_features, cols));
  a.n_ochunks = a.w.oc_start[1];
  a.n_slots = block_bound(e, resolvable_ids(e, stream));
  fused_split(&a, rank, d_model, e->n_cu);
  WP_HIP(launch_fused(dtype == WP_DTYPE_BF16, a, stream));
  return WP_OK;
}

int wp_shrink_expand_slices(wp_engine* e, const void* X, void* Y, int32_t d_model, int32_t n_slices,
                            const int32_t* id_offsets, int32_t ids_per_layer, const int32_t* out_features,
                            const int32_t* y_col_offsets, int32_t rank, int64_t T, int64_t y_row_stride, int32_t dtype,
                            void* stream_) {
  if (!e) return fail(WP_ERR_INVALID, "shrink_expand_slices: engine is NULL");
  if (n_slices < 1 || n_slices > kMaxSlices || !id_offsets || !out_features || !y_col_offsets)
    return fail(WP_ERR_INVALID, "shrink_expand_slices: 1..%d slices with their ids, widths and offsets", kMaxSlices);
  if (e->plan_kind != 2)
    return fail(WP_ERR_STATE, "shrink_expand_slices: needs a build_seg_bounds table (a build_segments table resolves "
                              "its adapters when it is built)");
  if (ids_per_layer < 0) return fail(WP_ERR_INVALID, "shrink_expand_slices: negative ids_per_layer");
  for (int s = 0; s < n_slices; ++s) {
    if (id_offsets[s] < 0 || id_offsets[s] > e->table_cap)
      return fail(WP_ERR_INVALID, "shrink_expand_slices: slice %d id offset %d outside the adapter table", s,
                  id_offsets[s]);
    if (out_features[s] <= 0 || out_features[s] % 4 != 0 || y_col_offsets[s] < 0 || y_col_offsets[s] % 4 != 0 ||
        y_col_offsets[s] + out_features[s] > y_row_stride)
      return fail(WP_ERR_INVALID, "shrink_expand_slices: slice %d window [%d, %d) does not fit Y (row stride %lld, "
                                  "4-aligned)", s, y_col_offsets[s], y_col_offsets[s] + out_features[s],
                  (long long)y_row_stride);
  }
  if (e->plan_T > kSmallPlanTokens || n_slices == 1) {
    // Large plans (and a single slice): one shrink_expand per slice, each
    // on its layer's adapters.
    const int32_t off0 = e->entry_offset, cnt0 = e->entry_count;
    int rc = WP_OK;
    for (int s = 0; s < n_slices && rc == WP_OK; ++s) {
      e->entry_offset = id_offsets[s];
      e->entry_count = ids_per_layer;
      rc = wp_shrink_expand(e, X, Y, d_model, out_features[s], rank, T, y_row_stride, y_col_offsets[s], dtype, stream_);
    }
    e->entry_offset = off0;
    e->entry_count = cnt0;
    return rc;
  }
  if (rank != 0 && !rank_ok(rank)) return fail(WP_ERR_INVALID, "shrink_expand_slices: unsupported rank (only 8/16/32/64)");
  int rc = check_io("shrink_expand_slices", dtype, X, "X");
  if (rc != WP_OK) return rc;
  if (!aligned(Y, 8)) return fail(WP_ERR_INVALID, "shrink_expand_slices: Y must be 8-byte aligned");
  if (d_model <= 0 || d_model % 8 != 0)
    return fail(WP_ERR_INVALID, "shrink_expand_slices: d_model must be a positive multiple of 8");
  if (y_row_stride % 4 != 0) return fail(WP_ERR_INVALID, "shrink_expand_slices: Y row stride must be a multiple of 4");
  if (e->plan_T > T)
    return fail(WP_ERR_INVALID, "shrink_expand_slices: segments reach token %lld but X has %lld rows",
                (long long)e->plan_T, (long long)T);
  DeviceGuard g(e->device);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  ApplyArgs a = base_args(e, rank);
  a.x = X;
  a.ldx = d_model;
  a.y = Y;
  a.ldy = y_row_stride;
  a.d_model = d_model;
  if (!stream_capturing(stream) && (rc = apply_ready_slots(e, stream)) != WP_OK) return rc;
  a.w.mode = kTable;
  a.w.entries = e->dtable;
  int32_t max_off = 0;
  for (int s = 0; s < n_slices; ++s) max_off = std::max(max_off, id_offsets[s]);
  a.w.num_ids = std::max(0, e->table_cap - max_off);
  if (ids_per_layer > 0) a.w.num_ids = std::min(a.w.num_ids, ids_per_layer);
  a.w.n_a = n_slices;
  a.w.n_slices = n_slices;
  a.hs1 = rank == 0 ? kMaxRank : rank;
  a.hs = n_slices * a.hs1;
  a.pad_rank = rank == 0 ? 1 : 0;
  const int cols = expand_cols_per_workgroup();
  int oc = 0;
  for (int s = 0; s < n_slices; ++s) {
    a.w.entry_off[s] = id_offsets[s];
    a.w.o_size[s] = out_features[s];
    a.w.y_off[s] = y_col_offsets[s];
    a.w.oc_start[s] = oc;
    oc += static_cast<int>(ceil_div(out_features[s], cols));
  }
  a.w.oc_start[n_slices] = oc;
  a.n_ochunks = oc;
  // Blocks: bounded as for one layer's window (an id registered in any
  // slice's layer forms a block).
  const int64_t window = ids_per_layer > 0 ? ids_per_layer : static_cast<int64_t>(e->table_cap);
  a.n_slots = block_bound(e, call_ids(e, stream, static_cast<int64_t>(e->adapters.size()), window));
  fused_split(&a, rank, d_model, e->n_cu);
  WP_HIP(launch_fused(dtype == WP_DTYPE_BF16, a, stream));
  return WP_OK;
}

}  // extern "C"

// ============================================================================
// vLLM V1's LoRA ops (PunicaWrapperGPU.add_shrink / add_expand /
// add_lora_linear's bias) on the current plan and stacked weights.
// ============================================================================

namespace {

// Launch fields of a stacked-weight call that every V1 op shares.
ApplyArgs stacked_base(const wp_engine* e, int32_t rank, int32_t num_loras, float scale) {
  ApplyArgs a = base_args(e, rank);
  a.w.mode = kStacked;
  a.w.num_ids = num_loras;
  a.w.scale = scale;
  a.w.n_slices = 1;
  a.n_slots = block_bound(e, num_loras);
  return a;
}

int check_plan_for(const wp_engine* e, const char* who, int64_t T) {
  if (e->plan_kind == 0) return fail(WP_ERR_STATE, "%s: no segment table (call build_seg_bounds first)", who);
  if (e->plan_T > T)
    return fail(WP_ERR_INVALID, "%s: segments reach token %lld but the call has %lld rows", who, (long long)e->plan_T,
                (long long)T);
  return WP_OK;
}

}  // namespace

extern "C" {

int wp_lora_shrink(wp_engine* e, float* out, int64_t out_slice_stride, int64_t out_row_stride, const void* x,
                   int32_t n_slices, const void* const* wa, const int64_t* wa_stride0, int32_t num_loras, float scale,
                   int32_t rank, int32_t d_model, int64_t T, int32_t dtype, void* stream_) {
  const char* who = "lora_shrink";
  if (!e) return fail(WP_ERR_INVALID, "%s: engine is NULL", who);
  if (!rank_ok(rank)) return WP_NOT_HANDLED;
  int rc = check_io(who, dtype, x, "x");
  if (rc != WP_OK) return rc;
  if (!out || !aligned(out, 16)) return fail(WP_ERR_INVALID, "%s: the fp32 output must be 16-byte aligned", who);
  if (out_row_stride < rank || out_row_stride % 4 != 0 || out_slice_stride < 0 || out_slice_stride % 4 != 0)
    return fail(WP_ERR_INVALID, "%s: output rows of >= rank fp32 and strides that are multiples of 4", who);
  if (n_slices < 1 || n_slices > kMaxSlices || !wa || !wa_stride0)
    return fail(WP_ERR_INVALID, "%s: 1..%d slices, each with its lora_a", who, kMaxSlices);
  for (int s = 0; s < n_slices; ++s) {
    if ((rc = check_io(who, dtype, wa[s], "lora_a")) != WP_OK) return rc;
    if (!wa[s] || wa_stride0[s] % 8 != 0) return fail(WP_ERR_INVALID, "%s: lora_a stride must be a multiple of 8", who);
  }
  if (d_model <= 0 || d_model % 8 != 0) return fail(WP_ERR_INVALID, "%s: d_model must be a positive multiple of 8", who);
  if (num_loras <= 0) return fail(WP_ERR_INVALID, "%s: num_loras must be positive", who);
  if ((rc = check_plan_for(e, who, T)) != WP_OK) return rc;
  DeviceGuard g(e->device);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  for (int s = 0; s < n_slices; ++s) {
    ApplyArgs a = stacked_base(e, rank, num_loras, scale);
    a.x = x;
    a.ldx = d_model;
    a.d_model = d_model;
    a.w.a_base[0] = wa[s];
    a.w.a_stride[0] = wa_stride0[s];
    a.h = out + s * out_slice_stride;
    a.ldh = out_row_stride;
    a.h_f32 = 1;
    if (e->plan_bt <= 16) {
      shrink_small_split(d_model, rank, &a);
      a.red_first = 2 * static_cast<int64_t>(a.n_slots) <= static_cast<int64_t>(e->n_cu) * shrink_small_waves_per_simd() ? 1 : 0;
      WP_HIP(launch_shrink_small(dtype == WP_DTYPE_BF16, a, stream));
    } else {
      shrink_range_split(d_model, &a);
      a.part = e->spart;
      a.ptok = e->tok_cap;
      WP_HIP(launch_shrink(dtype == WP_DTYPE_BF16, a, stream));
    }
  }
  return WP_OK;
}

int wp_add_bias(wp_engine* e, void* y, int64_t y_row_stride, int32_t n_slices, const void* const* bias,
                const int64_t* bias_stride0, const int32_t* out_features, const int32_t* y_col_offsets,
                int32_t num_loras, int64_t T, int32_t dtype, void* stream_) {
  const char* who = "add_bias";
  if (!e) return fail(WP_ERR_INVALID, "%s: engine is NULL", who);
  int rc = check_io(who, dtype, nullptr, "");
  if (rc != WP_OK) return rc;
  if (!y || !aligned(y, 8) || y_row_stride % 4 != 0) return fail(WP_ERR_INVALID, "%s: y must be 8-byte aligned with a row stride that is a multiple of 4", who);
  if (n_slices < 1 || n_slices > kMaxSlices || !bias || !bias_stride0 || !out_features || !y_col_offsets)
    return fail(WP_ERR_INVALID, "%s: 1..%d slices with their biases, strides, widths and offsets", who, kMaxSlices);
  if (num_loras <= 0) return fail(WP_ERR_INVALID, "%s: num_loras must be positive", who);
  PrepArgs p{};
  bool any = false;
  for (int s = 0; s < n_slices; ++s) {
    if (out_features[s] <= 0 || out_features[s] % 4 != 0 || y_col_offsets[s] < 0 || y_col_offsets[s] % 4 != 0 ||
        y_col_offsets[s] + out_features[s] > y_row_stride)
      return fail(WP_ERR_INVALID, "%s: slice %d window [%d, %d) does not fit y (row stride %lld, 4-aligned)", who, s,
                  y_col_offsets[s], y_col_offsets[s] + out_features[s], (long long)y_row_stride);
    if (bias[s] != nullptr && (!aligned(bias[s], 8) || bias_stride0[s] % 4 != 0 || bias_stride0[s] < out_features[s]))
      return fail(WP_ERR_INVALID, "%s: slice %d bias rows must be 8-byte aligned, >= the slice width and 4-aligned apart",
                  who, s);
    p.o_size[s] = out_features[s];
    p.y_off[s] = y_col_offsets[s];
    p.bias[s] = bias[s];
    p.bias_stride[s] = bias_stride0[s];
    any = any || bias[s] != nullptr;
  }
  if ((rc = check_plan_for(e, who, T)) != WP_OK) return rc;
  if (!any) return WP_OK;
  DeviceGuard g(e->device);
  p.plan = plan_view(e);
  p.n_slots = block_bound(e, num_loras);
  p.n_slices = n_slices;
  p.num_ids = num_loras;
  p.y = y;
  p.ldy = y_row_stride;
  WP_HIP(launch_prep(dtype == WP_DTYPE_BF16, p, static_cast<hipStream_t>(stream_)));
  return WP_OK;
}

int wp_lora_expand(wp_engine* e, void* y, int64_t y_row_stride, const void* h, int32_t h_is_f32, int64_t h_slice_stride,
                   int64_t h_row_stride, int32_t n_slices, const void* const* wb, const int64_t* wb_stride0,
                   const int32_t* out_features, const int32_t* y_col_offsets, const void* const* bias,
                   const int64_t* bias_stride0, int32_t num_loras, int32_t rank, int64_t T, int32_t add_inputs,
                   int32_t dtype, void* stream_) {
  const char* who = "lora_expand";
  if (!e) return fail(WP_ERR_INVALID, "%s: engine is NULL", who);
  if (!rank_ok(rank)) return WP_NOT_HANDLED;
  int rc = check_io(who, dtype, nullptr, "");
  if (rc != WP_OK) return rc;
  if (!h || !aligned(h, h_is_f32 ? 4 : 2)) return fail(WP_ERR_INVALID, "%s: null or misaligned input", who);
  if (h_row_stride < rank || h_slice_stride < 0) return fail(WP_ERR_INVALID, "%s: input rows must hold rank values", who);
  if (!y || !aligned(y, 8) || y_row_stride % 4 != 0)
    return fail(WP_ERR_INVALID, "%s: y must be 8-byte aligned with a row stride that is a multiple of 4", who);
  if (n_slices < 1 || n_slices > kMaxSlices || !wb || !wb_stride0 || !out_features || !y_col_offsets)
    return fail(WP_ERR_INVALID, "%s: 1..%d slices with their lora_b, widths and offsets", who, kMaxSlices);
  if (num_loras <= 0) return fail(WP_ERR_INVALID, "%s: num_loras must be positive", who);
  if ((rc = check_plan_for(e, who, T)) != WP_OK) return rc;
  if (e->plan_T > e->tok_cap) return fail(WP_ERR_CAPACITY, "%s: the table reaches past the engine's H rows", who);
  PrepArgs p{};
  ApplyArgs a{};
  {
    a = stacked_base(e, rank, num_loras, 1.0f);
    a.h = e->hbuf;
    a.ldh = static_cast<int64_t>(n_slices) * rank;
    a.y = y;
    a.ldy = y_row_stride;
    a.hs1 = rank;
    a.hs = n_slices * rank;
    a.w.n_a = n_slices;  // slice s reads H columns [s * rank, (s + 1) * rank)
    a.w.n_slices = n_slices;
    const int cols = expand_cols_per_workgroup();
    int oc = 0;
    for (int s = 0; s < n_slices; ++s) {
      if ((rc = check_io(who, dtype, wb[s], "lora_b")) != WP_OK) return rc;
      if (!wb[s] || wb_stride0[s] % 8 != 0) return fail(WP_ERR_INVALID, "%s: lora_b stride must be a multiple of 8", who);
      if (out_features[s] <= 0 || out_features[s] % 4 != 0 || y_col_offsets[s] < 0 || y_col_offsets[s] % 4 != 0 ||
          y_col_offsets[s] + out_features[s] > y_row_stride)
        return fail(WP_ERR_INVALID, "%s: slice %d window [%d, %d) does not fit y (row stride %lld, 4-aligned)", who, s,
                    y_col_offsets[s], y_col_offsets[s] + out_features[s], (long long)y_row_stride);
      const void* bs = bias ? bias[s] : nullptr;
      if (bs != nullptr && (!bias_stride0 || !aligned(bs, 8) || bias_stride0[s] % 4 != 0 || bias_stride0[s] < out_features[s]))
        return fail(WP_ERR_INVALID, "%s: slice %d bias rows must be 8-byte aligned, >= the slice width and 4-aligned apart",
                    who, s);
      a.w.b_base[s] = wb[s];
      a.w.b_stride[s] = wb_stride0[s];
      a.w.o_size[s] = out_features[s];
      a.w.y_off[s] = y_col_offsets[s];
      a.w.oc_start[s] = oc;
      oc += static_cast<int>(ceil_div(out_features[s], cols));
      p.o_size[s] = out_features[s];
      p.y_off[s] = y_col_offsets[s];
      p.bias[s] = add_inputs ? bs : nullptr;
      p.bias_stride[s] = bs ? bias_stride0[s] : 0;
    }
    a.w.oc_start[n_slices] = oc;
    a.n_ochunks = oc;
  }
  DeviceGuard g(e->device);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  // The input rounded into the engine's H rows (vLLM's lora_expand casts an
  // fp32 input to the weights' type before the product), the windows zeroed
  // when the expand overwrites, the biases added when it adds.
  p.plan = plan_view(e);
  p.n_slots = a.n_slots;
  p.n_slices = n_slices;
  p.num_ids = num_loras;
  p.rank = rank;
  p.h_src = h;
  p.h_f32 = h_is_f32 ? 1 : 0;
  p.h_slice_stride = h_slice_stride;
  p.h_row_stride = h_row_stride;
  p.h_dst = e->hbuf;
  p.ldh_dst = n_slices * rank;
  p.y = y;
  p.ldy = y_row_stride;
  p.zero_y = add_inputs ? 0 : 1;
  WP_HIP(launch_prep(dtype == WP_DTYPE_BF16, p, stream));
  WP_HIP(launch_expand(dtype == WP_DTYPE_BF16, a, stream));
  return WP_OK;
}

int wp_barrier_probe(const uint32_t* salts, int32_t rounds, int32_t threads, int32_t workgroups, uint32_t* mismatches,
                     void* stream) {
  if (!salts || !mismatches || rounds < 1 || workgroups < 1 || (threads != 256 && threads != 1024))
    return fail(WP_ERR_INVALID, "barrier_probe: salts[rounds], a mismatch word, 256 or 1024 threads");
  WP_HIP(launch_barrier_probe(salts, rounds, threads, workgroups, mismatches, static_cast<hipStream_t>(stream)));
  return WP_OK;
}

int wp_handoff_probe(const void* a, int64_t a_bytes, const void* b, int64_t b_bytes, void* y, int64_t y_bytes,
                     uint32_t* counters, uint32_t* err, int32_t group, int32_t mode, int32_t workgroups, void* stream) {
  if (a_bytes < 0 || b_bytes < 0 || y_bytes < 0 || a_bytes % 16 || b_bytes % 16 || y_bytes % 16 ||
      (a_bytes && !aligned(a, 16)) || (b_bytes && !aligned(b, 16)) || (y_bytes && !aligned(y, 16)) || !counters ||
      !err || group < 1 || mode < 0 || mode > 3 || workgroups < 1 || (mode == 3 && group >= workgroups))
    return fail(WP_ERR_INVALID, "handoff_probe: 16-byte aligned buffers of multiples of 16 bytes, counters, an error "
                                "word, group >= 1, mode 0..3 (mode 3: group < workgroups)");
  HandoffProbe p{};
  p.a = a;
  p.a16 = static_cast<uint64_t>(a_bytes) / 16;
  p.b = b;
  p.b16 = static_cast<uint64_t>(b_bytes) / 16;
  p.y = y;
  p.y16 = static_cast<uint64_t>(y_bytes) / 16;
  p.counters = counters;
  p.err = err;
  p.group = group;
  p.mode = mode;
  p.spin_limit = kDefaultSpinLimit;
  WP_HIP(launch_handoff_probe(p, workgroups, static_cast<hipStream_t>(stream)));
  return WP_OK;
}

}  // extern "C"

// ============================================================================
// No-allocation entry point: build_seg_bounds + add_lora in one call, with the
// plan, the fp32 partials and the per-block counters in this library's static
// device array `scratch` (each GPU holds its own copy until the process ends).
// ============================================================================

namespace {

constexpr size_t align256(size_t v) { return (v + 255) & ~size_t(255); }
// Tokens per call: the reference's build_seg_bounds limit (bindings:165-166).
constexpr int kStaticTokens = kRefMaxSegments;
// Segments and blocks each hold at least one token.
constexpr int kStaticSegCap = kStaticTokens;
constexpr int kStaticBlockCap = kStaticTokens;
constexpr size_t kSOffHdr = 0;
constexpr size_t kSOffSeg = align256(kSOffHdr + sizeof(uint32_t) * kHdrWords);
constexpr size_t kSOffBlk = align256(kSOffSeg + sizeof(Segment) * kStaticSegCap);
constexpr size_t kSOffPerm = align256(kSOffBlk + sizeof(Block) * kStaticBlockCap);
constexpr size_t kSOffBperm = align256(kSOffPerm + sizeof(int32_t) * kStaticTokens);
constexpr size_t kSOffCons = align256(kSOffBperm + sizeof(int32_t) * kStaticBlockCap * kBlockTokens);
constexpr size_t kSOffPart = align256(kSOffCons + sizeof(uint32_t) * kStaticBlockCap * kCounterStride);
constexpr size_t kStaticBytes = align256(kSOffPart + sizeof(float) * kMaxChunks * kStaticTokens * kMaxRank);
static_assert(kStaticBytes == WP_STATIC_SCRATCH_BYTES, "WP_STATIC_SCRATCH_BYTES in the C header");

}  // namespace

// In host code this name is a host-side stand-in, not the device address:
// host code uses the per-device pointer from hipGetSymbolAddress only.
static __device__ __align__(256) unsigned char scratch[kStaticBytes];

namespace {

constexpr int kStaticMaxDevices = 64;

struct StaticDevice {
  char* ptr = nullptr;  // this device's copy of `scratch`
  int n_cu = 256;
};

std::mutex g_static_mu;
StaticDevice g_static[kStaticMaxDevices];

// The current device's scratch, set up on its first use: the symbol's device
// address, then the counters and plan header cleared and the partials filled
// with kPartialEmpty (the state every call leaves behind), synchronously.
int static_scratch(int dev, hipStream_t stream, StaticDevice** out) {
  std::lock_guard<std::mutex> lock(g_static_mu);
  StaticDevice& sd = g_static[dev];
  if (sd.ptr == nullptr) {
    if (stream_capturing(stream))
      return fail(WP_ERR_STATE, "add_lora_static: the first call on a device sets up its scratch and cannot be "
                                "captured; call it once before capturing");
    void* p = nullptr;
    WP_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    char* base = static_cast<char*>(p);
    WP_HIP(launch_fill_u32(reinterpret_cast<uint32_t*>(base), 0u, kSOffPart / 4, stream));
    WP_HIP(launch_fill_u32(reinterpret_cast<uint32_t*>(base + kSOffPart), kPartialEmpty, (kStaticBytes - kSOffPart) / 4,
                           stream));
    WP_HIP(hipStreamSynchronize(stream));
    int n_cu = 0;
    if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n_cu > 0)
      sd.n_cu = n_cu;
    sd.ptr = base;
  }
  *out = &sd;
  return WP_OK;
}

}  // namespace

extern "C" {

int wp_add_lora_static(void* y, const void* x, const void* idx, int32_t idx_is_int64, int64_t T, const void* wa,
                       int64_t wa_stride0, int32_t num_loras, int32_t n_slices, const void* const* wb,
                       const int64_t* wb_stride0, const int32_t* out_features, const int32_t* y_col_offsets,
                       float scale, int32_t rank, int32_t d_model, int64_t y_row_stride, int32_t dtype,
                       void* stream_) {
  ApplyArgs a{};
  int rc = stacked_call_args("add_lora_static", y, x, 1, &wa, &wa_stride0, num_loras, n_slices, wb, wb_stride0,
                             out_features, y_col_offsets, scale, rank, d_model, y_row_stride, dtype, &a);
  if (rc != WP_OK) return rc;
  if (T < 0) return fail(WP_ERR_INVALID, "add_lora_static: negative token count");
  if (T > kStaticTokens)
    return fail(WP_ERR_CAPACITY, "add_lora_static: %lld tokens exceed the static scratch's %d", (long long)T,
                kStaticTokens);
  if (T == 0) return WP_OK;
  if (!idx) return fail(WP_ERR_INVALID, "add_lora_static: null indices");
  int dev = 0;
  WP_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kStaticMaxDevices) return fail(WP_ERR_NO_DEVICE, "add_lora_static: device %d out of range", dev);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  StaticDevice* sd = nullptr;
  if ((rc = static_scratch(dev, stream, &sd)) != WP_OK) return rc;
  char* base = sd->ptr;
  PlanView v;
  v.header = reinterpret_cast<uint32_t*>(base + kSOffHdr);
  v.segments = reinterpret_cast<const Segment*>(base + kSOffSeg);
  v.blocks = reinterpret_cast<const Block*>(base + kSOffBlk);
  v.perm = reinterpret_cast<const int32_t*>(base + kSOffPerm);
  v.bperm = reinterpret_cast<const int32_t*>(base + kSOffBperm);
  const int bt = plan_block_tokens(T);
  // The plan build repairs the partials after a give-up, as an engine's does.
  Maint m{};
  m.part = reinterpret_cast<float*>(base + kSOffPart);
  m.part_words = (kStaticBytes - kSOffPart) / 4;
  m.consumed = reinterpret_cast<uint32_t*>(base + kSOffCons);
  m.consumed_words = (kSOffPart - kSOffCons) / 4;
  WP_HIP(launch_plan(idx, idx_is_int64 ? 1 : 0, static_cast<int>(T), v.header, reinterpret_cast<Segment*>(base + kSOffSeg),
                     reinterpret_cast<Block*>(base + kSOffBlk), reinterpret_cast<int32_t*>(base + kSOffPerm),
                     reinterpret_cast<int32_t*>(base + kSOffBperm), nullptr, kStaticSegCap, kStaticBlockCap, bt, &m,
                     stream));
  a.tiles = 1;
  a.ptok = kStaticTokens;
  a.part = reinterpret_cast<float*>(base + kSOffPart);
  a.consumed = reinterpret_cast<uint32_t*>(base + kSOffCons);
  a.plan = v;
  // Blocks: sum over adapters of ceil(n / 16) <= T / 16 + adapters, and <= T.
  a.n_slots = static_cast<int>(std::min<int64_t>(T, T / bt + std::min<int64_t>(num_loras, T)));
  fused_split(&a, rank, d_model, sd->n_cu);
  WP_HIP(launch_fused(dtype == WP_DTYPE_BF16, a, stream));
  return WP_OK;
}

int wp_read_static_errors(int32_t device, uint32_t* out, void* stream_) {
  if (!out) return fail(WP_ERR_INVALID, "read_static_errors: out is NULL");
  int ndev = 0;
  WP_HIP(hipGetDeviceCount(&ndev));
  if (device < 0 || device >= ndev || device >= kStaticMaxDevices)
    return fail(WP_ERR_NO_DEVICE, "read_static_errors: device %d out of range", device);
  DeviceGuard g(device);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  StaticDevice* sd = nullptr;
  const int rc = static_scratch(device, stream, &sd);
  if (rc != WP_OK) return rc;
  WP_HIP(launch_take_word(reinterpret_cast<uint32_t*>(sd->ptr + kSOffHdr) + kHdrErrors, out, stream));
  return WP_OK;
}

int wp_prefetch_adapters(wp_engine* e, const int32_t* adapter_ids, int32_t n, int32_t* slots_out) {
  if (!e || (n > 0 && (!adapter_ids || !slots_out))) return fail(WP_ERR_INVALID, "prefetch_adapters: null argument");
  DeviceGuard g(e->device);
  StageJobs jobs{};
  std::vector<int> job_slot;
  auto flush = [&]() -> int {
    if (jobs.n == 0) return WP_OK;
    WP_HIP(launch_stage_copies(jobs, e->pstream));
    for (int s : job_slot) WP_HIP(hipEventRecord(e->slots[s].ready, e->pstream));
    jobs.n = 0;
    job_slot.clear();
    return WP_OK;
  };
  for (int k = 0; k < n; ++k) {
    slots_out[k] = -1;
    auto it = e->adapters.find(adapter_ids[k]);
    if (it == e->adapters.end()) continue;
    // Existing slot for the id, else the first free one, else none
    // (reference: StagingBufferPool::acquire_slot, staging_buffer.h:62-73).
    // A slot that already holds the id holds its current weights
    // (registering the id again releases the slot): nothing is copied again.
    int s = find_slot(e, adapter_ids[k]);
    if (s >= 0) {
      slots_out[k] = s;
      continue;
    }
    for (size_t i = 0; i < e->slots.size(); ++i)
      if (e->slots[i].adapter < 0) {
        s = static_cast<int>(i);
        break;
      }
    if (s < 0) continue;
    Slot& sl = e->slots[s];
    const Adapter& ad = it->second;
    // The registration copy comes first (a device-side wait only if it has
    // not completed yet); buffers nobody reads any more.
    if (ad.copied && hipEventQuery(ad.copied) != hipSuccess) WP_HIP(hipStreamWaitEvent(e->pstream, ad.copied, 0));
    int rcb = take_slot_buffer(e, ad.a_bytes, &sl.A);
    if (rcb == WP_OK) rcb = take_slot_buffer(e, ad.b_bytes, &sl.B);
    if (rcb != WP_OK) return rcb;
    sl.a_bytes = ad.a_bytes;
    sl.b_bytes = ad.b_bytes;
    // One copy kernel for the batch (from the pinned host store, or D2D);
    // its last workgroup per slot publishes the slot for the next plan build.
    StageJob& job = jobs.job[jobs.n++];
    job.src_a = ad.hA ? ad.hA : ad.dA;
    job.dst_a = sl.A;
    job.a_bytes = ad.a_bytes;
    job.src_b = ad.hB ? ad.hB : ad.dB;
    job.dst_b = sl.B;
    job.b_bytes = ad.b_bytes;
    job.pub = e->pubs + s;
    job.pub_id = adapter_ids[k];
    job.pub_gen = ++sl.gen;
    job.pub_entry = staged_entry(ad, sl);
    job_slot.push_back(s);
    sl.adapter = adapter_ids[k];
    sl.issued = true;
    sl.applied = false;
    slots_out[k] = s;
    if (jobs.n == kMaxStageJobs) {
      const int rc = flush();
      if (rc != WP_OK) return rc;
    }
  }
  const int rc = flush();
  if (rc != WP_OK) return rc;
  sweep_graveyard(e, false);
  return WP_OK;
}

int wp_prefetch_adapter(wp_engine* e, int32_t adapter_id, int32_t* slot_out) {
  if (!e || !slot_out) return fail(WP_ERR_INVALID, "prefetch_adapter: null argument");
  return wp_prefetch_adapters(e, &adapter_id, 1, slot_out);
}

int wp_is_prefetch_ready(wp_engine* e, int32_t adapter_id, int32_t* ready) {
  if (!e || !ready) return fail(WP_ERR_INVALID, "is_prefetch_ready: null argument");
  const int s = find_slot(e, adapter_id);
  *ready = (s >= 0 && slot_ready(e->slots[s])) ? 1 : 0;
  return WP_OK;
}

int wp_release_prefetches(wp_engine* e, const int32_t* adapter_ids, int32_t n, void* stream_) {
  if (!e || (n > 0 && !adapter_ids)) return fail(WP_ERR_INVALID, "release_prefetches: null argument");
  std::vector<int> slot_ids;
  for (int k = 0; k < n; ++k) {
    const int s = find_slot(e, adapter_ids[k]);
    if (s >= 0) slot_ids.push_back(s);
  }
  if (slot_ids.empty()) return WP_OK;
  DeviceGuard g(e->device);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (stream_capturing(stream)) return fail(WP_ERR_STATE, "release_prefetch cannot run during graph capture");
  return release_slots_on(e, slot_ids.data(), static_cast<int>(slot_ids.size()), stream);
}

int wp_release_prefetch(wp_engine* e, int32_t adapter_id, void* stream) {
  if (!e) return fail(WP_ERR_INVALID, "release_prefetch: engine is NULL");
  return wp_release_prefetches(e, &adapter_id, 1, stream);
}

int wp_wait_prefetches(wp_engine* e, const int32_t* adapter_ids, int32_t n, void* stream_) {
  if (!e || (n > 0 && !adapter_ids)) return fail(WP_ERR_INVALID, "wait_prefetches: null argument");
  DeviceGuard g(e->device);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (stream_capturing(stream)) return fail(WP_ERR_STATE, "wait_prefetch cannot run during graph capture");
  int rc = WP_OK;
  for (int k = 0; k < n; ++k) {
    const int s = find_slot(e, adapter_ids[k]);
    if (s < 0 || !e->slots[s].issued) {
      rc = WP_NOT_HANDLED;
      continue;
    }
    if (hipEventQuery(e->slots[s].ready) != hipSuccess) WP_HIP(hipStreamWaitEvent(stream, e->slots[s].ready, 0));
  }
  return rc;
}

int wp_wait_prefetch(wp_engine* e, int32_t adapter_id, void* stream) {
  if (!e) return fail(WP_ERR_INVALID, "wait_prefetch: engine is NULL");
  return wp_wait_prefetches(e, &adapter_id, 1, stream);
}

int wp_set_trace(wp_engine* e, void* buffer, int64_t n_words) {
  if (!e) return fail(WP_ERR_INVALID, "set_trace: engine is NULL");
  if (!traced_build()) return fail(WP_ERR_STATE, "set_trace: this library was built without WP_TRACE");
  if (buffer != nullptr && (n_words <= 0 || !aligned(buffer, 8)))
    return fail(WP_ERR_INVALID, "set_trace: a device buffer of n_words 8-byte words");
  e->trace = static_cast<uint64_t*>(buffer);
  e->trace_words = buffer != nullptr ? n_words : 0;
  return WP_OK;
}

int wp_read_probe(wp_engine* e, const void* buffer, int64_t bytes, void* sink, void* stream) {
  if (!e) return fail(WP_ERR_INVALID, "read_probe: engine is NULL");
  if (bytes < 0 || bytes % 16 != 0 || (bytes > 0 && !aligned(buffer, 16)) || !sink || !aligned(sink, 16))
    return fail(WP_ERR_INVALID, "read_probe: a 16-byte aligned buffer of a multiple of 16 bytes and a 8 KiB sink");
  DeviceGuard g(e->device);
  WP_HIP(launch_read_probe(buffer, static_cast<size_t>(bytes), sink, 2 * e->n_cu, static_cast<hipStream_t>(stream)));
  return WP_OK;
}

int wp_set_spin_limit(wp_engine* e, uint32_t polls) {
  if (!e) return fail(WP_ERR_INVALID, "set_spin_limit: engine is NULL");
  e->spin_limit = polls == 0xFFFFFFFFu ? kDefaultSpinLimit : polls;
  return WP_OK;
}

}  // extern "C"
