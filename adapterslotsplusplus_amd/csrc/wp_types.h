// wp_types.h -- layouts shared by the host engine and the gfx950 kernels.
//
// Device-resident plan of one decode step (all in one engine-owned allocation):
//
//   header[16]    u32  num_segments, num_blocks, num_groups, num_valid_tokens, T, errors
//   segments[]    Segment  the exported run-length table, bit-exact with the
//                          reference's build_seg_bounds (warp_pipe_r32.cu:461-512)
//   blocks[]      Block    work units: <= kBlockTokens tokens of ONE adapter
//   perm[]        i32      token indices grouped by adapter (blocks index into it)
//   bperm[]       i32      the same tokens, kBlockTokens slots per block, so a
//                          workgroup loads its tokens without first reading
//                          its block descriptor
//
// The reference keeps its table in mapped pinned host memory that every kernel
// block reads over PCIe (warp_pipe_bindings.cpp:21-27).  Here it lives in HBM
// and is written either by the plan kernel or by a stream-ordered upload.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wp {

// Longest segment of the exported table: WP_MAX_SEGMENT_TOKENS,
// csrc/bridge/warp_pipe_metadata.h:22.
constexpr int kMaxSegmentTokens = 32;
// The reference's table capacity WP_MAX_SEGMENTS (warp_pipe_metadata.h:10);
// build_segments keeps it as its K limit (segment_builder.cpp:12-14).
constexpr int kRefMaxSegments = 256;
// Most tokens per work block, and the slot stride of bperm: one adapter's
// weights are streamed once per block.
constexpr int kBlockTokens = 64;
// Plans over at most this many tokens (decode-sized steps) cut blocks at 16
// tokens instead, one MFMA token tile: more, shorter blocks spread a hot
// adapter over more workgroups, and its repeated weight reads are served by
// the caches while the blocks run side by side.
constexpr int kSmallPlanTokens = 512;
inline constexpr int plan_block_tokens(int64_t T) { return T <= kSmallPlanTokens ? 16 : kBlockTokens; }
// Word pattern of an empty fp32 partial: a quiet NaN whose payload has bits
// set below bit 13.  Partials are fp32 sums of products of bf16/fp16 values;
// a NaN among them is the canonical quiet NaN or carries a payload widened
// from a 16-bit input (bits 0..12 clear), so no computed partial equals it.
constexpr uint32_t kPartialEmpty = 0x7FC2A5A5u;
// Stride (in 32-bit words) between two blocks' cross-workgroup counters: one
// 256-byte line each, so polls and increments of different blocks never share
// a line.
constexpr int kCounterStride = 64;
// Largest T the on-device plan builder takes in one workgroup (LDS-resident).
constexpr int kPlanMaxTokens = 8192;
// Output slices one add_lora call may expand into (q/k/v/...).
constexpr int kMaxSlices = 4;
// Largest rank.
constexpr int kMaxRank = 64;
// Shrink work split: each block's shrink runs on d-ranges x rank groups
// workgroups, each owning `rows` rank rows over one d-range.  shrink() uses
// 16-row groups (one MFMA tile: its four token tiles in flight take the
// registers a second one would need); the fused kernel uses 32-row groups
// (two tiles that share every X fragment), which halves its shrink
// workgroups so that a decode call's whole grid is resident at once.
// Mixed-rank calls use kMaxRank / rows groups.
constexpr int kShrinkRows = 16;
constexpr int kShrinkRowsFused = 32;
// Shrink workgroups per block a split aims for (at least 8 d-ranges).
inline constexpr int shrink_workgroups(int rows) { return rows == kShrinkRowsFused ? 8 : 16; }
inline constexpr int shrink_rank_groups(int rank, int rows) {
  return rank == 0 ? kMaxRank / rows : (rank + rows - 1) / rows;
}
// Most d-ranges of a split (the partial buffer's depth).
constexpr int kMaxChunks = 16;

enum HeaderWord : int {
  kHdrNumSegments = 0,
  kHdrNumBlocks = 1,
  kHdrNumGroups = 2,
  kHdrNumValid = 3,
  kHdrT = 4,
  kHdrErrors = 5,
  kHdrBlockTokens = 6,
  // Non-zero once a wait on partials gave up (kErrSpin): the partial buffer may
  // hold words a late shrink workgroup wrote after its block's readers
  // emptied it.  Kernels that use the buffer skip their work while it is set;
  // the next plan build (or wp_read_device_errors) refills the buffer with
  // kPartialEmpty, clears the counters and resets the word.
  kHdrPoison = 7,
  // Raised by every write into the id-indexed adapter table (the entry-write
  // kernel, a plan build's installed publications).
  kHdrTableVer = 8,
  // The table version a plan build copied its blocks' entries at (see
  // Weights::a_base); the copies hold while the two words are equal.  A
  // build without copies stores the complement of the current version, so
  // copies an earlier build left behind never count as current.
  kHdrPlanVer = 9,
  kHdrWords = 16
};

// Bits of header[kHdrErrors], set by kernels that had to skip work.
enum DeviceError : uint32_t {
  kErrIdRange = 1u,       // stacked weights: adapter id >= num_loras
  kErrUnregistered = 2u,  // adapter table: id not registered / not resident
  kErrShape = 4u,         // adapter rank / d / o differs from the call's
  kErrSpin = 8u,          // a fused call's expand side gave up waiting (later calls skip until the next plan)
  kErrCapacity = 16u      // shrink() / expand(): the plan has more blocks than the call's grid
                          // (the routing names adapter ids that are not registered)
};

struct Segment {  // 16 B; the reference descriptor's first three fields
  int32_t adapter_id;
  int32_t token_start;
  int32_t token_count;
  int32_t pad;
};

struct Block {  // 16 B
  int32_t adapter_id;
  int32_t first;  // offset into perm
  int32_t count;  // 1..kBlockTokens
  int32_t entry;  // index into the call's adapter-entry table
};

struct Entry {  // 32 B: one registered adapter as the kernels see it
  uint64_t a_ptr;  // [rank, d] (0: not usable)
  uint64_t b_ptr;  // [o, rank]
  float alpha;
  int32_t rank_dtype;  // rank in bits 0..15, the weights' dtype (wp_dtype) in bits 16..23
  int32_t d_model;
  int32_t out_features;
};
inline constexpr int32_t pack_rank_dtype(int32_t rank, int32_t dtype) { return rank | (dtype << 16); }
__host__ __device__ inline constexpr int32_t entry_rank(int32_t rank_dtype) { return rank_dtype & 0xffff; }
__host__ __device__ inline constexpr int32_t entry_dtype(int32_t rank_dtype) { return (rank_dtype >> 16) & 0xff; }

// A staging slot's publication, written by the prefetch stream once the
// slot's copy has landed, and read by the plan kernel at the start of every
// step (which then writes `entry` into the adapter table at `id`, so that
// every kernel of the step sees one table).  A sequence lock guards it: the
// writer makes `seq` odd, writes id, gen and entry, then makes it even
// again; a reader uses what it read only if it saw the same even `seq`
// before and after.  id < 0: the slot publishes nothing.  Every fill of a
// slot has a new generation `gen` (from 1 up); releasing the fill raises the
// slot's retired generation (a separate word, in the releasing stream's
// order) to it, and a publication counts only while its generation is above
// the retired one -- so a release and the slot's next publication, issued on
// different streams, may land in either order.
struct SlotPub {  // 48 B
  uint32_t seq;
  int32_t id;
  uint32_t copies;  // the copy job's finished workgroups (zero between jobs)
  uint32_t gen;
  Entry entry;
};

static_assert(sizeof(Segment) == 16, "Segment layout");
static_assert(sizeof(Block) == 16, "Block layout");
static_assert(sizeof(Entry) == 32, "Entry layout");

// How a block finds its adapter's weights.
enum WeightsMode : int32_t {
  kStacked = 0,  // A = a_base + id * a_stride (vLLM wa_t_all / wb_t_all)
  kTable = 1     // entries[block.entry]
};

struct Weights {
  int32_t mode;
  int32_t num_ids;  // stacked: L; table: number of entries
  // A matrices: 1 (shared by every slice: one H) or n_slices (slice s has
  // its own A, stacked mode only: one H per slice, side by side in a row).
  int32_t n_a;
  float scale;       // stacked: the call's scale
  // Stacked: each A slice's wa_t_all.  Table mode on a device-built plan at
  // entry offset 0: a_base[0] holds the plan build's copy of each block's
  // entries[block.entry] (Entry[block slots]), loaded with the block
  // descriptor instead of after it (one memory latency less before the first
  // weight load) and used while header[kHdrTableVer] == header[kHdrPlanVer];
  // null otherwise.  (A field of its own grows the kernel arguments, which
  // measured ~0.2 us more per launch.)
  const void* a_base[kMaxSlices];
  int64_t a_stride[kMaxSlices];  // elements
  const Entry* entries;
  // Table mode, one A per slice: slice s reads entries[entry_off[s] + block's
  // id] (a layer of a multi-layer store per slice); 0 otherwise.
  int32_t entry_off[kMaxSlices];
  int32_t n_slices;
  int32_t oc_start[kMaxSlices + 1];  // prefix of o-chunks per slice
  const void* b_base[kMaxSlices];
  int64_t b_stride[kMaxSlices];
  int32_t o_size[kMaxSlices];
  int32_t y_off[kMaxSlices];
};

// What a plan build (or the engine's maintenance launch) keeps in order
// besides the plan: it writes every ready slot publication into the adapter
// table, and after a give-up (kHdrPoison) it refills the partial buffer with
// kPartialEmpty and clears the per-block counters.
struct Maint {
  float* part;           // fused calls' partial buffer
  uint64_t part_words;
  uint32_t* consumed;    // per-block counters
  uint64_t consumed_words;
  const SlotPub* pubs;   // staging slot publications (n_pubs of them)
  const uint32_t* retired;  // per slot: the highest generation released
  int32_t n_pubs;
  int32_t table_cap;     // entries in `table`
  Entry* table;          // id-indexed adapter table
  uint64_t* trace;       // traced builds (WP_TRACE) only: 8 phase timestamps of the plan build, or null
};

struct PlanView {
  uint32_t* header;
  const Segment* segments;
  const Block* blocks;
  const int32_t* perm;
  const int32_t* bperm;
};

}  // namespace wp
