// wp_device.h -- device-side helpers shared by the gfx950 kernels: vector
// types, MFMA and 16-byte load wrappers, device-coherent (sc1) loads and
// stores, adapter resolution, partial-word tests and the row-order Y tile
// helpers.  Everything sits in an anonymous namespace: each kernel source
// gets its own inlined copy.
#pragma once

#include <hip/hip_runtime.h>

#include "wp_apply.h"
#include "wp_sync.h"

namespace wp {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

template <typename T>
struct VecOf;
template <>
struct VecOf<__bf16> {
  using v8 = bf16x8;
  using v4 = bf16x4;
  using v2 = bf16x2;
};
template <>
struct VecOf<_Float16> {
  using v8 = f16x8;
  using v4 = f16x4;
  using v2 = f16x2;
};

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ typename VecOf<T>::v8 load8(const T* p) {
  return __builtin_bit_cast(typename VecOf<T>::v8, *reinterpret_cast<const u32x4*>(p));
}
// 16-byte load through the global (not the generic) address space: a
// generic load counts on both the vector-memory and the LDS counters, so a
// wait for LDS would also wait for it.
__device__ __forceinline__ u32x4 load16_global(const void* p) {
  return *reinterpret_cast<const __attribute__((address_space(1))) u32x4*>(reinterpret_cast<uintptr_t>(p));
}
template <typename T>
__device__ __forceinline__ typename VecOf<T>::v8 zero8() {
  return __builtin_bit_cast(typename VecOf<T>::v8, u32x4{0u, 0u, 0u, 0u});
}
template <typename T>
__device__ __forceinline__ f32x4 unpack4f(u32x2 q) {
  const auto v = __builtin_bit_cast(typename VecOf<T>::v4, q);
  return f32x4{static_cast<float>(v[0]), static_cast<float>(v[1]), static_cast<float>(v[2]), static_cast<float>(v[3])};
}
template <typename T>
__device__ __forceinline__ typename VecOf<T>::v4 round4(f32x4 v) {
  typename VecOf<T>::v4 o;
  o[0] = static_cast<T>(v[0]);
  o[1] = static_cast<T>(v[1]);
  o[2] = static_cast<T>(v[2]);
  o[3] = static_cast<T>(v[3]);
  return o;
}
template <typename T>
__device__ __forceinline__ void store4(T* p, f32x4 v) {
  *reinterpret_cast<u32x2*>(p) = __builtin_bit_cast(u32x2, round4<T>(v));
}
// Streaming store (nt): Y is written once per call and not read again by the
// call, so its lines need not stay dirty in L2 for the end-of-kernel writeback.
template <typename T>
__device__ __forceinline__ void store4_stream(T* p, f32x4 v) {
  __builtin_nontemporal_store(__builtin_bit_cast(u32x2, round4<T>(v)), reinterpret_cast<u32x2*>(p));
}

// Device-scope (sc1) 8-byte loads and stores: coherent across XCDs without
// cache maintenance.
__device__ __forceinline__ unsigned long long coherent_load8(const void* p) {
  return __hip_atomic_load(static_cast<const unsigned long long*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coherent_store8(void* p, unsigned long long v) {
  __hip_atomic_store(static_cast<unsigned long long*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ f32x4 coherent_load_f4(const float* p) {
  const u32x2 lo = __builtin_bit_cast(u32x2, coherent_load8(p));
  const u32x2 hi = __builtin_bit_cast(u32x2, coherent_load8(p + 2));
  return __builtin_bit_cast(f32x4, u32x4{lo[0], lo[1], hi[0], hi[1]});
}
__device__ __forceinline__ void coherent_store_f4(float* p, f32x4 v) {
  const u32x4 u = __builtin_bit_cast(u32x4, v);
  coherent_store8(p, __builtin_bit_cast(unsigned long long, u32x2{u[0], u[1]}));
  coherent_store8(p + 2, __builtin_bit_cast(unsigned long long, u32x2{u[2], u[3]}));
}
__device__ __forceinline__ unsigned atomic_load_u(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned atomic_add_u(uint32_t* p, unsigned v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void atomic_store_u(uint32_t* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until this wave's outstanding global loads, stores and atomics are
// acknowledged, which for sc1 stores means they are device-visible.
__device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ void flag_error(uint32_t* header, uint32_t bits) { atomicOr(&header[kHdrErrors], bits); }

// Traced builds (-DWP_TRACE, python -m adapterslotsplusplus_amd.build --trace):
// thread 0 of every workgroup records the 100 MHz real-time counter at the
// phase boundaries of the fused kernels, after waiting for wave 0's memory
// operations so that a stamp follows the data it names (which perturbs the
// timing a little).  Stamps: 0 entry, 1 plan loaded; shrink workgroups 2 first
// token tile's MFMAs done, 3 partials stored and acknowledged; expand
// workgroups 2 B and Y loaded, 3 gate open, 4 partials collected, 5 Y
// stored; shrink()'s block reducers (role 2) 4 H stored.  Word 7: role (1
// shrink, 2 expand or reducer) | block << 8.  shrink_kernel
// (role 3 | block << 8 | d-range << 32): 0 entry, 1 block resolved, 2 slice
// loop done, 3 partial stored and counted, 4 the last arriver's H stored;
// word 6: the wave's hardware ids (HW_ID low word, XCC id << 32).
// linear_kernel: shrink workgroups (role 1) as the fused ones; block reducers
// (role 4 | block << 8) 0 entry, 1 block resolved, 2 partials there, 3 H
// stored before the flag; GEMM workgroups (role 5 | tile << 8 | K-split <<
// 32) 0 entry, 1 K-range done, 2 partial stored, 3 counted, and the tile's
// last one 4 base summed and H flags seen, 5 barrier, 6 y stored.
#ifdef WP_TRACE
__device__ __forceinline__ void trace_stamp(const ApplyArgs& a, int i) {
  if (a.trace != nullptr && threadIdx.x == 0) {
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    a.trace[static_cast<size_t>(blockIdx.x) * kTraceWords + i] = wall_clock64();
  }
}
__device__ __forceinline__ void trace_tag(const ApplyArgs& a, uint64_t tag) {
  if (a.trace != nullptr && threadIdx.x == 0) a.trace[static_cast<size_t>(blockIdx.x) * kTraceWords + 7] = tag;
}
// HW_ID (register 4: wave, SIMD, CU, shader array, engine) and XCC_ID
// (register 20), read whole.
__device__ __forceinline__ void trace_hw(const ApplyArgs& a) {
  if (a.trace != nullptr && threadIdx.x == 0) {
    const uint32_t hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);
    const uint32_t xcc = __builtin_amdgcn_s_getreg((31 << 11) | 20);
    a.trace[static_cast<size_t>(blockIdx.x) * kTraceWords + 6] = hw | (static_cast<uint64_t>(xcc) << 32);
  }
}
#else
__device__ __forceinline__ void trace_stamp(const ApplyArgs&, int) {}
__device__ __forceinline__ void trace_tag(const ApplyArgs&, uint64_t) {}
__device__ __forceinline__ void trace_hw(const ApplyArgs&) {}
#endif

// A wait on partials that reached its bound: flagged (kErrSpin), and the
// partial buffer marked poisoned (kHdrPoison).  A shrink workgroup that was
// late may yet write its partial after the block's readers emptied the
// buffer, so later calls skip their work until the next plan build has
// refilled the buffer (nothing reads such a word as data).
__device__ __forceinline__ void give_up(uint32_t* header) {
  flag_error(header, kErrSpin);
  atomic_store_u(&header[kHdrPoison], 1u);
}
__device__ __forceinline__ bool poisoned(const uint32_t* header) { return atomic_load_u(&header[kHdrPoison]) != 0u; }

// A block's weights as the kernels see them.
// The adapter-table entry as two 16-byte loads (field by field, with a test
// between, the compiler issued three dependent loads).
__device__ __forceinline__ Entry load_entry(const Entry* p) {
  const u32x4 lo = load16_global(p);
  const u32x4 hi = load16_global(reinterpret_cast<const char*>(p) + 16);
  Entry e;
  e.a_ptr = static_cast<uint64_t>(lo[0]) | (static_cast<uint64_t>(lo[1]) << 32);
  e.b_ptr = static_cast<uint64_t>(lo[2]) | (static_cast<uint64_t>(lo[3]) << 32);
  e.alpha = __builtin_bit_cast(float, hi[0]);
  e.rank_dtype = static_cast<int32_t>(hi[1]);
  e.d_model = static_cast<int32_t>(hi[2]);
  e.out_features = static_cast<int32_t>(hi[3]);
  return e;
}

// wp_dtype code of the kernels' element type (adapter-table entries carry
// the dtype their weights were registered with).
template <typename T>
constexpr int32_t dtype_code();
template <>
constexpr int32_t dtype_code<_Float16>() { return 0; }
template <>
constexpr int32_t dtype_code<__bf16>() { return 1; }

template <typename T>
struct Resolved {
  const T* ptr = nullptr;
  float alpha = 0.f;
  int rank = 0;
  uint32_t err = 0;
};

// A block's adapter-table entry loaded ahead (Weights::a_base in table mode) and
// whether it may be used; passed by value so that it stays in registers.
struct PreEntry {
  Entry en;
  bool ok = false;
};

// A of A-slice sa (0 when every output slice shares one A).  TS: table mode
// with one adapter per slice (each slice's entries at its own offset; other
// table calls fold their one offset into a.w.entries).  pre: the block's
// entry already loaded (Weights::a_base in table mode, checked by the caller).
template <typename T, bool TS = false>
__device__ __forceinline__ Resolved<T> resolve_a(const ApplyArgs& a, const Block& blk, int sa = 0,
                                                 PreEntry pre = PreEntry{}) {
  Resolved<T> r;
  if (a.w.mode == kStacked) {
    if (blk.adapter_id < 0 || blk.adapter_id >= a.w.num_ids) {
      r.err = kErrIdRange;
      return r;
    }
    r.ptr = static_cast<const T*>(a.w.a_base[sa]) + static_cast<int64_t>(blk.adapter_id) * a.w.a_stride[sa];
    r.alpha = a.w.scale;
    r.rank = a.rank;
    return r;
  }
  if (blk.entry < 0 || blk.entry >= a.w.num_ids) {
    r.err = kErrUnregistered;
    return r;
  }
  const Entry en = !TS && pre.ok ? pre.en : load_entry(a.w.entries + (TS ? a.w.entry_off[sa] : 0) + blk.entry);
  const int32_t rank = entry_rank(en.rank_dtype);
  // One test over both halves, so that both loads go out before the wait.
  if ((en.a_ptr == 0) | (en.b_ptr == 0) | (rank <= 0)) {
    r.err = kErrUnregistered;
    return r;
  }
  if (en.d_model != a.d_model || (a.rank != 0 && rank != a.rank) || entry_dtype(en.rank_dtype) != dtype_code<T>()) {
    r.err = kErrShape;
    return r;
  }
  r.ptr = reinterpret_cast<const T*>(en.a_ptr);
  r.alpha = en.alpha;
  r.rank = rank;
  return r;
}

template <typename T, bool TS = false>
__device__ __forceinline__ Resolved<T> resolve_b(const ApplyArgs& a, const Block& blk, int slice,
                                                 PreEntry pre = PreEntry{}) {
  Resolved<T> r;
  if (a.w.mode == kStacked) {
    if (blk.adapter_id < 0 || blk.adapter_id >= a.w.num_ids) {
      r.err = kErrIdRange;
      return r;
    }
    r.ptr = static_cast<const T*>(a.w.b_base[slice]) + static_cast<int64_t>(blk.adapter_id) * a.w.b_stride[slice];
    r.alpha = a.w.scale;
    r.rank = a.rank;
    return r;
  }
  if (blk.entry < 0 || blk.entry >= a.w.num_ids) {
    r.err = kErrUnregistered;
    return r;
  }
  const Entry en =
      !TS && pre.ok ? pre.en : load_entry(a.w.entries + (TS ? a.w.entry_off[slice] : 0) + blk.entry);
  const int32_t rank = entry_rank(en.rank_dtype);
  // One test over both halves, so that both loads go out before the wait.
  if ((en.a_ptr == 0) | (en.b_ptr == 0) | (rank <= 0)) {
    r.err = kErrUnregistered;
    return r;
  }
  if (en.out_features != a.w.o_size[TS ? slice : 0] || (a.rank != 0 && rank != a.rank) ||
      (a.d_model != 0 && en.d_model != a.d_model) || entry_dtype(en.rank_dtype) != dtype_code<T>()) {
    r.err = kErrShape;
    return r;
  }
  r.ptr = reinterpret_cast<const T*>(en.b_ptr);
  r.alpha = en.alpha;
  r.rank = rank;
  return r;
}

// Token of row `tl` of block b (its block-padded list), or -1 past the block.
__device__ __forceinline__ int32_t block_token(const ApplyArgs& a, int b, int tl, int count) {
  return tl < count ? a.plan.bperm[static_cast<int64_t>(b) * kBlockTokens + tl] : -1;
}

__device__ __forceinline__ bool is_empty(float v) { return __builtin_bit_cast(uint32_t, v) == kPartialEmpty; }
__device__ __forceinline__ bool any_empty(f32x4 v) { return is_empty(v[0]) || is_empty(v[1]) || is_empty(v[2]) || is_empty(v[3]); }

// A lane's share of one 16-token x 64-column Y tile (the columns of its wave)
// in row order: rows lane/8 and lane/8 + 8, 16 bytes each at column 8*(lane%8).
// Eight lanes cover a 128-byte row, so every load and store moves whole
// lines; the MFMA layout (4 columns of one row per lane) is produced and
// consumed through the wave's LDS stage instead (1.6x the HBM rate of
// accessing Y in the MFMA layout directly, measured on MI355X).
struct YRows {
  u32x4 v[2];
};
// Elements per staged row: 64 + 4, so the 8-byte MFMA-layout accesses of 16
// rows fall in distinct banks (SQ_LDS_BANK_CONFLICT 0 on MI355X; 72 gave a
// two-way conflict).  Rows are then 8-byte aligned only: the row-order side
// moves its 16 bytes as two 8-byte halves.
constexpr int kStageStride = 68;

// A row-order 16-byte segment into / out of the stage, as two 8-byte halves.
template <typename T>
__device__ __forceinline__ void stage_put(T* p, u32x4 v) {
  reinterpret_cast<u32x2*>(p)[0] = u32x2{v[0], v[1]};
  reinterpret_cast<u32x2*>(p)[1] = u32x2{v[2], v[3]};
}
template <typename T>
__device__ __forceinline__ u32x4 stage_get(const T* p) {
  const u32x2 lo = reinterpret_cast<const u32x2*>(p)[0];
  const u32x2 hi = reinterpret_cast<const u32x2*>(p)[1];
  return u32x4{lo[0], lo[1], hi[0], hi[1]};
}

// Tokens of this lane's two rows, from `tok_row` (the token of row lane % 16).
__device__ __forceinline__ void yrows_tokens(int32_t tok_row, int32_t (&tok)[2]) {
  const int lane = threadIdx.x & 63;
  tok[0] = __shfl(tok_row, lane >> 3, 64);
  tok[1] = __shfl(tok_row, (lane >> 3) + 8, 64);
}

// Y is read once per call: non-temporal loads keep it from displacing the
// weights and X rows other workgroups still read from L2 (measured on
// MI355X: cfg2 step 1.40 -> 1.36 ms, cfg4 layer 226 -> 207 us; the same hint
// on X or A loads is slower).
template <typename T>
__device__ __forceinline__ YRows yrows_load(const ApplyArgs& a, int y_off, int ob, int o_size, const int32_t (&tok)[2]) {
  const int o = ob + (threadIdx.x & 7) * 8;
  const T* Y = static_cast<const T*>(a.y);
  YRows r;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    r.v[h] = u32x4{0u, 0u, 0u, 0u};
    if (tok[h] < 0) continue;
    const T* p = Y + static_cast<int64_t>(tok[h]) * a.ldy + y_off + o;
    if (o + 8 <= o_size) {
      r.v[h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    } else if (o + 4 <= o_size) {
      const u32x2 lo = *reinterpret_cast<const u32x2*>(p);
      r.v[h] = u32x4{lo[0], lo[1], 0u, 0u};
    }
  }
  return r;
}

template <typename T>
__device__ __forceinline__ void yrows_store(const ApplyArgs& a, int y_off, int ob, int o_size, const int32_t (&tok)[2],
                                            const YRows& r) {
  const int o = ob + (threadIdx.x & 7) * 8;
  T* Y = static_cast<T*>(a.y);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (tok[h] < 0) continue;
    T* p = Y + static_cast<int64_t>(tok[h]) * a.ldy + y_off + o;
    if (o + 8 <= o_size) {
      __builtin_nontemporal_store(r.v[h], reinterpret_cast<u32x4*>(p));
    } else if (o + 4 <= o_size) {
      __builtin_nontemporal_store(u32x2{r.v[h][0], r.v[h][1]}, reinterpret_cast<u32x2*>(p));
    }
  }
}

}  // namespace
}  // namespace wp
