// wp_apply.hip -- grouped LoRA shrink + expand for gfx950 (MI355X), one launch per call.
//
// Work units are the blocks of the step plan (wp_plan.hip): up to 64 tokens
// that share ONE adapter, so the adapter's weights stream from HBM once per
// block and the per-block work is a small dense GEMM on the matrix cores
// (v_mfma_f32_16x16x32_{bf16,f16}, fp32 accumulation).  Weight rows are the
// MFMA "M" side and the block's tokens the "N" side: every operand fragment
// is one 16-byte load of 8 contiguous elements straight into VGPRs, and a
// lane's output fragment is 4 consecutive ranks / output columns.
//
// The fused kernel (reference: bgmv_shrink_dsak_kernel + bgmv_expand_dsak_kernel,
// csrc/kernels/warp_pipe_r32.cu:280-423) runs both halves of a call in ONE
// launch, which saves a ~1.7 us graph launch per call:
//
//   shrink workgroups   block b, d-range c (split-K).  The four waves split the
//                       d-range and reduce through LDS; the workgroup stores
//                       its fp32 partial H coherently and counts done[b].
//   expand workgroups   block b, 256 output columns.  They load their B rows
//                       and current Y, wait until done[b] counts every shrink
//                       workgroup of the block, sum the partials in a fixed
//                       order (so every workgroup, and every run, gets the
//                       same bits), apply alpha once and round H to the I/O
//                       dtype in LDS (reference :129, :360), then run the
//                       MFMAs and store Y = rn(Y + H.B^T) (reference :194).
//                       The last one of the block resets its counters.
//
// Summing the partials in every expand workgroup re-reads a few KB per
// workgroup but keeps the cross-workgroup chain to one hop: partial stores,
// their acknowledgement, one counter increment, the expand side's poll.
// Data crosses workgroups only through device-scope atomic loads and stores
// (sc1: coherent across the XCDs' L2s) ordered by s_waitcnt, and counters --
// never through __threadfence, whose L2 writeback + invalidate costs
// ~60-100 ns serialised over the device, nor through accumulation atomics.
//
// Grid: the shrink workgroups of every block slot, then the expand (or, for
// shrink(), one finishing) workgroups.  Those wait only on shrink workgroups,
// which have lower ids and never wait, so with in-order dispatch every wait
// ends; it is bounded anyway and reports kErrSpin if the bound is hit.  Slots
// past the device block count exit at once.
//
// The shrink-only and expand-only variants serve shrink()/expand() of the
// engine API: shrink's finishing workgroup writes the token-indexed H.
#include <hip/hip_runtime.h>

#include "wp_apply.h"

namespace wp {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct VecOf;
template <>
struct VecOf<__bf16> {
  using v8 = bf16x8;
  using v4 = bf16x4;
};
template <>
struct VecOf<_Float16> {
  using v8 = f16x8;
  using v4 = f16x4;
};

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kOT = 4;                  // output tiles per wave in expand
constexpr int kOC = kWaves * kOT * 16;  // output columns per expand workgroup (256)
constexpr int kShrinkKSteps = 2;        // 32-wide K-steps per wave per load batch
// Bound of the partials wait: polls of ~1 us each, so about 0.1 s.
constexpr unsigned kSpinLimit = 1u << 17;

enum Role : int { kFused = 0, kShrinkOnly = 1, kExpandOnly = 2 };

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

// A block's weights as the kernels see them.
template <typename T>
struct Resolved {
  const T* ptr = nullptr;
  float alpha = 0.f;
  int rank = 0;
  uint32_t err = 0;
};

template <typename T>
__device__ __forceinline__ Resolved<T> resolve_a(const ApplyArgs& a, const Block& blk) {
  Resolved<T> r;
  if (a.w.mode == kStacked) {
    if (blk.adapter_id < 0 || blk.adapter_id >= a.w.num_ids) {
      r.err = kErrIdRange;
      return r;
    }
    r.ptr = static_cast<const T*>(a.w.a_base) + static_cast<int64_t>(blk.adapter_id) * a.w.a_stride;
    r.alpha = a.w.scale;
    r.rank = a.rank;
    return r;
  }
  if (blk.entry < 0 || blk.entry >= a.w.num_ids) {
    r.err = kErrUnregistered;
    return r;
  }
  const Entry en = a.w.entries[blk.entry];
  if (en.a_ptr == 0 || en.b_ptr == 0) {
    r.err = kErrUnregistered;
    return r;
  }
  if (en.d_model != a.d_model || (a.rank != 0 && en.rank != a.rank)) {
    r.err = kErrShape;
    return r;
  }
  r.ptr = reinterpret_cast<const T*>(en.a_ptr);
  r.alpha = en.alpha;
  r.rank = en.rank;
  return r;
}

template <typename T>
__device__ __forceinline__ Resolved<T> resolve_b(const ApplyArgs& a, const Block& blk, int slice) {
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
  const Entry en = a.w.entries[blk.entry];
  if (en.a_ptr == 0 || en.b_ptr == 0) {
    r.err = kErrUnregistered;
    return r;
  }
  if (en.out_features != a.w.o_size[0] || (a.rank != 0 && en.rank != a.rank) ||
      (a.d_model != 0 && en.d_model != a.d_model)) {
    r.err = kErrShape;
    return r;
  }
  r.ptr = reinterpret_cast<const T*>(en.b_ptr);
  r.alpha = en.alpha;
  r.rank = en.rank;
  return r;
}

// Token of row `tl` of block b (its block-padded list), or -1 past the block.
__device__ __forceinline__ int32_t block_token(const ApplyArgs& a, int b, int tl, int count) {
  return tl < count ? a.plan.bperm[static_cast<int64_t>(b) * kBlockTokens + tl] : -1;
}

// ---------------------------------------------------------------- shrink ----

// Partial H of block b over d-range c, stored coherently to part[c].  Token
// tiles are processed one after another (the wave's A rows are re-read from
// L1 for tiles after the first); within a tile the loads of each batch of
// K-steps are issued before the MFMAs that consume them.  Every shrink
// workgroup then counts done[b], whether or not the block was computable.
template <typename T, int RANK>
__device__ __forceinline__ void shrink_body(const ApplyArgs& a, int b, int c, const Block& blk, int32_t tok0,
                                            const Resolved<T>& res, f32x4* s_red) {
  using V8 = typename VecOf<T>::v8;
  constexpr int RT = (RANK + 15) / 16;
  constexpr int KB = kShrinkKSteps;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = lane & 15;
  const int kq = (lane >> 4) * 8;
  if (res.ptr != nullptr) {
    const int d = a.d_model;
    const int kw_len = a.dc / kWaves;
    const int k_begin = c * a.dc + wave * kw_len;
    const int k_end = min(k_begin + kw_len, d);
    const int ntt = (blk.count + 15) >> 4;
    const T* X = static_cast<const T*>(a.x);
    const T* ar[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int r = rt * 16 + row;
      ar[rt] = r < RANK ? res.ptr + static_cast<int64_t>(r) * d : nullptr;
    }
    float* prow = a.part + (static_cast<int64_t>(c) * a.ptok + blk.first) * a.hs;
    for (int tt = 0; tt < ntt; ++tt) {
      const int32_t tok = tt == 0 ? tok0 : block_token(a, b, tt * 16 + row, blk.count);
      const T* xr = tok >= 0 ? X + static_cast<int64_t>(tok) * a.ldx : nullptr;
      f32x4 acc[RT];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) acc[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int k = k_begin; k < k_end; k += 32 * KB) {
        V8 af[KB][RT];
        V8 xf[KB];
#pragma unroll
        for (int st = 0; st < KB; ++st) {
          const int kk = k + st * 32 + kq;
          const bool in = kk < k_end;
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) af[st][rt] = (ar[rt] != nullptr && in) ? load8(ar[rt] + kk) : zero8<T>();
          xf[st] = (xr != nullptr && in) ? load8(xr + kk) : zero8<T>();
        }
#pragma unroll
        for (int st = 0; st < KB; ++st)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) acc[rt] = mfma16(af[st][rt], xf[st], acc[rt]);
      }
      // Reduce the four waves' d-slices through LDS (fixed order) and store
      // this tile's partial, coherently.
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) s_red[(wave * RT + rt) * 64 + lane] = acc[rt];
      __syncthreads();
      if (threadIdx.x < RT * 64) {
        const int ln = threadIdx.x & 63;
        const int rt = threadIdx.x >> 6;
        const int tl = tt * 16 + (ln & 15);
        const int r0 = rt * 16 + (ln >> 4) * 4;
        if (tl < blk.count && r0 < RANK) {
          f32x4 sum = s_red[(0 * RT + rt) * 64 + ln];
#pragma unroll
          for (int w = 1; w < kWaves; ++w) sum += s_red[(w * RT + rt) * 64 + ln];
          coherent_store_f4(prow + static_cast<int64_t>(tl) * a.hs + r0, sum);
        }
      }
      __syncthreads();
    }
  }
  // Publish: every wave's stores are acknowledged before the count.
  wait_vm();
  __syncthreads();
  if (threadIdx.x == 0) atomic_add_u(&a.done[b * kCounterStride], 1u);
}

// ---------------------------------------------------------------- reduce ----

// Waits (thread 0 polls, bounded) until all shrink workgroups of block b
// have published their partials.  Returns false after kErrSpin.
__device__ __forceinline__ bool wait_partials(const ApplyArgs& a, int b, int* s_flag) {
  if (threadIdx.x == 0) {
    int ok = 1;
    unsigned spins = 0;
    const unsigned need = static_cast<unsigned>(a.n_chunks);
    while (atomic_load_u(&a.done[b * kCounterStride]) < need) {
      __builtin_amdgcn_s_sleep(8);
      if (++spins > kSpinLimit) {
        ok = 0;
        flag_error(a.plan.header, kErrSpin);
        break;
      }
    }
    *s_flag = ok;
  }
  __syncthreads();
  return *s_flag != 0;
}

// H of block b: rn(alpha * sum_c part[c]) for its count x RANK values.  P
// threads share one 4-wide unit (P = 2 when there are more than 8 chunks):
// sub-sum s takes chunks s, s+P, ... in order, and the sub-sums are added in
// order s = 0..P-1, so every workgroup that reduces the block gets the same
// bits.  Each thread issues its (at most 8) loads back to back, unpredicated:
// a load past the last chunk re-reads the last chunk and is discarded.
// emit(j, r0, v4) receives each unit.
template <int RANK, typename Emit>
__device__ __forceinline__ void reduce_partials(const ApplyArgs& a, const Block& blk, float alpha, f32x4* s_tmp,
                                                Emit emit) {
  constexpr int R4 = RANK / 4;
  const int n_units = blk.count * R4;
  const int nch = a.n_chunks;
  const int P = nch > 8 ? 2 : 1;
  // Byte offsets from a uniform base: the workspace keeps them below 2^32.
  const uint32_t cstride = static_cast<uint32_t>(a.ptok) * static_cast<uint32_t>(a.hs) * 4u;
  const char* pbase = reinterpret_cast<const char*>(a.part + static_cast<int64_t>(blk.first) * a.hs);
  const int total = n_units * P;
  for (int t0 = 0; t0 < total; t0 += kThreads) {
    const int t = t0 + static_cast<int>(threadIdx.x);
    const int u = t / P;
    const int s = t - u * P;
    const int j = u / R4;
    const int r0 = (u - j * R4) * 4;
    f32x4 sum{0.f, 0.f, 0.f, 0.f};
    if (t < total) {
      const uint32_t o0 = static_cast<uint32_t>(j * a.hs + r0) * 4u;
      f32x4 v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int cc = min(s + i * P, nch - 1);
        v[i] = coherent_load_f4(reinterpret_cast<const float*>(pbase + (o0 + static_cast<uint32_t>(cc) * cstride)));
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (s + i * P < nch) sum += v[i];
    }
    if (P > 1) {
      s_tmp[threadIdx.x] = sum;
      __syncthreads();
      if (t < total && s == 0) sum += s_tmp[threadIdx.x + 1];
      __syncthreads();
    }
    if (t < total && s == 0) emit(j, r0, sum * alpha);
  }
}

// ---------------------------------------------------------------- expand ----

// Row stride (elements) of the block's H in LDS: RANK plus 8 to spread banks.
template <int RANK>
constexpr int lds_h_stride() { return RANK + 8; }

template <typename T, int RANK, int ROLE>
__device__ __forceinline__ void expand_body(const ApplyArgs& a, int b, const Block& blk, int32_t tok0,
                                            const Resolved<T>& res, int o_first, int o_size, int y_off,
                                            T* s_h, f32x4* s_tmp, int* s_flag) {
  using V8 = typename VecOf<T>::v8;
  constexpr int KS = (RANK + 31) / 32;
  constexpr bool kFused_ = ROLE == kFused;
  constexpr int HS = lds_h_stride<RANK>();
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = lane & 15;
  const int kq = (lane >> 4) * 8;
  const int oq = (lane >> 4) * 4;
  const int ob = o_first + wave * (kOT * 16);
  const int ntt = (blk.count + 15) >> 4;
  T* Y = static_cast<T*>(a.y);
  const bool ok = res.ptr != nullptr;

  // Issued before the wait: this wave's 64 rows of B and token tile 0 of Y
  // (kept packed until the MFMAs, to spare registers during the reduction).
  V8 bf[kOT][KS];
  u32x2 yq[kOT];
  f32x4 acc[kOT];
#pragma unroll
  for (int ot = 0; ot < kOT; ++ot) {
    const int o = ob + ot * 16 + row;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int k = ks * 32 + kq;
      bf[ot][ks] = (ok && o < o_size && k < RANK) ? load8(res.ptr + static_cast<int64_t>(o) * RANK + k) : zero8<T>();
    }
  }
  T* yrow0 = (ok && tok0 >= 0) ? Y + static_cast<int64_t>(tok0) * a.ldy + y_off : nullptr;
#pragma unroll
  for (int ot = 0; ot < kOT; ++ot) {
    const int o = ob + ot * 16 + oq;
    yq[ot] = (yrow0 != nullptr && o < o_size) ? *reinterpret_cast<const u32x2*>(yrow0 + o) : u32x2{0u, 0u};
  }

  bool go = ok;
  if constexpr (kFused_) {
    // Every expand workgroup waits, even one that cannot compute, so that the
    // last one to finish may reset the block's counters.
    const bool arrived = wait_partials(a, b, s_flag);
    go = go && arrived;
    if (go) {
      reduce_partials<RANK>(a, blk, res.alpha, s_tmp, [&](int j, int r0, f32x4 v) {
        *reinterpret_cast<typename VecOf<T>::v4*>(s_h + j * HS + r0) = round4<T>(v);
      });
    }
    __syncthreads();
  }
  if (go) {
    for (int tt = 0; tt < ntt; ++tt) {
      const int32_t tok = tt == 0 ? tok0 : block_token(a, b, tt * 16 + row, blk.count);
      T* yrow = (tok >= 0) ? Y + static_cast<int64_t>(tok) * a.ldy + y_off : nullptr;
      if (tt > 0) {
#pragma unroll
        for (int ot = 0; ot < kOT; ++ot) {
          const int o = ob + ot * 16 + oq;
          yq[ot] = (yrow != nullptr && o < o_size) ? *reinterpret_cast<const u32x2*>(yrow + o) : u32x2{0u, 0u};
        }
      }
#pragma unroll
      for (int ot = 0; ot < kOT; ++ot) acc[ot] = unpack4f<T>(yq[ot]);
      V8 hf[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int k = ks * 32 + kq;
        if (tok < 0 || k >= RANK) {
          hf[ks] = zero8<T>();
        } else if constexpr (kFused_) {
          hf[ks] = __builtin_bit_cast(V8, *reinterpret_cast<const u32x4*>(s_h + (tt * 16 + row) * HS + k));
        } else {
          hf[ks] = load8(static_cast<const T*>(a.h) + static_cast<int64_t>(tok) * a.ldh + k);
        }
      }
#pragma unroll
      for (int ot = 0; ot < kOT; ++ot)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) acc[ot] = mfma16(bf[ot][ks], hf[ks], acc[ot]);
#pragma unroll
      for (int ot = 0; ot < kOT; ++ot) {
        const int o = ob + ot * 16 + oq;
        if (yrow != nullptr && o < o_size) store4(yrow + o, acc[ot]);
      }
    }
  }

  if constexpr (kFused_) {
    // The last expand workgroup of the block resets its counters; every
    // expand workgroup has passed its wait by then, and every shrink
    // workgroup has counted.
    if (threadIdx.x == 0) {
      if (atomic_add_u(&a.consumed[b * kCounterStride], 1u) == static_cast<unsigned>(a.n_ochunks - 1)) {
        atomic_store_u(&a.consumed[b * kCounterStride], 0u);
        atomic_store_u(&a.done[b * kCounterStride], 0u);
      }
    }
  }
}

// shrink(): one workgroup per block reduces the partials into H[token].
template <typename T, int RANK>
__device__ __forceinline__ void finish_body(const ApplyArgs& a, int b, const Block& blk, const Resolved<T>& res,
                                            f32x4* s_tmp, int* s_flag) {
  const bool arrived = wait_partials(a, b, s_flag);
  if (arrived && res.ptr != nullptr) {
    T* H = static_cast<T*>(a.h);
    reduce_partials<RANK>(a, blk, res.alpha, s_tmp, [&](int j, int r0, f32x4 v) {
      store4(H + static_cast<int64_t>(block_token(a, b, j, blk.count)) * a.ldh + r0, v);
    });
  }
  if (threadIdx.x == 0) atomic_store_u(&a.done[b * kCounterStride], 0u);
}

// ---------------------------------------------------------------- kernels ----

// Occupancy target: rank 64 and mixed ranks need the most registers and run
// at 5 waves per SIMD; for ranks up to 32 the fused kernel (B and Y held
// across the partials' reduction) runs at 6 (<= 80 VGPRs), shrink() and
// expand() at 8 (<= 64 VGPRs).
template <int RANK, int ROLE>
constexpr int waves_per_simd() { return (RANK == 0 || RANK == 64) ? 5 : (ROLE == kFused ? 6 : 8); }

// LDS of one workgroup: shrink's cross-wave tiles, or expand's block H plus
// the reduction's exchange buffer.
template <typename T, int RANK>
struct alignas(16) SharedMem {
  static constexpr int RR = RANK == 0 ? kMaxRank : RANK;
  static constexpr int RT = (RR + 15) / 16;
  static constexpr int kRed = kWaves * RT * 64;                        // f32x4
  static constexpr int kH = (kBlockTokens * (RR + 8) * 2 + 15) / 16;   // f32x4 worth of T
  static constexpr int kExp = kH + kThreads;
  f32x4 buf[kRed > kExp ? kRed : kExp];
};

template <typename T, int RANK, int ROLE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(waves_per_simd<RANK, ROLE>())))
void apply_kernel(ApplyArgs a) {
  using SM = SharedMem<T, RANK>;
  __shared__ SM smem;
  __shared__ int s_flag;
  f32x4* s_red = smem.buf;
  T* s_h = reinterpret_cast<T*>(smem.buf);
  f32x4* s_tmp = smem.buf + SM::kH;
  const int S = ROLE == kExpandOnly ? 0 : a.n_slots * a.n_chunks;
  const int per_block = ROLE == kShrinkOnly ? 1 : a.n_ochunks;
  const int wg = static_cast<int>(blockIdx.x);
  const bool shrink_role = wg < S;
  int b, part;
  if (shrink_role) {
    b = wg / a.n_chunks;
    part = wg - b * a.n_chunks;
  } else {
    const int e = wg - S;
    b = e / per_block;
    part = e - b * per_block;
  }
  // Independent loads: block count, block descriptor, this lane's first token.
  const int n_blocks = static_cast<int>(a.plan.header[kHdrNumBlocks]);
  const Block blk = a.plan.blocks[b];
  const int row = threadIdx.x & 15;
  const int32_t tok0 = a.plan.bperm[static_cast<int64_t>(b) * kBlockTokens + row];
  if (b >= n_blocks) return;
  const int32_t t0 = row < blk.count ? tok0 : -1;

  if (shrink_role || ROLE == kShrinkOnly) {
    const Resolved<T> res = resolve_a<T>(a, blk);
    if (shrink_role) {
      if (res.err != 0 && part == 0 && threadIdx.x == 0) flag_error(a.plan.header, res.err);
      if constexpr (RANK != 0) {
        shrink_body<T, RANK>(a, b, part, blk, t0, res, s_red);
      } else {
        switch (res.rank) {
          case 16: shrink_body<T, 16>(a, b, part, blk, t0, res, s_red); break;
          case 32: shrink_body<T, 32>(a, b, part, blk, t0, res, s_red); break;
          case 64: shrink_body<T, 64>(a, b, part, blk, t0, res, s_red); break;
          default: shrink_body<T, 8>(a, b, part, blk, t0, res, s_red); break;
        }
      }
    } else if constexpr (ROLE == kShrinkOnly) {
      if constexpr (RANK != 0) {
        finish_body<T, RANK>(a, b, blk, res, s_tmp, &s_flag);
      } else {
        switch (res.rank) {
          case 16: finish_body<T, 16>(a, b, blk, res, s_tmp, &s_flag); break;
          case 32: finish_body<T, 32>(a, b, blk, res, s_tmp, &s_flag); break;
          case 64: finish_body<T, 64>(a, b, blk, res, s_tmp, &s_flag); break;
          default: finish_body<T, 8>(a, b, blk, res, s_tmp, &s_flag); break;
        }
      }
    }
    return;
  }
  if constexpr (ROLE != kShrinkOnly) {
    int s = 0;
    while (s + 1 < a.w.n_slices && part >= a.w.oc_start[s + 1]) ++s;
    const int o_first = (part - a.w.oc_start[s]) * kOC;
    const Resolved<T> res = resolve_b<T>(a, blk, s);
    if (res.err != 0 && part == 0 && threadIdx.x == 0) flag_error(a.plan.header, res.err);
    const int o_size = a.w.o_size[s];
    const int y_off = a.w.y_off[s];
    if constexpr (RANK != 0) {
      expand_body<T, RANK, ROLE>(a, b, blk, t0, res, o_first, o_size, y_off, s_h, s_tmp, &s_flag);
    } else {
      switch (res.rank) {
        case 16: expand_body<T, 16, ROLE>(a, b, blk, t0, res, o_first, o_size, y_off, s_h, s_tmp, &s_flag); break;
        case 32: expand_body<T, 32, ROLE>(a, b, blk, t0, res, o_first, o_size, y_off, s_h, s_tmp, &s_flag); break;
        case 64: expand_body<T, 64, ROLE>(a, b, blk, t0, res, o_first, o_size, y_off, s_h, s_tmp, &s_flag); break;
        default: expand_body<T, 8, ROLE>(a, b, blk, t0, res, o_first, o_size, y_off, s_h, s_tmp, &s_flag); break;
      }
    }
  }
}

template <typename T, int ROLE>
hipError_t launch_rank(const ApplyArgs& a, hipStream_t stream) {
  const int64_t S = ROLE == kExpandOnly ? 0 : static_cast<int64_t>(a.n_slots) * a.n_chunks;
  const int64_t E = static_cast<int64_t>(a.n_slots) * (ROLE == kShrinkOnly ? 1 : a.n_ochunks);
  const int64_t n = S + E;
  if (n <= 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(n));
  switch (a.rank) {
    case 0: apply_kernel<T, 0, ROLE><<<grid, kThreads, 0, stream>>>(a); break;
    case 8: apply_kernel<T, 8, ROLE><<<grid, kThreads, 0, stream>>>(a); break;
    case 16: apply_kernel<T, 16, ROLE><<<grid, kThreads, 0, stream>>>(a); break;
    case 32: apply_kernel<T, 32, ROLE><<<grid, kThreads, 0, stream>>>(a); break;
    case 64: apply_kernel<T, 64, ROLE><<<grid, kThreads, 0, stream>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int ROLE>
hipError_t launch_role(int dtype_bf16, const ApplyArgs& a, hipStream_t stream) {
  return dtype_bf16 ? launch_rank<__bf16, ROLE>(a, stream) : launch_rank<_Float16, ROLE>(a, stream);
}

}  // namespace

int expand_cols_per_workgroup() { return kOC; }

hipError_t launch_fused(int dtype_bf16, const ApplyArgs& a, hipStream_t stream) {
  return launch_role<kFused>(dtype_bf16, a, stream);
}
hipError_t launch_shrink(int dtype_bf16, const ApplyArgs& a, hipStream_t stream) {
  return launch_role<kShrinkOnly>(dtype_bf16, a, stream);
}
hipError_t launch_expand(int dtype_bf16, const ApplyArgs& a, hipStream_t stream) {
  return launch_role<kExpandOnly>(dtype_bf16, a, stream);
}

}  // namespace wp
