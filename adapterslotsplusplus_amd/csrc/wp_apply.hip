// wp_apply.hip -- grouped LoRA shrink and expand for gfx950 (MI355X).
//
// Both kernels run on the by-adapter blocks of the step plan (wp_plan.hip):
// a block is up to 64 tokens that share ONE adapter, so the adapter's weights
// are streamed once per block and the per-block work is a small dense GEMM.
// That GEMM runs on the matrix cores (v_mfma_f32_16x16x32_{bf16,f16}, fp32
// accumulation): the weight rows are the MFMA "M" side (16 rows per tile) and
// the block's tokens the "N" side, so every operand fragment is one 16-byte
// global load of 8 contiguous elements straight from HBM into VGPRs, and each
// lane's output fragment is 4 consecutive ranks / output columns.
//
// shrink  (reference: csrc/kernels/warp_pipe_r32.cu:56-132, :280-363 and
//          warp_pipe_rgen.cuh:42-135)
//   grid = max_blocks x n_chunks workgroups of 256 threads.  Workgroup (b, c)
//   covers d-range [c*dc, (c+1)*dc) of block b; its 4 waves split that range,
//   reduce through LDS, and store an fp32 partial H.  The last workgroup of a
//   block to arrive (device-scope counter, threadfence release/acquire) sums
//   the n_chunks partials in fixed chunk order -- the result is deterministic --
//   applies alpha once and rounds H to the I/O dtype (reference :129, :360),
//   then resets the counter for the next launch.  No memset, no host sync.
//
// expand  (reference: warp_pipe_r32.cu:141-200, :365-423, rgen.cuh:137-189)
//   grid = max_blocks x n_ochunks workgroups; workgroup (b, oc) produces 256
//   output columns (64 per wave, 4 MFMA tiles) for the tokens of block b:
//   Y = rn(Y + H . B^T) (reference :194), with up to 4 output slices, each with
//   its own B and column offset into a wider Y (packed q/k/v).
//
// Grids are sized on the host from an upper bound on the block count (capped;
// workgroups loop over blocks with a stride) and read the real count from the
// device plan, so a call is graph-capturable with fixed launch parameters
// while the routing changes between replays.
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
constexpr int kTT = kBlockTokens / 16;  // token tiles per block
constexpr int kOT = 4;                  // output tiles per wave in expand
constexpr int kOC = kWaves * kOT * 16;  // output columns per expand workgroup (256)

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
__device__ __forceinline__ f32x4 load4f(const T* p) {
  const auto v = __builtin_bit_cast(typename VecOf<T>::v4, *reinterpret_cast<const u32x2*>(p));
  return f32x4{static_cast<float>(v[0]), static_cast<float>(v[1]), static_cast<float>(v[2]), static_cast<float>(v[3])};
}
template <typename T>
__device__ __forceinline__ void store4(T* p, f32x4 v) {
  typename VecOf<T>::v4 o;
  o[0] = static_cast<T>(v[0]);
  o[1] = static_cast<T>(v[1]);
  o[2] = static_cast<T>(v[2]);
  o[3] = static_cast<T>(v[3]);
  *reinterpret_cast<u32x2*>(p) = __builtin_bit_cast(u32x2, o);
}

__device__ __forceinline__ void flag_error(uint32_t* header, uint32_t bits) {
  atomicOr(&header[kHdrErrors], bits);
}

// Resolves the shrink weights of a block.  rank_call = 0: any rank (mixed).
template <typename T>
__device__ __forceinline__ bool resolve_a(const ApplyArgs& a, const Block& blk, const T*& A, float& alpha, int& rank,
                                          uint32_t& err) {
  if (a.w.mode == kStacked) {
    if (blk.adapter_id < 0 || blk.adapter_id >= a.w.num_ids) {
      err = kErrIdRange;
      return false;
    }
    A = static_cast<const T*>(a.w.a_base) + static_cast<int64_t>(blk.adapter_id) * a.w.a_stride;
    alpha = a.w.scale;
    rank = a.rank;
    return true;
  }
  if (blk.entry < 0 || blk.entry >= a.w.num_ids) {
    err = kErrUnregistered;
    return false;
  }
  const Entry en = a.w.entries[blk.entry];
  if (en.a_ptr == 0) {
    err = kErrUnregistered;
    return false;
  }
  if (en.d_model != a.d_model || (a.rank != 0 && en.rank != a.rank)) {
    err = kErrShape;
    return false;
  }
  A = reinterpret_cast<const T*>(en.a_ptr);
  alpha = en.alpha;
  rank = en.rank;
  return true;
}

template <typename T>
__device__ __forceinline__ bool resolve_b(const ApplyArgs& a, const Block& blk, int slice, const T*& B, int& rank,
                                          uint32_t& err) {
  if (a.w.mode == kStacked) {
    if (blk.adapter_id < 0 || blk.adapter_id >= a.w.num_ids) {
      err = kErrIdRange;
      return false;
    }
    B = static_cast<const T*>(a.w.b_base[slice]) + static_cast<int64_t>(blk.adapter_id) * a.w.b_stride[slice];
    rank = a.rank;
    return true;
  }
  if (blk.entry < 0 || blk.entry >= a.w.num_ids) {
    err = kErrUnregistered;
    return false;
  }
  const Entry en = a.w.entries[blk.entry];
  if (en.b_ptr == 0) {
    err = kErrUnregistered;
    return false;
  }
  if (en.out_features != a.w.o_size[0] || (a.rank != 0 && en.rank != a.rank)) {
    err = kErrShape;
    return false;
  }
  B = reinterpret_cast<const T*>(en.b_ptr);
  rank = en.rank;
  return true;
}

// ---------------------------------------------------------------- shrink ----

template <typename T, int RANK>
__device__ __forceinline__ void shrink_body(const ApplyArgs& a, const Block& blk, int b, int c, const T* A,
                                            float alpha, f32x4* s_red, int* s_last) {
  using V8 = typename VecOf<T>::v8;
  constexpr int RT = (RANK + 15) / 16;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = lane & 15;
  const int kq = (lane >> 4) * 8;
  const int d = a.d_model;
  const int kw_len = a.dc / kWaves;
  const int k_begin = c * a.dc + wave * kw_len;
  const int k_end = min(k_begin + kw_len, d);
  const int ntt = (blk.count + 15) >> 4;

  const T* X = static_cast<const T*>(a.x);
  const T* xr[kTT];
#pragma unroll
  for (int tt = 0; tt < kTT; ++tt) {
    const int tl = tt * 16 + row;
    xr[tt] = (tl < blk.count) ? X + static_cast<int64_t>(a.plan.perm[blk.first + tl]) * a.ldx : nullptr;
  }
  const T* ar[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int r = rt * 16 + row;
    ar[rt] = r < RANK ? A + static_cast<int64_t>(r) * d : nullptr;
  }

  f32x4 acc[RT][kTT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int tt = 0; tt < kTT; ++tt) acc[rt][tt] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int k = k_begin; k < k_end; k += 64) {
    V8 af[2][RT];
    V8 xf[2][kTT];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int kk = k + s * 32 + kq;
      const bool in = kk < k_end;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) af[s][rt] = (ar[rt] != nullptr && in) ? load8(ar[rt] + kk) : zero8<T>();
#pragma unroll
      for (int tt = 0; tt < kTT; ++tt) xf[s][tt] = (xr[tt] != nullptr && in) ? load8(xr[tt] + kk) : zero8<T>();
    }
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int tt = 0; tt < kTT; ++tt) {
        if (tt < ntt) {
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) acc[rt][tt] = mfma16(af[s][rt], xf[s][tt], acc[rt][tt]);
        }
      }
  }

  // Cross-wave reduction of the four k-slices (fixed wave order).
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int tt = 0; tt < kTT; ++tt)
      if (tt < ntt) s_red[((wave * RT + rt) * kTT + tt) * 64 + lane] = acc[rt][tt];
  __syncthreads();
  const int pst = a.pstride;
  for (int u = threadIdx.x; u < RT * kTT * 64; u += kThreads) {
    const int ln = u & 63;
    const int tt = (u >> 6) % kTT;
    const int rt = (u >> 6) / kTT;
    if (tt >= ntt) continue;
    const int tl = tt * 16 + (ln & 15);
    const int r0 = rt * 16 + (ln >> 4) * 4;
    if (tl >= blk.count || r0 >= RANK) continue;
    f32x4 s = s_red[((0 * RT + rt) * kTT + tt) * 64 + ln];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) s += s_red[((w * RT + rt) * kTT + tt) * 64 + ln];
    *reinterpret_cast<f32x4*>(a.partials + (static_cast<int64_t>(c) * a.ptok + blk.first + tl) * pst + r0) = s;
  }

  // Last-arriver reduction over the chunks.
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = atomicAdd(&a.plan.counters[b], 1u);
    *s_last = (prev == static_cast<unsigned>(a.n_chunks - 1)) ? 1 : 0;
  }
  __syncthreads();
  if (*s_last == 0) return;
  __threadfence();
  T* H = static_cast<T*>(a.h);
  constexpr int R4 = RANK / 4;
  const int64_t chunk_stride = static_cast<int64_t>(a.ptok) * pst;
  for (int u = threadIdx.x; u < blk.count * R4; u += kThreads) {
    const int tl = u / R4;
    const int r0 = (u - tl * R4) * 4;
    const float* p = a.partials + static_cast<int64_t>(blk.first + tl) * pst + r0;
    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
    for (int cc = 0; cc < a.n_chunks; ++cc) s += *reinterpret_cast<const f32x4*>(p + cc * chunk_stride);
    s *= alpha;
    store4(H + static_cast<int64_t>(a.plan.perm[blk.first + tl]) * a.ldh + r0, s);
  }
  if (threadIdx.x == 0) a.plan.counters[b] = 0u;
}

template <typename T, int RANK>
__global__ __launch_bounds__(kThreads) void shrink_kernel(ApplyArgs a) {
  constexpr int RR = RANK == 0 ? kMaxRank : RANK;
  constexpr int RT = (RR + 15) / 16;
  __shared__ f32x4 s_red[kWaves * RT * kTT * 64];
  __shared__ int s_last;
  const int b_stride = gridDim.x / a.n_chunks;
  const int c = blockIdx.x % a.n_chunks;
  const int n_blocks = static_cast<int>(a.plan.header[kHdrNumBlocks]);
  // Block-stride loop: the grid may be capped below the block count.  Every
  // workgroup of a given block b uses the same loop trip, so the shrink body's
  // barriers stay uniform.
  for (int b = blockIdx.x / a.n_chunks; b < n_blocks; b += b_stride) {
    const Block blk = a.plan.blocks[b];
    const T* A = nullptr;
    float alpha = 0.f;
    int rank = 0;
    uint32_t err = 0;
    if (!resolve_a<T>(a, blk, A, alpha, rank, err)) {
      if (c == 0 && threadIdx.x == 0) flag_error(a.plan.header, err);
      continue;
    }
    if constexpr (RANK != 0) {
      shrink_body<T, RANK>(a, blk, b, c, A, alpha, s_red, &s_last);
    } else {
      switch (rank) {
        case 8: shrink_body<T, 8>(a, blk, b, c, A, alpha, s_red, &s_last); break;
        case 16: shrink_body<T, 16>(a, blk, b, c, A, alpha, s_red, &s_last); break;
        case 32: shrink_body<T, 32>(a, blk, b, c, A, alpha, s_red, &s_last); break;
        case 64: shrink_body<T, 64>(a, blk, b, c, A, alpha, s_red, &s_last); break;
        default:
          if (c == 0 && threadIdx.x == 0) flag_error(a.plan.header, kErrShape);
          break;
      }
    }
  }
}

// ---------------------------------------------------------------- expand ----

template <typename T, int RANK>
__device__ __forceinline__ void expand_body(const ApplyArgs& a, const Block& blk, const T* B, int o_first, int o_size,
                                            int y_off) {
  using V8 = typename VecOf<T>::v8;
  constexpr int KS = (RANK + 31) / 32;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = lane & 15;
  const int kq = (lane >> 4) * 8;
  const int oq = (lane >> 4) * 4;
  const int ob = o_first + wave * (kOT * 16);
  const int ntt = (blk.count + 15) >> 4;
  const T* H = static_cast<const T*>(a.h);
  T* Y = static_cast<T*>(a.y);

  // This wave's 64 rows of B stay in VGPRs for all token tiles of the block.
  V8 bf[kOT][KS];
#pragma unroll
  for (int ot = 0; ot < kOT; ++ot) {
    const int o = ob + ot * 16 + row;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int k = ks * 32 + kq;
      bf[ot][ks] = (o < o_size && k < RANK) ? load8(B + static_cast<int64_t>(o) * RANK + k) : zero8<T>();
    }
  }
  for (int tt = 0; tt < ntt; ++tt) {
    // Token (lane & 15) of this tile: the H row it reads and the Y row it owns.
    const int tl = tt * 16 + row;
    const int tok = tl < blk.count ? a.plan.perm[blk.first + tl] : -1;
    V8 hf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int k = ks * 32 + kq;
      hf[ks] = (tok >= 0 && k < RANK) ? load8(H + static_cast<int64_t>(tok) * a.ldh + k) : zero8<T>();
    }
    // Accumulators start from the current Y, in the MFMA output layout:
    // columns ob + ot*16 + (lane >> 4)*4 + [0, 4) of token `tok`.
    T* yrow = tok >= 0 ? Y + static_cast<int64_t>(tok) * a.ldy + y_off : nullptr;
    f32x4 acc[kOT];
#pragma unroll
    for (int ot = 0; ot < kOT; ++ot) {
      const int o = ob + ot * 16 + oq;
      acc[ot] = (yrow != nullptr && o < o_size) ? load4f(yrow + o) : f32x4{0.f, 0.f, 0.f, 0.f};
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

template <typename T, int RANK>
__global__ __launch_bounds__(kThreads) void expand_kernel(ApplyArgs a) {
  const int b_stride = gridDim.x / a.n_ochunks;
  const int oc = blockIdx.x % a.n_ochunks;
  const int n_blocks = static_cast<int>(a.plan.header[kHdrNumBlocks]);
  int s = 0;
  while (s + 1 < a.w.n_slices && oc >= a.w.oc_start[s + 1]) ++s;
  const int o_first = (oc - a.w.oc_start[s]) * kOC;
  const int o_size = a.w.o_size[s];
  const int y_off = a.w.y_off[s];
  for (int b = blockIdx.x / a.n_ochunks; b < n_blocks; b += b_stride) {
    const Block blk = a.plan.blocks[b];
    const T* B = nullptr;
    int rank = 0;
    uint32_t err = 0;
    if (!resolve_b<T>(a, blk, s, B, rank, err)) {
      if (oc == 0 && threadIdx.x == 0) flag_error(a.plan.header, err);
      continue;
    }
    if constexpr (RANK != 0) {
      expand_body<T, RANK>(a, blk, B, o_first, o_size, y_off);
    } else {
      switch (rank) {
        case 8: expand_body<T, 8>(a, blk, B, o_first, o_size, y_off); break;
        case 16: expand_body<T, 16>(a, blk, B, o_first, o_size, y_off); break;
        case 32: expand_body<T, 32>(a, blk, B, o_first, o_size, y_off); break;
        case 64: expand_body<T, 64>(a, blk, B, o_first, o_size, y_off); break;
        default:
          if (oc == 0 && threadIdx.x == 0) flag_error(a.plan.header, kErrShape);
          break;
      }
    }
  }
}

template <typename T, int RANK>
hipError_t launch_shrink_t(const ApplyArgs& a, int max_blocks, hipStream_t stream) {
  const int64_t n = static_cast<int64_t>(max_blocks) * a.n_chunks;  // max_blocks: block slots of the grid
  if (n <= 0) return hipSuccess;
  shrink_kernel<T, RANK><<<dim3(static_cast<unsigned>(n)), dim3(kThreads), 0, stream>>>(a);
  return hipGetLastError();
}

template <typename T, int RANK>
hipError_t launch_expand_t(const ApplyArgs& a, int max_blocks, hipStream_t stream) {
  const int64_t n = static_cast<int64_t>(max_blocks) * a.n_ochunks;
  if (n <= 0) return hipSuccess;
  expand_kernel<T, RANK><<<dim3(static_cast<unsigned>(n)), dim3(kThreads), 0, stream>>>(a);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_shrink_dt(const ApplyArgs& a, int max_blocks, hipStream_t stream) {
  switch (a.rank) {
    case 0: return launch_shrink_t<T, 0>(a, max_blocks, stream);
    case 8: return launch_shrink_t<T, 8>(a, max_blocks, stream);
    case 16: return launch_shrink_t<T, 16>(a, max_blocks, stream);
    case 32: return launch_shrink_t<T, 32>(a, max_blocks, stream);
    case 64: return launch_shrink_t<T, 64>(a, max_blocks, stream);
    default: return hipErrorInvalidValue;
  }
}

template <typename T>
hipError_t launch_expand_dt(const ApplyArgs& a, int max_blocks, hipStream_t stream) {
  switch (a.rank) {
    case 0: return launch_expand_t<T, 0>(a, max_blocks, stream);
    case 8: return launch_expand_t<T, 8>(a, max_blocks, stream);
    case 16: return launch_expand_t<T, 16>(a, max_blocks, stream);
    case 32: return launch_expand_t<T, 32>(a, max_blocks, stream);
    case 64: return launch_expand_t<T, 64>(a, max_blocks, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

int expand_cols_per_workgroup() { return kOC; }

hipError_t launch_shrink(int dtype_bf16, const ApplyArgs& a, int max_blocks, hipStream_t stream) {
  return dtype_bf16 ? launch_shrink_dt<__bf16>(a, max_blocks, stream)
                    : launch_shrink_dt<_Float16>(a, max_blocks, stream);
}

hipError_t launch_expand(int dtype_bf16, const ApplyArgs& a, int max_blocks, hipStream_t stream) {
  return dtype_bf16 ? launch_expand_dt<__bf16>(a, max_blocks, stream)
                    : launch_expand_dt<_Float16>(a, max_blocks, stream);
}

}  // namespace wp
