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
//   shrink workgroups   block b, d-range c, 16 rank rows (32 in calls with
//                       several output slices).  The four waves split the
//                       d-range and reduce through LDS; the workgroup
//                       stores its fp32 partial H coherently.
//   expand workgroups   block b, 256 output columns (of each slice).  They
//                       load their B rows and current Y, poll the block's
//                       partials until they hold values (the buffer holds
//                       the NaN pattern kPartialEmpty between calls, which no
//                       bf16/fp16 computation produces) -- the polling loads
//                       are the reads -- sum them in a fixed order (so every
//                       workgroup, and every run, gets the same bits), apply
//                       alpha once and round H to the I/O dtype in LDS
//                       (reference :129, :360), then run the MFMAs and store
//                       Y = rn(Y + H.B^T) (reference :194).  The last one of
//                       the block empties its partials again.
//
// Summing the partials in every expand workgroup re-reads a few KB per
// workgroup but keeps the cross-workgroup chain to one hop: the partial
// stores themselves are the publication (no acknowledgement wait, no
// counter), and the readers validate every word they use.  Data crosses
// workgroups only through device-scope atomic loads and stores (sc1:
// coherent across the XCDs' L2s) -- never through __threadfence, whose L2
// writeback + invalidate costs ~60-100 ns serialised over the device, nor
// through accumulation atomics.
//
// Grid: the shrink workgroups of every block slot, then the expand
// workgroups.  Those wait only on shrink workgroups,
// which have lower ids and never wait, so with in-order dispatch every wait
// ends; it is bounded anyway and reports kErrSpin if the bound is hit.  Slots
// past the device block count exit at once.
//
// The expand-only variant serves expand() of the engine API and the expand
// half of large-plan calls.  shrink() of decode-sized plans runs the shrink
// side with one reducer workgroup per block (kShrinkOnly); larger plans use
// shrink_kernel, which computes every rank row of a block per workgroup and
// streams the d-range through LDS.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "wp_apply.h"
#include "wp_device.h"

namespace wp {
namespace {


constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kOT = 4;                  // output tiles per wave in expand
constexpr int kOC = kWaves * kOT * 16;  // output columns per expand workgroup (256)
constexpr int kShrinkKSteps = 4;        // 32-wide K-steps per wave per load batch
// Token tiles an expand() workgroup keeps in flight (blocks of 64 tokens in
// large plans); the fused kernel, which decode-sized plans use, works one
// tile at a time to keep its registers for occupancy.
constexpr int kTilesInFlight = kBlockTokens / 16;
// shrink(): its LDS (two A slices and one X tile per wave: 52 KB at rank 64)
// holds three workgroups per compute unit.
constexpr int kShrinkWavesPerSimd = 3;

// kFusedMulti: fused, with several output chunks per expand workgroup.
// kShrinkOnly: shrink() of decode-sized plans: the fused shrink side, and
// one workgroup per block that sums the partials into H.
enum Role : int { kFused = 0, kShrinkOnly = 1, kExpandOnly = 2, kFusedMulti = 3 };


// ---------------------------------------------------------------- shrink ----

// Fused kernel, shrink side: partial H of block b over d-range c for rank
// rows [r_begin, r_begin + 16 * MT), stored coherently to part[c].  The rows
// are the M side of MT MFMA tiles that share every X fragment (rows past the
// adapter's rank load zeros and are not stored; a tile with no rows is
// skipped).  The four waves split the d-range; each loads kShrinkKSteps
// K-steps of A and X at once, then runs the MFMAs.  With a staging tile
// (stg, the apply kernel's shrink side) the loads are in row order and the
// fragments come back from LDS: 8 rows x 128 bytes (whole lines) per
// instruction instead of 16 rows x 64 bytes measured cfg2 qkv 18.47 -> 18.0,
// o_proj 12.80 -> 12.28 us, step 1.267 -> 1.223 ms on MI355X.  Without one
// (linear_kernel, whose LDS holds its GEMM tiles) the fragments load straight
// into registers in the MFMA layout.  The stores are
// the publication: the partial buffer holds kPartialEmpty between calls, and
// the readers poll for real values (no acknowledgement wait, no counter).
// Row-order staging (stg != null): lane l loads 16 bytes of row (l >> 3) + 8i
// at column 8 (l & 7) of a 64-column half, so an instruction moves whole
// 128-byte lines of 8 rows; the wave writes them into its own LDS tile (16-byte
// chunk j of row r at chunk j ^ (r & 7): the MFMA-layout reads of 16 rows
// spread over the banks) and reads the MFMA fragments back.  The tile holds
// 16 * MT A rows and 16 X rows of 64 columns.
constexpr int kStgCols = 64;
template <int MT>
constexpr int stg_elems_per_wave() { return (16 * MT + 16) * kStgCols; }

template <typename T, int MT>
__device__ __forceinline__ void shrink_body(const ApplyArgs& a, int b, int c, int sa, int r_begin, const Block& blk,
                                            int32_t tok0, const Resolved<T>& res, f32x4* s_red, T* stg = nullptr) {
  using V8 = typename VecOf<T>::v8;
  constexpr int KB = kShrinkKSteps;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = lane & 15;
  const int kq = (lane >> 4) * 8;
  const int n_rows = min(16 * MT, res.rank - r_begin);
  // Zero-padded slices (a.pad_rank) store every row of the group, zeros past
  // the adapter's rank, so that all slices' partials have one width.
  const int store_rows = a.pad_rank ? 16 * MT : n_rows;
  if (res.ptr == nullptr || store_rows <= 0) return;
  const int mt_used = n_rows > 0 ? (n_rows + 15) >> 4 : 0;
  const int d = a.d_model;
  const int kw_len = a.dc / kWaves;
  const int k_begin = c * a.dc + wave * kw_len;
  const int k_end = min(k_begin + kw_len, d);
  const int ntt = (blk.count + 15) >> 4;
  const T* X = static_cast<const T*>(a.x);
  const T* ar[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m)
    ar[m] = m * 16 + row < n_rows ? res.ptr + static_cast<int64_t>(r_begin + m * 16 + row) * d : nullptr;
  float* prow = a.part + (static_cast<int64_t>(c) * a.ptok + blk.first) * a.hs + sa * a.hs1 + r_begin;
  for (int tt = 0; tt < ntt; ++tt) {
    const int32_t tok = tt == 0 ? tok0 : block_token(a, b, tt * 16 + row, blk.count);
    const T* xr = tok >= 0 ? X + static_cast<int64_t>(tok) * a.ldx : nullptr;
    f32x4 acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (stg != nullptr) {
      static_assert(KB * 32 == 2 * kStgCols, "a load batch is two staged halves");
      T* tile = stg + wave * stg_elems_per_wave<MT>();
      const int lr = lane >> 3;
      const int lc = (lane & 7) * 8;
      // Row pointers of this lane's row-order rows: A rows g * 8 + lr, X rows
      // of token slots g * 8 + lr (tokens from the MFMA-layout lanes 0..15).
      const T* arw[2 * MT];
#pragma unroll
      for (int g = 0; g < 2 * MT; ++g) {
        const int r = g * 8 + lr;
        arw[g] = r < n_rows ? res.ptr + static_cast<int64_t>(r_begin + r) * d : nullptr;
      }
      const T* xrw[2];
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int32_t tk = __shfl(tok, g * 8 + lr, 64);
        xrw[g] = tk >= 0 ? X + static_cast<int64_t>(tk) * a.ldx : nullptr;
      }
      for (int k = k_begin; mt_used > 0 && k < k_end; k += 32 * KB) {
        u32x4 ra[2][2 * MT];
        u32x4 rx[2][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int col = k + h * kStgCols + lc;
          const bool in = col < k_end;
#pragma unroll
          for (int g = 0; g < 2 * MT; ++g)
            ra[h][g] = (arw[g] != nullptr && in) ? load16_global(arw[g] + col) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
          for (int g = 0; g < 2; ++g)
            rx[h][g] = (xrw[g] != nullptr && in) ? load16_global(xrw[g] + col) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int g = 0; g < 2 * MT; ++g) {
            const int r = g * 8 + lr;
            *reinterpret_cast<u32x4*>(tile + r * kStgCols + (((lane & 7) ^ (r & 7)) << 3)) = ra[h][g];
          }
#pragma unroll
          for (int g = 0; g < 2; ++g) {
            const int r = 16 * MT + g * 8 + lr;
            *reinterpret_cast<u32x4*>(tile + r * kStgCols + (((lane & 7) ^ (r & 7)) << 3)) = rx[h][g];
          }
#pragma unroll
          for (int st = 0; st < 2; ++st) {
            const int ch = st * 4 + (kq >> 3);
            const int rxr = 16 * MT + row;
            const V8 xf = __builtin_bit_cast(
                V8, *reinterpret_cast<const u32x4*>(tile + rxr * kStgCols + ((ch ^ (rxr & 7)) << 3)));
#pragma unroll
            for (int m = 0; m < MT; ++m) {
              if (m < mt_used) {
                const int rar = m * 16 + row;
                const V8 af = __builtin_bit_cast(
                    V8, *reinterpret_cast<const u32x4*>(tile + rar * kStgCols + ((ch ^ (rar & 7)) << 3)));
                acc[m] = mfma16(af, xf, acc[m]);
              }
            }
          }
        }
      }
      // Other waves' tiles overlap s_red.
      lds_barrier();
    } else {
      for (int k = k_begin; mt_used > 0 && k < k_end; k += 32 * KB) {
        V8 af[KB][MT];
        V8 xf[KB];
#pragma unroll
        for (int st = 0; st < KB; ++st) {
          const int kk = k + st * 32 + kq;
          const bool in = kk < k_end;
#pragma unroll
          for (int m = 0; m < MT; ++m) af[st][m] = (ar[m] != nullptr && in) ? load8(ar[m] + kk) : zero8<T>();
          xf[st] = (xr != nullptr && in) ? load8(xr + kk) : zero8<T>();
        }
#pragma unroll
        for (int st = 0; st < KB; ++st)
#pragma unroll
          for (int m = 0; m < MT; ++m)
            if (m < mt_used) acc[m] = mfma16(af[st][m], xf[st], acc[m]);
      }
    }
    if (tt == 0) trace_stamp(a, 2);
    // Reduce the four waves' d-slices through LDS (fixed order) and store
    // the tile's partial, coherently.
#pragma unroll
    for (int m = 0; m < MT; ++m) s_red[(m * kWaves + wave) * 64 + lane] = acc[m];
    __syncthreads();
    if (static_cast<int>(threadIdx.x) < 64 * (a.pad_rank ? MT : mt_used)) {
      const int m = threadIdx.x >> 6;
      const int tl = tt * 16 + (lane & 15);
      const int r0 = m * 16 + (lane >> 4) * 4;
      if (tl < blk.count && r0 < store_rows) {
        f32x4 sum = s_red[m * kWaves * 64 + lane];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) sum += s_red[(m * kWaves + w) * 64 + lane];
        coherent_store_f4(prow + static_cast<int64_t>(tl) * a.hs + r0, sum);
      }
    }
    __syncthreads();
  }
  trace_stamp(a, 3);
}

// ---------------------------------------------------------------- reduce ----


// Waits (wave 0 polls, bounded) until one probe word of every shrink
// workgroup's partial of block b holds a value: a cheap gate before the full
// read, which validates every word itself.  Shrink workgroups are (d-range,
// rank group, A slice); a lane probes up to kProbesPerLane of them.  Returns
// false after a give-up.
// PA: one A per slice (more shrink workgroups than one probe per lane).
constexpr int kProbesPerLane = 4;
template <bool PA>
__device__ __forceinline__ bool wait_partials(const ApplyArgs& a, const Block& blk, int rank, int* s_flag,
                                              uint32_t wmask = 1u) {
  constexpr int kProbes = PA ? kProbesPerLane : 1;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int n_rg = (rank + a.srows - 1) / a.srows;
    const int per_a = a.n_chunks * n_rg;
    const int n_probe = PA ? per_a * a.w.n_a : per_a;
    // Word offsets into the partial buffer (at most 16 x 512 x 256 words).
    constexpr uint32_t kNone = 0xFFFFFFFFu;
    uint32_t probe[kProbes];
#pragma unroll
    for (int q = 0; q < kProbes; ++q) {
      const int i = lane + 64 * q;
      probe[q] = kNone;
      if (i < n_probe) {
        const int sa = PA ? i / per_a : 0;
        const int k = i - sa * per_a;
        const int rg = k / a.n_chunks;
        const int kc = k - rg * a.n_chunks;
        // Only slices whose shrink side writes (one A per slice, table mode).
        if (!PA || ((wmask >> sa) & 1u))
          probe[q] = static_cast<uint32_t>((kc * a.ptok + blk.first) * a.hs + sa * a.hs1 + rg * a.srows);
      }
    }
    int ok = 1;
    for (unsigned spins = 0;; ++spins) {
      // Both tests are uniform over the wave.  After the bound, or once
      // another wait of the call gave up, the block is abandoned.
      if (spins >= a.spin_limit || (spins > 0 && poisoned(a.plan.header))) {
        ok = 0;
        if (lane == 0 && spins >= a.spin_limit) give_up(a.plan.header);
        break;
      }
      bool here = true;
#pragma unroll
      for (int q = 0; q < kProbes; ++q)
        here = here && (probe[q] == kNone || !is_empty(__builtin_bit_cast(
                                                 float, atomic_load_u(reinterpret_cast<const uint32_t*>(a.part) + probe[q]))));
      if (__all(here)) break;
      __builtin_amdgcn_s_sleep(2);
    }
    if (lane == 0) *s_flag = ok;
  }
  __syncthreads();
  return *s_flag != 0;
}

// H of block b: rn(alpha * sum_c part[c]), each thread polling the partial
// words it sums until they hold values (CB d-ranges per load batch), so the
// loads that find a block's last partial also bring its data: once the gate
// has opened there is no separate read.  A thread owns whole 2-wide units
// (8-byte loads: half the registers per d-range in flight of 4-wide ones,
// so more d-ranges go out per batch) and adds their d-ranges in increasing
// order, so every workgroup that reduces the block gets the same bits.
// (Sharing a unit between lanes and combining with shuffles cost the
// single-slice kernel spills and measured slower.)  emit(j, r0, v2)
// receives each unit.
template <int CB, typename Emit>
__device__ __forceinline__ void collect_partials(const ApplyArgs& a, const Block& blk, const int R2, float alpha,
                                                  Emit emit) {
  const int n_units = blk.count * R2;
  const int nch = a.n_chunks;
  const uint32_t cstride = static_cast<uint32_t>(a.ptok) * static_cast<uint32_t>(a.hs) * 4u;
  const char* pbase = reinterpret_cast<const char*>(a.part + static_cast<int64_t>(blk.first) * a.hs);
  for (int u = threadIdx.x; u < n_units; u += kThreads) {
    const int j = u / R2;
    const int r0 = (u - j * R2) * 2;
    const uint32_t o0 = static_cast<uint32_t>(j * a.hs + r0) * 4u;
    f32x2 sum = f32x2{0.f, 0.f};
    for (int c0 = 0; c0 < nch; c0 += CB) {
      f32x2 v[CB];
      for (unsigned spins = 0;; ++spins) {
        if (spins >= a.spin_limit || (spins > 0 && poisoned(a.plan.header))) {
          if (spins >= a.spin_limit) give_up(a.plan.header);
#pragma unroll
          for (int i = 0; i < CB; ++i) v[i] = f32x2{0.f, 0.f};
          break;
        }
        bool missing = false;
#pragma unroll
        for (int i = 0; i < CB; ++i) {
          const int cc = min(c0 + i, nch - 1);
          v[i] = __builtin_bit_cast(f32x2, coherent_load8(pbase + (o0 + static_cast<uint32_t>(cc) * cstride)));
        }
#pragma unroll
        for (int i = 0; i < CB; ++i) missing = missing || is_empty(v[i][0]) || is_empty(v[i][1]);
        if (!missing) break;
        __builtin_amdgcn_s_sleep(2);
      }
#pragma unroll
      for (int i = 0; i < CB; ++i)
        if (c0 + i < nch) sum += v[i];
    }
    emit(j, r0, sum * alpha);
  }
}

// Waits until every partial word the block's shrink workgroups write (count x
// rank values of every d-range) holds a value, without using them.
__device__ __forceinline__ void await_partials(const ApplyArgs& a, const Block& blk, int rank) {
  const int r4 = rank / 4;
  const int per_chunk = blk.count * r4;
  const int total = per_chunk * a.n_chunks;
  for (int u = threadIdx.x; u < total; u += kThreads) {
    const int c = u / per_chunk;
    const int q = u - c * per_chunk;
    const int j = q / r4;
    const int r0 = (q - j * r4) * 4;
    const float* p = a.part + (static_cast<int64_t>(c) * a.ptok + blk.first + j) * a.hs + r0;
    for (unsigned spins = 0;; ++spins) {
      if (spins >= a.spin_limit || (spins > 0 && poisoned(a.plan.header))) {
        if (spins >= a.spin_limit) give_up(a.plan.header);
        break;
      }
      if (!any_empty(coherent_load_f4(p))) break;
      __builtin_amdgcn_s_sleep(4);
    }
  }
}

// Restores kPartialEmpty over everything the block's shrink workgroups wrote
// (count x rank values of every d-range) once its last reader is done, so the
// next call finds the buffer empty.  `nthreads` threads take part.  Like every
// access to the partial buffer, the stores are device-coherent.
__device__ __forceinline__ void clear_partials(const ApplyArgs& a, const Block& blk, int rank, int tid, int nthreads) {
  const int r4 = rank / 4;
  const int per_chunk = blk.count * r4;
  const int total = per_chunk * a.n_chunks;
  const f32x4 e = __builtin_bit_cast(f32x4, u32x4{kPartialEmpty, kPartialEmpty, kPartialEmpty, kPartialEmpty});
  for (int u = tid; u < total; u += nthreads) {
    const int c = u / per_chunk;
    const int q = u - c * per_chunk;
    const int j = q / r4;
    const int r0 = (q - j * r4) * 4;
    coherent_store_f4(a.part + (static_cast<int64_t>(c) * a.ptok + blk.first + j) * a.hs + r0, e);
  }
}

// One A per slice: the partial row holds n_a slices of hs1 columns; slice sa
// (if bit sa of wmask is set: its shrink side wrote) has W columns at
// sa * hs1 (W = the rank, or hs1 for zero-padded slices).  The same as
// collect_partials / await_partials / clear_partials otherwise; emit gets the
// column in the row, and each slice's alpha (alphas[sa]) is applied.
__device__ __forceinline__ float slice_alpha(const float (&al)[kMaxSlices], int sa) {
  return sa == 0 ? al[0] : sa == 1 ? al[1] : sa == 2 ? al[2] : al[3];
}

template <int CB, typename Emit>
__device__ __forceinline__ void collect_partials_pa(const ApplyArgs& a, const Block& blk, int W, uint32_t wmask,
                                                     const float (&alphas)[kMaxSlices], Emit emit) {
  const int W2 = W / 2;
  const int per_tok = a.w.n_a * W2;
  const int n_units = blk.count * per_tok;
  const int nch = a.n_chunks;
  const uint32_t cstride = static_cast<uint32_t>(a.ptok) * static_cast<uint32_t>(a.hs) * 4u;
  const char* pbase = reinterpret_cast<const char*>(a.part + static_cast<int64_t>(blk.first) * a.hs);
  for (int u = threadIdx.x; u < n_units; u += kThreads) {
    const int j = u / per_tok;
    const int rem = u - j * per_tok;
    const int sa = rem / W2;
    const int col = sa * a.hs1 + (rem - sa * W2) * 2;
    if (!((wmask >> sa) & 1u)) {
      emit(j, col, f32x2{0.f, 0.f});
      continue;
    }
    const uint32_t o0 = static_cast<uint32_t>(j * a.hs + col) * 4u;
    f32x2 sum = f32x2{0.f, 0.f};
    for (int c0 = 0; c0 < nch; c0 += CB) {
      f32x2 v[CB];
      for (unsigned spins = 0;; ++spins) {
        if (spins >= a.spin_limit || (spins > 0 && poisoned(a.plan.header))) {
          if (spins >= a.spin_limit) give_up(a.plan.header);
#pragma unroll
          for (int i = 0; i < CB; ++i) v[i] = f32x2{0.f, 0.f};
          break;
        }
        bool missing = false;
#pragma unroll
        for (int i = 0; i < CB; ++i) {
          const int cc = min(c0 + i, nch - 1);
          v[i] = __builtin_bit_cast(f32x2, coherent_load8(pbase + (o0 + static_cast<uint32_t>(cc) * cstride)));
        }
#pragma unroll
        for (int i = 0; i < CB; ++i) missing = missing || is_empty(v[i][0]) || is_empty(v[i][1]);
        if (!missing) break;
        __builtin_amdgcn_s_sleep(2);
      }
#pragma unroll
      for (int i = 0; i < CB; ++i)
        if (c0 + i < nch) sum += v[i];
    }
    emit(j, col, sum * slice_alpha(alphas, sa));
  }
}

// The words of the written slices, each (d-range, token, slice, 4 columns):
// visit(c, j, col) for every unit `tid` owns.
template <typename Visit>
__device__ __forceinline__ void for_pa_units(const ApplyArgs& a, const Block& blk, int W, uint32_t wmask, int tid,
                                             int nthreads, Visit visit) {
  const int W4 = W / 4;
  const int per_chunk = blk.count * a.w.n_a * W4;
  const int total = per_chunk * a.n_chunks;
  for (int u = tid; u < total; u += nthreads) {
    const int c = u / per_chunk;
    const int q = u - c * per_chunk;
    const int j = q / (a.w.n_a * W4);
    const int rem = q - j * (a.w.n_a * W4);
    const int sa = rem / W4;
    if (!((wmask >> sa) & 1u)) continue;
    visit(c, j, sa * a.hs1 + (rem - sa * W4) * 4);
  }
}

__device__ __forceinline__ void await_partials_pa(const ApplyArgs& a, const Block& blk, int W, uint32_t wmask) {
  for_pa_units(a, blk, W, wmask, threadIdx.x, kThreads, [&](int c, int j, int col) {
    const float* p = a.part + (static_cast<int64_t>(c) * a.ptok + blk.first + j) * a.hs + col;
    for (unsigned spins = 0;; ++spins) {
      if (spins >= a.spin_limit || (spins > 0 && poisoned(a.plan.header))) {
        if (spins >= a.spin_limit) give_up(a.plan.header);
        break;
      }
      if (!any_empty(coherent_load_f4(p))) break;
      __builtin_amdgcn_s_sleep(4);
    }
  });
}

__device__ __forceinline__ void clear_partials_pa(const ApplyArgs& a, const Block& blk, int W, uint32_t wmask, int tid,
                                                  int nthreads) {
  const f32x4 e = __builtin_bit_cast(f32x4, u32x4{kPartialEmpty, kPartialEmpty, kPartialEmpty, kPartialEmpty});
  for_pa_units(a, blk, W, wmask, tid, nthreads, [&](int c, int j, int col) {
    coherent_store_f4(a.part + (static_cast<int64_t>(c) * a.ptok + blk.first + j) * a.hs + col, e);
  });
}

// ---------------------------------------------------------------- expand ----

// Row stride (elements) of the block's H in LDS: RANK plus 8 to spread banks.
template <int RANK>
constexpr int lds_h_stride() { return RANK + 8; }

// One 256-column output chunk of an expand workgroup: its slice's B rows and
// where its columns land in Y.
template <typename T>
struct OutChunk {
  Resolved<T> res;
  int o_first = 0;  // first output column inside the slice
  int o_size = 0;   // the slice's output columns
  int y_off = 0;    // the slice's first column in Y
  int h_col = 0;    // the slice's first column in an H row (its A slice's H)
};

// kSliceH: a slice may have its own H (one A per slice, or expand() of such
// a call's H); otherwise every slice reads H from column 0.  TS: as resolve_b.
template <typename T, bool kSliceH, bool TS = false>
__device__ __forceinline__ OutChunk<T> out_chunk(const ApplyArgs& a, const Block& blk, int oc,
                                                 PreEntry pre = PreEntry{}) {
  int s = 0;
  while (s + 1 < a.w.n_slices && oc >= a.w.oc_start[s + 1]) ++s;
  OutChunk<T> c;
  c.res = resolve_b<T, TS>(a, blk, s, pre);
  c.o_first = (oc - a.w.oc_start[s]) * kOC;
  c.o_size = a.w.o_size[s];
  c.y_off = a.w.y_off[s];
  c.h_col = (kSliceH && a.w.n_a > 1) ? s * a.hs1 : 0;
  return c;
}


// This wave's 64 rows of the chunk's B and token tile 0 of its Y columns.
// DYN: B's row stride is the chunk's adapter rank (zero-padded slices of
// mixed ranks, expanded at RANK = 64); otherwise RANK.
template <typename T, int RANK, bool DYN = false>
__device__ __forceinline__ void load_chunk(const ApplyArgs& a, const OutChunk<T>& c, int32_t tok0,
                                           typename VecOf<T>::v8 (&bf)[kOT][(RANK + 31) / 32], YRows& y0) {
  constexpr int KS = (RANK + 31) / 32;
  const int rb = DYN ? c.res.rank : RANK;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = lane & 15;
  const int kq = (lane >> 4) * 8;
  const int ob = c.o_first + wave * (kOT * 16);
  const bool ok = c.res.ptr != nullptr;
#pragma unroll
  for (int ot = 0; ot < kOT; ++ot) {
    const int o = ob + ot * 16 + row;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int k = ks * 32 + kq;
      bf[ot][ks] = (ok && o < c.o_size && k < rb) ? load8(c.res.ptr + static_cast<int64_t>(o) * rb + k)
                                                    : zero8<T>();
    }
  }
  int32_t tok[2];
  yrows_tokens(ok ? tok0 : -1, tok);
  y0 = yrows_load<T>(a, c.y_off, ob, c.o_size, tok);
}

// Y[tokens, chunk columns] = rn(Y + H.B^T) for every token tile of the block;
// H comes from LDS (fused; rows of hsl elements) or from the caller's
// token-indexed H (expand()), at the chunk's column c.h_col.  MAXT tiles are
// in flight at once: their Y (and H) loads are issued together before the
// MFMAs; y0 holds tile 0's Y, already loaded.  `stage` is this wave's
// 16 x kStageStride LDS tile.
template <typename T, int RANK, bool kHFromLds, int MAXT>
__device__ __forceinline__ void compute_chunk(const ApplyArgs& a, int b, const Block& blk, int32_t tok0,
                                              const OutChunk<T>& c,
                                              const typename VecOf<T>::v8 (&bf)[kOT][(RANK + 31) / 32],
                                              const YRows& y0, const T* s_h, int hsl, T* stage) {
  using V8 = typename VecOf<T>::v8;
  constexpr int KS = (RANK + 31) / 32;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = lane & 15;
  const int kq = (lane >> 4) * 8;
  const int oq = (lane >> 4) * 4;
  const int ob = c.o_first + wave * (kOT * 16);
  const int ntt = (blk.count + 15) >> 4;
  T* st_row = stage + row * kStageStride;                                 // MFMA-layout row of this lane
  T* st_seg = stage + (lane >> 3) * kStageStride + (lane & 7) * 8;        // row-order segment of this lane
  for (int t0 = 0; t0 < ntt; t0 += MAXT) {
    int32_t tok_row[MAXT];
    int32_t tok[MAXT][2];
    YRows yt[MAXT];
    V8 hf[MAXT][KS];
#pragma unroll
    for (int i = 0; i < MAXT; ++i) {
      const int tt = t0 + i;
      tok_row[i] = tt == 0 ? tok0 : (tt < ntt ? block_token(a, b, tt * 16 + row, blk.count) : -1);
      yrows_tokens(tok_row[i], tok[i]);
      if (tt == 0)
        yt[i] = y0;
      else
        yt[i] = yrows_load<T>(a, c.y_off, ob, c.o_size, tok[i]);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int k = ks * 32 + kq;
        if (tok_row[i] < 0 || k >= RANK) {
          hf[i][ks] = zero8<T>();
        } else if constexpr (kHFromLds) {
          hf[i][ks] = __builtin_bit_cast(V8, *reinterpret_cast<const u32x4*>(s_h + (tt * 16 + row) * hsl + c.h_col + k));
        } else {
          hf[i][ks] = load8(static_cast<const T*>(a.h) + static_cast<int64_t>(tok_row[i]) * a.ldh + c.h_col + k);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < MAXT; ++i) {
      if (t0 + i >= ntt) break;
      // Row order -> MFMA layout through the stage (one wave, in order).
      stage_put(st_seg, yt[i].v[0]);
      stage_put(st_seg + 8 * kStageStride, yt[i].v[1]);
      f32x4 acc[kOT];
#pragma unroll
      for (int ot = 0; ot < kOT; ++ot) acc[ot] = unpack4f<T>(*reinterpret_cast<const u32x2*>(st_row + ot * 16 + oq));
#pragma unroll
      for (int ot = 0; ot < kOT; ++ot)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) acc[ot] = mfma16(bf[ot][ks], hf[i][ks], acc[ot]);
      // MFMA layout -> row order, then whole-line stores.
#pragma unroll
      for (int ot = 0; ot < kOT; ++ot)
        *reinterpret_cast<u32x2*>(st_row + ot * 16 + oq) = __builtin_bit_cast(u32x2, round4<T>(acc[ot]));
      YRows out;
      out.v[0] = stage_get(st_seg);
      out.v[1] = stage_get(st_seg + 8 * kStageStride);
      yrows_store<T>(a, c.y_off, ob, c.o_size, tok[i], out);
    }
  }
}

// Expand workgroup `p` of block b: output chunks p, p + n_owg, ... (at most
// n_sub of them; with several slices of equal width, one chunk per slice).
// Chunk 0's B and Y are loaded before the wait.  MIX: mixed ranks in a
// fused role, expanded at RANK = kMaxRank whatever the block's adapter rank:
// B rows at the adapter's own stride (zeros past its rank), H columns past
// it zero in LDS.  One body instead of one per rank keeps the multi-chunk
// kernel within its registers.
template <typename T, int RANK, int ROLE, int TILES, bool PA, bool MIX = false>
__device__ __forceinline__ void expand_body(const ApplyArgs& a, int b, int p, const Block& blk, int32_t tok0,
                                            T* s_h, T* s_stage, int* s_flag, PreEntry pre = PreEntry{}) {
  using V8 = typename VecOf<T>::v8;
  constexpr int KS = (RANK + 31) / 32;
  constexpr bool kFusedRole = ROLE == kFused || ROLE == kFusedMulti;
  constexpr bool kDyn = PA || MIX;  // B row stride: the adapter's rank
  // LDS row of the block's H: every A slice's H side by side (hs1 columns
  // each), plus 8 elements to spread banks.
  const int hsl = PA ? a.w.n_a * a.hs1 + 8 : RANK + 8;
  constexpr bool kSliceH = PA || ROLE == kExpandOnly;
  const int n_owg = (a.n_ochunks + a.n_sub - 1) / a.n_sub;
  T* stage = s_stage + (threadIdx.x >> 6) * 16 * kStageStride;
  OutChunk<T> cur = out_chunk<T, kSliceH, PA>(a, blk, p, pre);
  if (cur.res.err != 0 && cur.o_first == 0 && threadIdx.x == 0) flag_error(a.plan.header, cur.res.err);
  // Rank rows the block's shrink side writes (0: it could not resolve the
  // adapter and writes nothing).
  int wrote = kFusedRole ? resolve_a<T, PA>(a, blk, 0, pre).rank : 0;
  // One A per slice: the slices whose shrink side writes (the same
  // resolution as theirs), the columns each writes (W: the rank, or all hs1
  // of a zero-padded slice) and each one's alpha.
  uint32_t wmask = 1u;
  int W = RANK;
  float alphas[kMaxSlices] = {0.f, 0.f, 0.f, 0.f};
  if constexpr (PA && kFusedRole) {
    W = a.pad_rank ? a.hs1 : RANK;
    if (a.w.mode == kStacked) {
      wmask = wrote > 0 ? (1u << a.w.n_a) - 1u : 0u;
#pragma unroll
      for (int s = 0; s < kMaxSlices; ++s) alphas[s] = a.w.scale;
    } else {
      wmask = 0u;
#pragma unroll
      for (int s = 0; s < kMaxSlices; ++s) {
        if (s >= a.w.n_a) break;
        const Resolved<T> rs = resolve_a<T, true>(a, blk, s);
        if (rs.ptr != nullptr) {
          wmask |= 1u << s;
          alphas[s] = rs.alpha;
        }
      }
    }
    wrote = wmask != 0u ? W : 0;
  }
  // Partial words per token the block's shrink side writes.
  const int wrote_all = PA ? W * __builtin_popcount(wmask) : wrote;
  V8 bf[kOT][KS];
  YRows yq;
  load_chunk<T, RANK, kDyn>(a, cur, tok0, bf, yq);
  trace_stamp(a, 2);

  bool go = cur.res.ptr != nullptr;
  unsigned consumed_prev = 0;
  if constexpr (kFusedRole) {
    // One A per slice over several chunks: a later chunk's slice may have
    // resolved where the first one's did not (table mode), so the workgroup
    // collects H if any slice wrote, and each chunk is tested on its own.
    go = (PA && ROLE == kFusedMulti ? true : go) && wrote > 0;
    if (go) {
      // Workgroups of small blocks (at most 2048 partial words) poll the
      // data straight away; the probe gate in front pays off for larger
      // blocks.  Measured on MI355X with the gate on every single-slice
      // block: cfg5 (88 calls) 736 -> 696 us, cfg1 8.23 -> 7.78 us, cfg2
      // o_proj unchanged.
      go = (blk.count * wrote_all * a.n_chunks > 2048)
               ? wait_partials<PA>(a, blk, wrote, s_flag, wmask)
               : true;
      trace_stamp(a, 3);
      if (go) {
        const auto to_lds = [&](int j, int r0, f32x2 v) {
          typename VecOf<T>::v2 o;
          o[0] = static_cast<T>(v[0]);
          o[1] = static_cast<T>(v[1]);
          *reinterpret_cast<typename VecOf<T>::v2*>(s_h + j * hsl + r0) = o;
        };
        // Batches of d-ranges: all eight of a multi-slice call's at once;
        // four in the single-slice kernel (eight cost it a spill and
        // measured slower).
        if constexpr (PA) {
          if constexpr (ROLE == kFusedMulti) {
            collect_partials_pa<8>(a, blk, W, wmask, alphas, to_lds);
          } else {
            collect_partials_pa<4>(a, blk, W, wmask, alphas, to_lds);
          }
        } else if constexpr (MIX) {
          // The adapter's rank columns from the partials, zeros past it.
          const int zp = (RANK - wrote) / 2;
          for (int u = threadIdx.x; u < blk.count * zp; u += kThreads) {
            const int j = u / zp;
            to_lds(j, wrote + (u - j * zp) * 2, f32x2{0.f, 0.f});
          }
          if constexpr (ROLE == kFusedMulti) {
            collect_partials<8>(a, blk, wrote / 2, cur.res.alpha, to_lds);
          } else {
            collect_partials<4>(a, blk, wrote / 2, cur.res.alpha, to_lds);
          }
        } else if constexpr (ROLE == kFusedMulti) {
          collect_partials<8>(a, blk, RANK / 2, cur.res.alpha, to_lds);
        } else {
          collect_partials<4>(a, blk, RANK / 2, cur.res.alpha, to_lds);
        }
      }
    } else if (wrote > 0) {
      // Nothing to compute, but this may be the workgroup that empties the
      // partials: every store must have landed first.
      if constexpr (PA) {
        await_partials_pa(a, blk, W, wmask);
      } else {
        await_partials(a, blk, wrote_all);
      }
    }
    __syncthreads();
    trace_stamp(a, 4);
    // This workgroup has read everything it needs from the partials; the
    // count's latency hides behind the MFMAs.
    if (threadIdx.x == 0) consumed_prev = atomic_add_u(&a.consumed[b * kCounterStride], 1u);
  }
  if (go) {
    if constexpr (ROLE == kFusedMulti && RANK <= 32) {
      // Chunks 1 and 2 (the k and v slices of a qkv call) load together
      // once the partials are in, so their latency is paid once: qkv
      // 18.55 -> 18.19 us at 4 waves per SIMD, measured on MI355X (holding
      // them before the collection instead, with 5 waves, was slower).
      OutChunk<T> cn[2];
      V8 bfn[2][kOT][KS];
      YRows yqn[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int oc = p + (j + 1) * n_owg;
        cn[j].res.ptr = nullptr;
        if (j + 1 < a.n_sub && oc < a.n_ochunks) {
          cn[j] = out_chunk<T, kSliceH, PA>(a, blk, oc, pre);
          if (cn[j].res.err != 0 && cn[j].o_first == 0 && threadIdx.x == 0) flag_error(a.plan.header, cn[j].res.err);
          if (cn[j].res.ptr != nullptr) load_chunk<T, RANK, kDyn>(a, cn[j], tok0, bfn[j], yqn[j]);
        }
      }
      if (cur.res.ptr != nullptr) compute_chunk<T, RANK, true, 1>(a, b, blk, tok0, cur, bf, yq, s_h, hsl, stage);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        if (cn[j].res.ptr != nullptr) compute_chunk<T, RANK, true, 1>(a, b, blk, tok0, cn[j], bfn[j], yqn[j], s_h, hsl, stage);
      for (int i = 3; i < a.n_sub; ++i) {
        const int oc = p + i * n_owg;
        if (oc >= a.n_ochunks) break;
        cur = out_chunk<T, kSliceH, PA>(a, blk, oc, pre);
        if (cur.res.err != 0 && cur.o_first == 0 && threadIdx.x == 0) flag_error(a.plan.header, cur.res.err);
        load_chunk<T, RANK, kDyn>(a, cur, tok0, bf, yq);
        if (cur.res.ptr != nullptr) compute_chunk<T, RANK, true, 1>(a, b, blk, tok0, cur, bf, yq, s_h, hsl, stage);
      }
    } else if constexpr (ROLE == kFusedMulti) {
      // Rank 64: chunks after the first load when they are reached (its
      // doubled B fragments leave no room for more sets).
      for (int i = 0; i < a.n_sub; ++i) {
        const int oc = p + i * n_owg;
        if (oc >= a.n_ochunks) break;
        if (i > 0) {
          cur = out_chunk<T, kSliceH, PA>(a, blk, oc, pre);
          if (cur.res.err != 0 && cur.o_first == 0 && threadIdx.x == 0) flag_error(a.plan.header, cur.res.err);
          load_chunk<T, RANK, kDyn>(a, cur, tok0, bf, yq);
        }
        if (cur.res.ptr != nullptr) compute_chunk<T, RANK, true, 1>(a, b, blk, tok0, cur, bf, yq, s_h, hsl, stage);
      }
    } else {
      compute_chunk<T, RANK, kFusedRole, kFusedRole ? 1 : TILES>(a, b, blk, tok0, cur, bf, yq, s_h, hsl, stage);
    }
  }

  trace_stamp(a, 5);
  if constexpr (kFusedRole) {
    // The last expand workgroup of the block to finish reading (every other
    // one has counted) empties the block's partials and resets the counter.
    if (threadIdx.x == 0) *s_flag = consumed_prev == static_cast<unsigned>(n_owg - 1) ? 1 : 0;
    __syncthreads();
    if (*s_flag != 0) {
      if (threadIdx.x == 0) atomic_store_u(&a.consumed[b * kCounterStride], 0u);
      if constexpr (PA) {
        if (wmask != 0u) clear_partials_pa(a, blk, W, wmask, threadIdx.x, kThreads);
      } else {
        if (wrote > 0) clear_partials(a, blk, wrote_all, threadIdx.x, kThreads);
      }
    }
  }
}

// shrink() of decode-sized plans (role kShrinkOnly): block b's one reader
// sums its partials into H[token] = rn(alpha * sum_c part[c]) and, once
// every thread has read its words, restores kPartialEmpty over them.
template <typename T>
__device__ __forceinline__ void reduce_to_h(const ApplyArgs& a, int b, const Block& blk, int* s_flag,
                                            PreEntry pre = PreEntry{}) {
  const Resolved<T> res = resolve_a<T>(a, blk, 0, pre);
  // Rank rows the shrink side wrote (none if it could not resolve the adapter).
  const int wrote = res.ptr != nullptr ? res.rank : 0;
  if (wrote <= 0) return;
  if (blk.count * wrote * a.n_chunks > 2048) wait_partials<false>(a, blk, wrote, s_flag);
  T* H = static_cast<T*>(a.h);
  const int32_t* toks = a.plan.bperm + static_cast<int64_t>(b) * kBlockTokens;
  const bool f32 = a.h_f32 != 0;
  collect_partials<8>(a, blk, wrote / 2, res.alpha, [&](int j, int r0, f32x2 v) {
    const int64_t at = static_cast<int64_t>(toks[j]) * a.ldh + r0;
    if (f32) {
      // fp32 H (vLLM's lora_shrink buffer): added to, not rounded.
      f32x2* hp = reinterpret_cast<f32x2*>(static_cast<float*>(a.h) + at);
      *hp = *hp + v;
      return;
    }
    typename VecOf<T>::v2 o;
    o[0] = static_cast<T>(v[0]);
    o[1] = static_cast<T>(v[1]);
    *reinterpret_cast<typename VecOf<T>::v2*>(H + at) = o;
  });
  trace_stamp(a, 4);
  __syncthreads();
  clear_partials(a, blk, wrote, threadIdx.x, kThreads);
}

// ---------------------------------------------------------------- kernels ----

// apply_kernel's explicit arguments, as laid out in its kernel-argument
// segment: touch_kernel_args reads below this size only.
struct ApplyKernelArgs {
  const uint32_t* header;
  const Block* blocks;
  const int32_t* bperm;
  int32_t per_shrink, n_shrink, per_block;
  ApplyArgs a;
};
static_assert(offsetof(ApplyKernelArgs, a) == 40 && sizeof(ApplyKernelArgs) == 40 + sizeof(ApplyArgs),
              "apply_kernel's argument size as passed to touch_kernel_args");

// Occupancy target (waves per SIMD), from the registers each variant needs
// without spilling: the fused kernel holds B and Y across the partials'
// collection, the multi-slice one also two 16-row shrink tiles; expand()
// keeps four token tiles in flight; rank 64 and mixed ranks hold twice the B
// fragments.
template <int RANK, int ROLE, int TILES>
constexpr int waves_per_simd() {
  constexpr bool wide = RANK == 0 || RANK == 64;
  if (ROLE == kFused) return wide ? 5 : 7;
  if (ROLE == kFusedMulti) return 4;
  if (ROLE == kShrinkOnly) return 5;
  if (TILES == 1) return wide ? 5 : 8;
  return wide ? 3 : 5;
}

// LDS of one workgroup: shrink's cross-wave tiles, or expand's block H.
// The shrink side's row-order staging tiles (SMT: its MFMA tiles, 0 for
// roles without a shrink side) overlay both regions: they are used before
// the cross-wave reduction and never by expand workgroups.
template <typename T, int RANK, int SMT>
struct alignas(16) SharedMem {
  static constexpr int RR = RANK == 0 ? kMaxRank : RANK;
  static constexpr int kRed = kShrinkRowsFused / 16 * kWaves * 64;    // f32x4
  // H rows of one block: the fused roles run on plans of 16-token blocks
  // (launch_fused checks); no other role keeps H in LDS.
  static constexpr int kH = (16 * (kMaxSlices * RR + 8) * 2 + 15) / 16;  // f32x4 worth of T
  static constexpr int kBuf = kRed > kH ? kRed : kH;
  static constexpr int kStage = (kWaves * 16 * kStageStride * static_cast<int>(sizeof(T)) + 15) / 16;
  static constexpr int kStg = SMT > 0 ? (kWaves * stg_elems_per_wave<(SMT > 0 ? SMT : 1)>() * static_cast<int>(sizeof(T)) + 15) / 16 : 0;
  f32x4 mem[kBuf + kStage > kStg ? kBuf + kStage : kStg];
  __device__ f32x4* buf() { return mem; }
  __device__ T* stage() { return reinterpret_cast<T*>(mem + kBuf); }  // each wave's Y tile (expand)
  __device__ T* stg() { return reinterpret_cast<T*>(mem); }
};

// TILES: token tiles in flight per workgroup in expand() (4 for plans of
// 64-token blocks, else 1); the fused kernel always works with 1.
//
// The leading scalar arguments repeat what a workgroup needs before its
// first memory access (the plan's header, blocks and token lists, and the
// grid's split into roles).  The library is built with kernarg preloading
// (-amdgpu-kernarg-preload-count), so these arrive in SGPRs at wave launch
// and the plan loads go out without a kernel-argument load ahead of them.
template <typename T, int RANK, int ROLE, int TILES, bool PA>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(waves_per_simd<RANK, ROLE, TILES>())))
void apply_kernel(const uint32_t* header, const Block* __restrict__ blocks,
                  const int32_t* __restrict__ bperm, int32_t per_shrink, int32_t n_shrink, int32_t per_block,
                  ApplyArgs a) {
  // Arguments: ApplyKernelArgs.  Their lines are loaded here and, in the shared-A kernels,
  // waited for with the plan loads below (cfg2 step 1177 -> 1166 us, cfg3
  // 122.3 -> 120.6 us per layer, against waiting here, which made the
  // mixed-rank ones slower); the fixed-rank one-A-per-slice kernels wait here
  // (cfg5's 44-launch step 430 vs 437 us); the mixed-rank ones wait with the
  // plan loads (cfg3's gate and up in one launch 123.9 -> 122.6 us per layer).
  constexpr int kArgBytes = static_cast<int>(sizeof(ApplyKernelArgs));
  uint32_t ka_touch = 0;
  if constexpr (RANK != 0 && PA) touch_kernel_args<kArgBytes>();
  if constexpr (!PA || RANK == 0) ka_touch = touch_kernel_args_issue<kArgBytes>();
  using SM = SharedMem<T, RANK, ROLE == kFused ? 1 : (ROLE == kExpandOnly ? 0 : kShrinkRowsFused / 16)>;
  __shared__ SM smem;
  __shared__ int s_flag;
  trace_stamp(a, 0);
  f32x4* s_red = smem.buf();
  T* s_h = reinterpret_cast<T*>(smem.buf());
  const int S = ROLE == kExpandOnly ? 0 : n_shrink;
  const int wg = static_cast<int>(blockIdx.x);
  // shrink() with a.red_first: the block reducers are workgroups
  // 0..n_slots-1, resident from the start, and the shrink workgroups follow.
  const bool red_first = ROLE == kShrinkOnly && a.red_first != 0;
  const bool shrink_role = ROLE != kExpandOnly && (red_first ? wg >= a.n_slots : wg < S);
  int b, part;
  if (shrink_role) {
    const int sw = red_first ? wg - a.n_slots : wg;
    b = sw / per_shrink;
    part = sw - b * per_shrink;
  } else {
    const int e = red_first ? wg : wg - S;
    b = e / per_block;
    part = e - b * per_block;
  }
  // Independent loads: block count, block descriptor, this lane's first token
  // (blocks and bperm hold every slot of the grid).  The exit test reads all
  // three so that they are issued together, one memory latency in all:
  // tested on the count alone, the compiler would load the descriptor and the
  // token only after the count had arrived.
  const int n_blocks = static_cast<int>(header[kHdrNumBlocks]);
  // Roles that use the partial buffer do nothing while it is poisoned.
  const uint32_t poison = ROLE == kExpandOnly ? 0u : header[kHdrPoison];
  const Block blk = blocks[b];
  const int row = threadIdx.x & 15;
  const int32_t tok0 = bperm[static_cast<int64_t>(b) * kBlockTokens + row];
  // Table mode on a device plan: the block's entry as the plan build copied
  // it, loaded with the descriptor, used while no table write has followed
  // that build (one memory latency less before the first weight load).
  // Only in shrink()'s and expand()'s roles and the mixed-rank fused kernels
  // (table mode only): in the fixed-rank fused kernels, which stacked-weight
  // decode calls use, the test alone cost 0.3 us per qkv call and the
  // entry's registers a wave per SIMD at ranks 8-32 (cfg2 step 1217 -> 1227
  // us, cfg5's 88 calls 697 -> 736 us, measured on MI355X).
  PreEntry pre;
  if constexpr (ROLE == kShrinkOnly || ROLE == kExpandOnly || RANK == 0) {
    if (a.w.mode == kTable && a.w.a_base[0] != nullptr) {
      pre.en = load_entry(static_cast<const Entry*>(a.w.a_base[0]) + b);
      pre.ok = header[kHdrTableVer] == header[kHdrPlanVer];
    }
  }
  // A plan with more blocks than the grid's slots (only routings that name
  // ids the call cannot resolve produce one) is reported, not silently cut.
  if (b == a.n_slots - 1 && part == 0 && threadIdx.x == 0 && n_blocks > a.n_slots)
    flag_error(a.plan.header, kErrCapacity);
  if constexpr (!PA || RANK == 0) touch_kernel_args_wait(ka_touch);
  if ((b >= n_blocks) | (blk.count <= 0) | (tok0 < -1) | (poison != 0u)) return;
  const int32_t t0 = row < blk.count ? tok0 : -1;
  trace_stamp(a, 1);
  trace_tag(a, (shrink_role ? 1u : 2u) | (static_cast<uint64_t>(b) << 8));

  if (shrink_role) {
    // part = (A slice, rank group, d-range), d-range fastest.
    const int per_a = a.n_chunks * a.n_rgroups;
    const int sa = PA ? part / per_a : 0;
    const int k = part - sa * per_a;
    const int rg = k / a.n_chunks;
    const int c = k - rg * a.n_chunks;
    const Resolved<T> res = resolve_a<T, PA>(a, blk, sa, pre);
    // Each slice's first workgroup reports its resolution error.
    if (res.err != 0 && k == 0 && threadIdx.x == 0) flag_error(a.plan.header, res.err);
    if constexpr (ROLE == kFusedMulti || ROLE == kShrinkOnly) {
      shrink_body<T, kShrinkRowsFused / 16>(a, b, c, sa, rg * kShrinkRowsFused, blk, t0, res, s_red, smem.stg());
    } else {
      shrink_body<T, 1>(a, b, c, sa, rg * kShrinkRows, blk, t0, res, s_red, smem.stg());
    }
    return;
  }
  if constexpr (ROLE == kShrinkOnly) {
    reduce_to_h<T>(a, b, blk, &s_flag, pre);
  } else if constexpr (RANK != 0) {
    expand_body<T, RANK, ROLE, TILES, PA>(a, b, part, blk, t0, s_h, smem.stage(), &s_flag, pre);
  } else if constexpr (PA) {
    // Mixed ranks with one A per slice (zero-padded slices): every block at
    // the largest rank, B read at each adapter's own row stride.
    expand_body<T, kMaxRank, ROLE, TILES, PA>(a, b, part, blk, t0, s_h, smem.stage(), &s_flag, pre);
  } else if constexpr (ROLE == kFusedMulti) {
    // Mixed ranks over several chunks per workgroup: one body at the largest
    // rank (four per-rank bodies here spill).
    expand_body<T, kMaxRank, ROLE, TILES, false, true>(a, b, part, blk, t0, s_h, smem.stage(), &s_flag, pre);
  } else {
    // Mixed ranks: the block's adapter decides (resolved again inside).
    const Resolved<T> r0 = resolve_b<T>(a, blk, 0, pre);
    switch (r0.rank) {
      case 16: expand_body<T, 16, ROLE, TILES, PA>(a, b, part, blk, t0, s_h, smem.stage(), &s_flag, pre); break;
      case 32: expand_body<T, 32, ROLE, TILES, PA>(a, b, part, blk, t0, s_h, smem.stage(), &s_flag, pre); break;
      case 64: expand_body<T, 64, ROLE, TILES, PA>(a, b, part, blk, t0, s_h, smem.stage(), &s_flag, pre); break;
      default: expand_body<T, 8, ROLE, TILES, PA>(a, b, part, blk, t0, s_h, smem.stage(), &s_flag, pre); break;
    }
  }
}

// ------------------------------------------------------------- shrink() ----
//
// shrink(), and the shrink half of large-plan add_lora calls: one workgroup
// per (block, d-range) computes every rank row of the block, so each X
// element is read once per call.  The d-range is streamed in K-slices of
// kSliceK elements, software pipelined one slice ahead: the slice of A
// (rank rows x kSliceK) is loaded once per workgroup and shared by the four
// waves through LDS (double buffered), and each wave, which owns one
// 16-token tile, loads its X fragments straight into registers.  The
// block's d-ranges are summed by its last workgroup to finish (a per-block
// counter), in d-range order, so the bits do not depend on timing; nothing
// waits on another workgroup.
constexpr int kSliceK = 128;
constexpr int kSliceStride = kSliceK + 8;  // LDS row stride of an A slice: 16-byte skew per row

template <typename T, int MAXR, bool kMixed>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(kShrinkWavesPerSimd)))
void shrink_kernel(ApplyArgs a) {
  using V8 = typename VecOf<T>::v8;
  constexpr int MT = (MAXR + 15) / 16;          // 16-row MFMA tiles of the largest rank
  constexpr int KS = kSliceK / 32;              // K-steps per slice
  constexpr int XL = 16 * kSliceK / (64 * 8);   // a wave's whole-row X loads per slice (4)
  __shared__ T s_a[2][MT * 16 * kSliceStride];
  // Each wave's X tile of the current slice: only that wave reads it, after
  // writing it, so one buffer suffices.
  __shared__ T s_x[kWaves][16 * kSliceStride];
  __shared__ int s_last;
  const int tid = static_cast<int>(threadIdx.x);
  const int n_kc = a.n_chunks;
  const int b = static_cast<int>(blockIdx.x) / n_kc;
  const int c = static_cast<int>(blockIdx.x) - b * n_kc;
  trace_stamp(a, 0);
  trace_hw(a);
  const int n_blocks = static_cast<int>(a.plan.header[kHdrNumBlocks]);
  if (b == a.n_slots - 1 && c == 0 && tid == 0 && n_blocks > a.n_slots) flag_error(a.plan.header, kErrCapacity);
  if (b >= n_blocks) return;
  const Block blk = a.plan.blocks[b];
  const Resolved<T> res = resolve_a<T>(a, blk);
  if (res.ptr == nullptr) {
    if (res.err != 0 && c == 0 && tid == 0) flag_error(a.plan.header, res.err);
    return;
  }
  trace_tag(a, 3u | (static_cast<uint64_t>(b) << 8) | (static_cast<uint64_t>(c) << 32));
  trace_stamp(a, 1);
  const int rank = kMixed ? res.rank : MAXR;
  const int n_mt = kMixed ? (rank + 15) >> 4 : MT;
  const int d = a.d_model;
  // The d-range [c * dc, ...) in groups of kShrinkSlices slices; k0/k1 are
  // the current group's bounds.
  const int kc_end = min((c + 1) * a.dc, d);
  int k0 = c * a.dc;
  int k1 = min(k0 + kShrinkSlices * kSliceK, kc_end);
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int row = lane & 15;
  const int kq = (lane >> 4) * 8;
  const int tl = wave * 16 + row;  // this lane's token slot in the block (MFMA layout)
  const int32_t* bp = a.plan.bperm + static_cast<int64_t>(b) * kBlockTokens;
  const int32_t tok = tl < blk.count ? bp[tl] : -1;
  const bool wave_live = wave * 16 < blk.count;
  // Every load below is unconditional, at an address clamped into the
  // operand (a missing token reads X row 0, a rank row past the adapter's
  // reads its last row, a column past the d-range its last 8 columns); what
  // is not part of the product is zeroed where the data is used.  Straight
  // loads let the compiler wait for exactly the slice it needs while the
  // next one stays in flight.
  // X is loaded in whole rows (16 lanes per 256-byte row of a slice; lane
  // moves 8 elements of rows xrow + 4i of its wave's tile) into the wave's
  // LDS tile and read back in the MFMA layout: X loaded straight in the MFMA
  // layout moves 64 bytes of 16 rows per instruction, 4.6 vs 6.2 TB/s for
  // the same bytes, measured on MI355X.
  const int xrow = lane >> 4;
  const int xcol = (lane & 15) * 8;
  const T* xr[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int t = wave * 16 + xrow + 4 * i;
    const int32_t tk = t < blk.count ? bp[t] : -1;
    xr[i] = static_cast<const T*>(a.x) + static_cast<int64_t>(tk >= 0 ? tk : 0) * a.ldx;
  }
  T* sx = s_x[wave];
  // A slice loads: thread t moves 8 elements of rows t/16 + 16p.
  const int arow = tid >> 4;
  const int acol = (tid & 15) * 8;
  // Element offsets from the adapter's A (rank x d < 2^31 elements).
  const int arow0 = min(arow, rank - 1) * d;
  struct Slice {
    u32x4 a[MT];
    u32x4 x[XL];
  };
  auto load_slice = [&](Slice& sl, int ks0) {
#pragma unroll
    for (int p = 0; p < MT; ++p) {
      const int off = (kMixed ? min(p * 16 + arow, rank - 1) * d : arow0 + p * 16 * d) + min(ks0 + acol, k1 - 8);
      sl.a[p] = load16_global(res.ptr + off);
    }
#pragma unroll
    for (int i = 0; i < XL; ++i) sl.x[i] = load16_global(xr[i] + min(ks0 + xcol, k1 - 8));
  };
  f32x4 acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Slice at ks0 from `sl` (landed) through LDS buffer `buf`; then `sl`
  // takes the slice two ahead, next_k (past the range's last slice it
  // re-reads one of its slices, which is never used).
  auto run_slice = [&](Slice& sl, int buf, int ks0, bool live, bool more, int next_k) {
#pragma unroll
    for (int p = 0; p < MT; ++p) {
      const bool ok = ks0 + acol < k1 && (!kMixed || p * 16 + arow < rank);
      *reinterpret_cast<u32x4*>(&s_a[buf][(p * 16 + arow) * kSliceStride + acol]) = ok ? sl.a[p] : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < XL; ++i) *reinterpret_cast<u32x4*>(&sx[(xrow + 4 * i) * kSliceStride + xcol]) = sl.x[i];
    // The slice is in LDS for every wave; the other buffer was last read
    // before this barrier, so the next slice may be written into it.
    lds_barrier();
    if (wave_live && live) {
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const V8 xv = __builtin_bit_cast(V8, *reinterpret_cast<const u32x4*>(&sx[row * kSliceStride + s * 32 + kq]));
        const V8 xf = (tok >= 0 && ks0 + s * 32 + kq < k1) ? xv : zero8<T>();
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          if (!kMixed || m < n_mt) {
            const V8 af = __builtin_bit_cast(
                V8, *reinterpret_cast<const u32x4*>(&s_a[buf][(m * 16 + row) * kSliceStride + s * 32 + kq]));
            acc[m] = mfma16(af, xf, acc[m]);
          }
        }
      }
    }
    if (more) load_slice(sl, next_k);
  };
  // Fully unrolled over the workgroup's kShrinkSlices slices: every path
  // issues the same loads, so each wait is for exactly one slice.  A short
  // last d-range skips the MFMAs of its missing slices, not their loads.
  // Blocks of one adapter read the same A slices; each block starts at a
  // different slice of its range (rotation by block index) so that they do
  // not all hit the same lines at once.
  Slice s0, s1;
  for (; k0 < kc_end; k0 += kShrinkSlices * kSliceK, k1 = min(k0 + kShrinkSlices * kSliceK, kc_end)) {
    const int n_sl = (k1 - k0 + kSliceK - 1) / kSliceK;
    const int rot = b % n_sl;
    auto slice_k = [&](int i) { return k0 + (i + rot < n_sl ? i + rot : i + rot - n_sl) * kSliceK; };
    load_slice(s0, slice_k(0));
    load_slice(s1, slice_k(1 % n_sl));
#pragma unroll
    for (int i = 0; i < kShrinkSlices; i += 2) {
      run_slice(s0, 0, slice_k(i % n_sl), i < n_sl, i + 2 < kShrinkSlices, slice_k((i + 2) % n_sl));
      run_slice(s1, 1, slice_k((i + 1) % n_sl), i + 1 < n_sl, i + 3 < kShrinkSlices, slice_k((i + 3) % n_sl));
    }
  }
  trace_stamp(a, 2);
  // acc[m]: ranks m*16 + 4*(lane/16) + [0, 4) of token slot tl.
  const int rq = (lane >> 4) * 4;
  T* H = static_cast<T*>(a.h);
  // fp32 H (vLLM's lora_shrink buffer): alpha * sum added to it, unrounded.
  const bool f32 = a.h_f32 != 0;
  auto put_h = [&](int64_t at, f32x4 v) {
    if (f32) {
      f32x4* hp = reinterpret_cast<f32x4*>(static_cast<float*>(a.h) + at);
      *hp = *hp + v;
    } else {
      store4(H + at, v);
    }
  };
  if (n_kc == 1) {
    if (tok >= 0) {
#pragma unroll
      for (int m = 0; m < MT; ++m)
        if (m * 16 + rq < rank) put_h(static_cast<int64_t>(tok) * a.ldh + m * 16 + rq, acc[m] * res.alpha);
    }
    return;
  }
  // Partial of this d-range, stored coherently; the stores have landed
  // before the count (s_waitcnt), so the last workgroup sees them all.
  if (tok >= 0) {
    float* prow = a.part + (static_cast<int64_t>(c) * a.ptok + blk.first + tl) * a.hs;
#pragma unroll
    for (int m = 0; m < MT; ++m)
      if (m * 16 + rq < rank) coherent_store_f4(prow + m * 16 + rq, acc[m]);
  }
  wait_vm();
  __syncthreads();
  uint32_t* counter = &a.consumed[static_cast<int64_t>(b) * kCounterStride];
  if (tid == 0) s_last = atomic_add_u(counter, 1u) == static_cast<unsigned>(n_kc - 1) ? 1 : 0;
  __syncthreads();
  trace_stamp(a, 3);
  if (s_last == 0) return;
  // Last workgroup of the block: H = rn(alpha * sum_c part[c]) in d-range
  // order, then the counter is reset for the next call.  The partials are
  // left as they are: every launch writes each word it later reads (the
  // buffer is shrink()'s own, not the fused calls' with its empty pattern).
  const int r4 = rank >> 2;
  const int units = blk.count * r4;
  const int64_t cs = static_cast<int64_t>(a.ptok) * a.hs;
  // A thread's units are tid + 256 i (at most kBlockTokens * kMaxRank / 4 /
  // 256 = 4); their loads go out together, four d-ranges at a time.
  constexpr int kUnits = kBlockTokens * kMaxRank / 4 / kThreads;
  const float* p0[kUnits];
  f32x4 sum[kUnits];
#pragma unroll
  for (int i = 0; i < kUnits; ++i) {
    const int u = min(tid + i * kThreads, units - 1);
    const int j = u / r4;
    p0[i] = a.part + (static_cast<int64_t>(blk.first) + j) * a.hs + (u - j * r4) * 4;
    sum[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  for (int c0 = 0; c0 < n_kc; c0 += 4) {
    f32x4 v[4][kUnits];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int i = 0; i < kUnits; ++i) v[q][i] = coherent_load_f4(p0[i] + min(c0 + q, n_kc - 1) * cs);
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int i = 0; i < kUnits; ++i)
        if (c0 + q < n_kc) sum[i] += v[q][i];
  }
#pragma unroll
  for (int i = 0; i < kUnits; ++i) {
    const int u = tid + i * kThreads;
    if (u < units) {
      const int j = u / r4;
      const int32_t tj = a.plan.bperm[static_cast<int64_t>(b) * kBlockTokens + j];
      put_h(static_cast<int64_t>(tj) * a.ldh + (u - j * r4) * 4, sum[i] * res.alpha);
    }
  }
  if (tid == 0) atomic_store_u(counter, 0u);
  trace_stamp(a, 4);
}

template <typename T>
hipError_t launch_shrink_t(const ApplyArgs& a0, hipStream_t stream) {
  const int64_t n = static_cast<int64_t>(a0.n_slots) * a0.n_chunks;
  if (n <= 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(n));
  ApplyArgs a = a0;
  if (a.trace != nullptr && n * kTraceWords > a.trace_words) a.trace = nullptr;
  switch (a.rank) {
    case 8: shrink_kernel<T, 8, false><<<grid, kThreads, 0, stream>>>(a); break;
    case 16: shrink_kernel<T, 16, false><<<grid, kThreads, 0, stream>>>(a); break;
    case 32: shrink_kernel<T, 32, false><<<grid, kThreads, 0, stream>>>(a); break;
    case 64: shrink_kernel<T, 64, false><<<grid, kThreads, 0, stream>>>(a); break;
    case 0:  // mixed ranks: each block's adapter decides, up to kMaxRank
      shrink_kernel<T, kMaxRank, true><<<grid, kThreads, 0, stream>>>(a);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T, int RANK, int ROLE, int TILES>
void launch_kernel(const ApplyArgs& a, dim3 grid, int32_t per_shrink, int32_t n_shrink, int32_t per_block,
                   hipStream_t stream) {
  // One A per slice only in the fused roles; a separate instantiation, so the
  // shared-A kernels keep their constant indexing and single-probe gate.
  if constexpr (ROLE == kFused || ROLE == kFusedMulti) {
    if (a.w.n_a > 1) {
      apply_kernel<T, RANK, ROLE, TILES, true><<<grid, kThreads, 0, stream>>>(
          a.plan.header, a.plan.blocks, a.plan.bperm, per_shrink, n_shrink, per_block, a);
      return;
    }
  }
  apply_kernel<T, RANK, ROLE, TILES, false><<<grid, kThreads, 0, stream>>>(a.plan.header, a.plan.blocks, a.plan.bperm,
                                                                          per_shrink, n_shrink, per_block, a);
}

template <typename T, int ROLE, int TILES>
hipError_t launch_rank(const ApplyArgs& a, hipStream_t stream) {
  const int64_t S = ROLE == kExpandOnly ? 0 : static_cast<int64_t>(a.n_slots) * a.n_chunks * a.n_rgroups * a.w.n_a;
  const int64_t E = static_cast<int64_t>(a.n_slots) *
                    ((a.n_ochunks + a.n_sub - 1) / a.n_sub);
  const int64_t n = S + E;
  if (n <= 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(n));
  const int32_t per_shrink = a.n_chunks * a.n_rgroups * a.w.n_a;
  const int32_t per_block = (a.n_ochunks + a.n_sub - 1) / a.n_sub;
  const int32_t ns = static_cast<int32_t>(S);
  ApplyArgs at;
  if (a.trace != nullptr && n * kTraceWords > a.trace_words) {
    at = a;
    at.trace = nullptr;
  }
  const ApplyArgs& a2 = (a.trace != nullptr && n * kTraceWords > a.trace_words) ? at : a;
  if constexpr (ROLE == kShrinkOnly) {
    // Its shrink side takes the rank from each block's adapter.
    launch_kernel<T, 0, ROLE, TILES>(a2, grid, per_shrink, ns, per_block, stream);
  } else {
    switch (a.rank) {
      case 0:  // mixed ranks (registered adapters): each block's adapter decides
        launch_kernel<T, 0, ROLE, TILES>(a2, grid, per_shrink, ns, per_block, stream);
        break;
      case 8: launch_kernel<T, 8, ROLE, TILES>(a2, grid, per_shrink, ns, per_block, stream); break;
      case 16: launch_kernel<T, 16, ROLE, TILES>(a2, grid, per_shrink, ns, per_block, stream); break;
      case 32: launch_kernel<T, 32, ROLE, TILES>(a2, grid, per_shrink, ns, per_block, stream); break;
      case 64: launch_kernel<T, 64, ROLE, TILES>(a2, grid, per_shrink, ns, per_block, stream); break;
      default: return hipErrorInvalidValue;
    }
  }
  return hipGetLastError();
}

template <int ROLE>
hipError_t launch_role(int dtype_bf16, const ApplyArgs& a, hipStream_t stream) {
  if constexpr (ROLE != kFused && ROLE != kFusedMulti) {
    if (a.tiles > 1)
      return dtype_bf16 ? launch_rank<__bf16, ROLE, kTilesInFlight>(a, stream)
                        : launch_rank<_Float16, ROLE, kTilesInFlight>(a, stream);
  }
  return dtype_bf16 ? launch_rank<__bf16, ROLE, 1>(a, stream) : launch_rank<_Float16, ROLE, 1>(a, stream);
}

// ------------------------------------------------------- linear + LoRA ----
//
// y = rn(rn(x . W^T + bias) + H_tok . B_tok^T), H = rn(scale . x . A_tok^T):
// a decode step's base linear and its per-token LoRA delta (add_lora's
// stacked weights, device plan of 16-token blocks) in one launch.  Roles, in
// dispatch order; a role waits only on roles dispatched before it, so the
// waits end whatever the residency:
//   * shrink workgroups: the fused kernels' (block, rank group, d-range)
//     partials of H into the partial buffer;
//   * one reducer per block: the block's H rows (token-indexed, device-
//     coherent stores) from its partials, kPartialEmpty restored, then the
//     block's H flag set;
//   * GEMM workgroups (token group g of kLinTokens, column tile of kLinCols
//     outputs, K-range s of l.splits): x . W^T over the K-range into the GEMM
//     partial buffer.  X goes through a wave-private LDS tile in whole rows
//     and W through a shared, double-buffered one (K-slices of kSliceK); each
//     wave owns 32 tokens.  The tile's last workgroup to count sums the
//     partials in K order, adds the bias and rounds (the base output), waits
//     for every block's H flag, adds each block's H . B^T (one MFMA per 32
//     ranks) into the tokens' rows, rounds and stores y; it then counts itself
//     on every block's flag, and the flag's last reader clears it.
constexpr int kLinTokens = 128;
constexpr int kLinCols = 16;
constexpr int kLinWavesPerSimd = 3;  // its LDS (43.5 KB) holds three workgroups per compute unit
constexpr int kLinDeltaBlocks = 8;   // blocks a wave of the epilogue has in flight (half at rank 64)

template <typename T>
__device__ __forceinline__ void coherent_store_pair(T* p, float x, float y) {
  typename VecOf<T>::v2 o;
  o[0] = static_cast<T>(x);
  o[1] = static_cast<T>(y);
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __builtin_bit_cast(uint32_t, o), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T, int RANK>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(kLinWavesPerSimd)))
void linear_kernel(const uint32_t* header, const Block* __restrict__ blocks, const int32_t* __restrict__ bperm,
                   int32_t n_shrink, ApplyArgs a, LinearArgs l) {
  using V8 = typename VecOf<T>::v8;
  constexpr int KS = (RANK + 31) / 32;
  constexpr int XL = 32 * kSliceK / (64 * 8);      // a wave's whole-row X loads per slice (8)
  constexpr int WL = kLinCols * kSliceK / (kThreads * 8);  // W loads per thread per slice (1)
  static_assert(WL == 1, "one W load per thread and slice");
  // sx: each wave's 32 X rows of the slice; sw: the slice's W rows, double
  // buffered.  The epilogue's fp32 tile reuses sx.
  __shared__ T sx[kLinTokens * kSliceStride];
  __shared__ T sw[2][kLinCols * kSliceStride];
  __shared__ int s_flag;
  __shared__ int s_hok;  // the epilogue's H flags seen (s_flag still holds the last-arriver test)
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int row = lane & 15;
  const int kq = (lane >> 4) * 8;
  const int wg = static_cast<int>(blockIdx.x);
  // Blocks the grid has reducer slots for; a plan with more (only ids the
  // call cannot resolve make one) is reported, and the rest skipped.
  const int n_plan = static_cast<int>(header[kHdrNumBlocks]);
  const int n_blocks = min(n_plan, a.n_slots);
  if (wg == 0 && tid == 0 && n_plan > a.n_slots) flag_error(a.plan.header, kErrCapacity);
  const uint32_t poison = header[kHdrPoison];
  trace_stamp(a, 0);

  if (wg < n_shrink) {
    // --- shrink: the kShrinkOnly role's split (32-row rank groups).
    const int per = a.n_chunks * a.n_rgroups;
    const int b = wg / per;
    const int part = wg - b * per;
    const int rg = part / a.n_chunks;
    const int c = part - rg * a.n_chunks;
    if (b >= n_blocks || poison != 0u) return;
    const Block blk = blocks[b];
    const int32_t tok0 = bperm[static_cast<int64_t>(b) * kBlockTokens + row];
    const int32_t t0 = row < blk.count ? tok0 : -1;
    const Resolved<T> res = resolve_a<T>(a, blk);
    if (res.err != 0 && part == 0 && tid == 0) flag_error(a.plan.header, res.err);
    trace_tag(a, 1u | (static_cast<uint64_t>(b) << 8));
    trace_stamp(a, 1);
    shrink_body<T, kShrinkRowsFused / 16>(a, b, c, 0, rg * kShrinkRowsFused, blk, t0, res,
                                          reinterpret_cast<f32x4*>(sx));
    return;
  }
  if (wg < n_shrink + a.n_slots) {
    // --- reducer of block b: H rows, then the flag.
    const int b = wg - n_shrink;
    if (b >= n_blocks) return;
    const Block blk = blocks[b];
    trace_tag(a, 4u | (static_cast<uint64_t>(b) << 8));
    if (poison == 0u) {
      const Resolved<T> res = resolve_a<T>(a, blk);
      const int wrote = res.ptr != nullptr ? res.rank : 0;
      trace_stamp(a, 1);
      if (wrote > 0) {
        bool ok = true;
        if (blk.count * wrote * a.n_chunks > 2048) ok = wait_partials<false>(a, blk, wrote, &s_flag);
        trace_stamp(a, 2);
        if (ok) {
          T* H = static_cast<T*>(a.h);
          const int32_t* toks = bperm + static_cast<int64_t>(b) * kBlockTokens;
          collect_partials<8>(a, blk, wrote / 2, res.alpha, [&](int j, int r0, f32x2 v) {
            coherent_store_pair<T>(H + static_cast<int64_t>(toks[j]) * a.ldh + r0, v[0], v[1]);
          });
          __syncthreads();
          clear_partials(a, blk, wrote, tid, kThreads);
        }
      }
    }
    // The H stores have landed (s_waitcnt) before the flag.
    wait_vm();
    __syncthreads();
    trace_stamp(a, 3);
    if (tid == 0) atomic_store_u(&l.hflag[b], 1u);
    return;
  }

  // --- GEMM.
  const int n_tiles = l.n_out / kLinCols;
  const int gw = wg - n_shrink - a.n_slots;
  const int ks = gw % l.splits;
  const int jt = (gw / l.splits) % n_tiles;
  const int g = gw / (l.splits * n_tiles);
  trace_tag(a, 5u | (static_cast<uint64_t>(g * n_tiles + jt) << 8) | (static_cast<uint64_t>(ks) << 32));
  const int K = a.d_model;
  const int kb = ks * l.k_range;
  const int ke = min(kb + l.k_range, K);
  const int n_sl = (ke - kb) / kSliceK;
  const int xrow = lane >> 4;
  const int xcol = (lane & 15) * 8;
  const T* X = static_cast<const T*>(a.x);
  const T* Wt = static_cast<const T*>(l.w);
  // This lane's X rows (clamped to the last token: rows past T are computed
  // and never stored) and its W row.
  const T* xr[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int t = g * kLinTokens + wave * 32 + xrow + 4 * i;
    xr[i] = X + static_cast<int64_t>(min(t, l.tokens - 1)) * a.ldx;
  }
  const T* wr = Wt + static_cast<int64_t>(jt * kLinCols + (tid >> 4)) * l.ldw + (tid & 15) * 8;
  T* sxw = sx + wave * 32 * kSliceStride;
  struct Slice {
    u32x4 x[XL];
    u32x4 w;
  };
  auto load_slice = [&](Slice& sl, int i) {
    const int k = kb + min(i, n_sl - 1) * kSliceK;
#pragma unroll
    for (int q = 0; q < XL; ++q) sl.x[q] = load16_global(xr[q] + k + xcol);
    sl.w = load16_global(wr + k);
  };
  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  auto run_slice = [&](Slice& sl, int buf, int i) {
#pragma unroll
    for (int q = 0; q < XL; ++q) *reinterpret_cast<u32x4*>(&sxw[(xrow + 4 * q) * kSliceStride + xcol]) = sl.x[q];
    *reinterpret_cast<u32x4*>(&sw[buf][(tid >> 4) * kSliceStride + (tid & 15) * 8]) = sl.w;
    lds_barrier();
    if (i < n_sl) {
#pragma unroll
      for (int s = 0; s < kSliceK / 32; ++s) {
        const V8 wf = __builtin_bit_cast(V8, *reinterpret_cast<const u32x4*>(&sw[buf][row * kSliceStride + s * 32 + kq]));
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          const V8 xf = __builtin_bit_cast(
              V8, *reinterpret_cast<const u32x4*>(&sxw[(m * 16 + row) * kSliceStride + s * 32 + kq]));
          acc[m] = mfma16(wf, xf, acc[m]);
        }
      }
    }
    load_slice(sl, i + 2);
  };
  Slice s0, s1;
  load_slice(s0, 0);
  load_slice(s1, 1);
  for (int i = 0; i < n_sl; i += 2) {
    run_slice(s0, 0, i);
    run_slice(s1, 1, i + 1);
  }
  trace_stamp(a, 1);
  // Epilogue state (if this workgroup turns out to be its tile's last): the
  // blocks of this wave, NB at a time, their token rows and their B rows
  // jt*16 + row (the delta MFMA's A operand).  A lane's token is -1 past its
  // block or when the block's adapter is out of range.
  constexpr int kUnits = kLinTokens * kLinCols / 4 / kThreads;  // f32x4 units per thread (2)
  constexpr int kSumBatch = 8;                                  // K-split partials per load batch
  constexpr int NB = RANK <= 32 ? kLinDeltaBlocks : kLinDeltaBlocks / 2;
  Block blk[NB];
  int32_t tk[NB];
  V8 bf[NB][KS];
  auto load_blocks = [&](int b0) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int b = b0 + i;
      blk[i] = b < n_blocks ? blocks[b] : Block{-1, 0, 0, -1};
      tk[i] = b < n_blocks ? bperm[static_cast<int64_t>(b) * kBlockTokens + row] : -1;
    }
  };
  auto load_b = [&]() {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const Resolved<T> rb = resolve_b<T>(a, blk[i], 0);
      if (row >= blk[i].count || rb.ptr == nullptr) tk[i] = -1;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int k = s * 32 + kq;
        bf[i][s] = rb.ptr != nullptr && k < RANK
                       ? load8(rb.ptr + static_cast<int64_t>(jt * kLinCols + row) * RANK + k)
                       : zero8<T>();
      }
    }
  };
  // acc[m]: output columns jt*16 + 4*(lane/16) + [0, 4) of token
  // g*128 + wave*32 + m*16 + lane%16.  Stored coherently; counted below.
  const int rq = (lane >> 4) * 4;
  const int64_t tile = static_cast<int64_t>(g) * n_tiles + jt;
  float* gp = l.gpart + tile * l.splits * (kLinTokens * kLinCols);
#pragma unroll
  for (int m = 0; m < 2; ++m)
    coherent_store_f4(gp + static_cast<int64_t>(ks) * (kLinTokens * kLinCols) + (wave * 32 + m * 16 + row) * kLinCols + rq,
                      acc[m]);
  wait_vm();
  __syncthreads();
  trace_stamp(a, 2);
  if (tid == 0) s_flag = atomic_add_u(&l.tile_cnt[tile], 1u) == static_cast<unsigned>(l.splits - 1) ? 1 : 0;
  __syncthreads();
  trace_stamp(a, 3);
  if (s_flag == 0) return;

  // --- epilogue of the tile (one workgroup): base output, then the delta.
  // The first batch of K-split partials goes out with this wave's first
  // blocks and token rows, then their B rows; the H flags are polled once
  // the base is summed, and only the H rows load after that.
  float* et = reinterpret_cast<float*>(sx);  // [kLinTokens][kLinCols] fp32
  f32x4 sum[kUnits];
  auto load_sums = [&](int s0, f32x4(&v)[kSumBatch][kUnits]) {
#pragma unroll
    for (int q = 0; q < kSumBatch; ++q)
#pragma unroll
      for (int i = 0; i < kUnits; ++i)
        v[q][i] = s0 + q < l.splits ? coherent_load_f4(gp + static_cast<int64_t>(s0 + q) * (kLinTokens * kLinCols) +
                                                       (tid + i * kThreads) * 4)
                                    : f32x4{0.f, 0.f, 0.f, 0.f};
  };
#pragma unroll
  for (int i = 0; i < kUnits; ++i) sum[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < l.splits; s0 += kSumBatch) {
    f32x4 v[kSumBatch][kUnits];
    load_sums(s0, v);
    if (s0 == 0) load_blocks(wave * NB);
#pragma unroll
    for (int i = 0; i < kUnits; ++i)
#pragma unroll
      for (int q = 0; q < kSumBatch; ++q) sum[i] += v[q][i];
  }
  load_b();
#pragma unroll
  for (int i = 0; i < kUnits; ++i) {
    const int u = tid + i * kThreads;
    const int c4 = (u * 4) % kLinCols;
    if (l.bias != nullptr) {
      const T* bias = static_cast<const T*>(l.bias) + jt * kLinCols + c4;
#pragma unroll
      for (int q = 0; q < 4; ++q) sum[i][q] += static_cast<float>(bias[q]);
    }
    // The base output is rounded to the I/O type, as the base linear's is.
#pragma unroll
    for (int q = 0; q < 4; ++q) sum[i][q] = static_cast<float>(static_cast<T>(sum[i][q]));
    *reinterpret_cast<f32x4*>(et + u * 4) = sum[i];
  }
  if (tid == 0) atomic_store_u(&l.tile_cnt[tile], 0u);
  // Every block's H flag (one wave polls, bounded; after a give-up, or
  // while the partial buffer is poisoned, the delta is left out).
  if (tid < 64) {
    int ok = poison == 0u ? 1 : 0;
    for (unsigned spins = 0; ok; ++spins) {
      bool here = true;
      for (int b = lane; b < n_blocks; b += 64) here = here && atomic_load_u(&l.hflag[b]) != 0u;
      if (__all(here)) break;
      if (spins >= a.spin_limit || poisoned(a.plan.header)) {
        ok = 0;
        if (lane == 0 && spins >= a.spin_limit) give_up(a.plan.header);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    // A give-up elsewhere in the call leaves H unreliable: no delta then.
    if (lane == 0) s_hok = ok && !poisoned(a.plan.header);
  }
  trace_stamp(a, 4);
  __syncthreads();
  trace_stamp(a, 5);
  if (s_hok != 0) {
    const T* H = static_cast<const T*>(a.h);
    // NB blocks per wave at a time; each token is in one block, so the
    // waves add into distinct rows of et.
    for (int b0 = wave * NB; b0 < n_blocks; b0 += kWaves * NB) {
      if (b0 != wave * NB) {
        load_blocks(b0);
        load_b();
      }
      V8 hf[NB][KS];
#pragma unroll
      for (int i = 0; i < NB; ++i) {
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const int k = s * 32 + kq;
          hf[i][s] = zero8<T>();
          if (tk[i] >= 0 && k < RANK) {
            const T* hp = H + static_cast<int64_t>(tk[i]) * a.ldh + k;
            const u32x2 lo = __builtin_bit_cast(u32x2, coherent_load8(hp));
            const u32x2 hi = __builtin_bit_cast(u32x2, coherent_load8(hp + 4));
            hf[i][s] = __builtin_bit_cast(V8, u32x4{lo[0], lo[1], hi[0], hi[1]});
          }
        }
      }
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s) d = mfma16(bf[i][s], hf[i][s], d);
        // d: columns rq..rq+3 of token tk.  Tokens of other groups and
        // padding rows are not this tile's.
        const int tl = tk[i] - g * kLinTokens;
        if (tk[i] >= 0 && tl >= 0 && tl < kLinTokens) {
          float* dst = et + tl * kLinCols + rq;
#pragma unroll
          for (int q = 0; q < 4; ++q) dst[q] += d[q];
        }
      }
    }
  }
  __syncthreads();
  T* Y = static_cast<T*>(a.y);
#pragma unroll
  for (int i = 0; i < kUnits; ++i) {
    const int u = tid + i * kThreads;
    const int tl = (u * 4) / kLinCols;
    const int c4 = (u * 4) % kLinCols;
    const int t = g * kLinTokens + tl;
    if (t < l.tokens) store4(Y + static_cast<int64_t>(t) * a.ldy + jt * kLinCols + c4, *reinterpret_cast<const f32x4*>(et + u * 4));
  }
  trace_stamp(a, 6);
  // This tile has read every flag and H row it needs.
  const unsigned readers = static_cast<unsigned>(l.groups * n_tiles);
  for (int b = tid; b < n_blocks; b += kThreads) {
    if (atomic_add_u(&l.hcnt[b], 1u) == readers - 1) {
      atomic_store_u(&l.hcnt[b], 0u);
      atomic_store_u(&l.hflag[b], 0u);
    }
  }
}

template <typename T>
hipError_t launch_linear_t(const ApplyArgs& a0, const LinearArgs& l, int32_t n_shrink, hipStream_t stream) {
  const int64_t n = static_cast<int64_t>(n_shrink) + a0.n_slots +
                    static_cast<int64_t>(l.groups) * (l.n_out / kLinCols) * l.splits;
  const dim3 grid(static_cast<unsigned>(n));
  ApplyArgs a = a0;
  if (a.trace != nullptr && n * kTraceWords > a.trace_words) a.trace = nullptr;
  switch (a.rank) {
    case 8: linear_kernel<T, 8><<<grid, kThreads, 0, stream>>>(a.plan.header, a.plan.blocks, a.plan.bperm, n_shrink, a, l); break;
    case 16: linear_kernel<T, 16><<<grid, kThreads, 0, stream>>>(a.plan.header, a.plan.blocks, a.plan.bperm, n_shrink, a, l); break;
    case 32: linear_kernel<T, 32><<<grid, kThreads, 0, stream>>>(a.plan.header, a.plan.blocks, a.plan.bperm, n_shrink, a, l); break;
    case 64: linear_kernel<T, 64><<<grid, kThreads, 0, stream>>>(a.plan.header, a.plan.blocks, a.plan.bperm, n_shrink, a, l); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Read probe: each workgroup streams a contiguous share of `n16` 16-byte
// words with non-temporal loads, eight per thread in flight, and folds them
// into one word that is stored only if it equals a value no input here
// produces (so the loads cannot be dropped).
constexpr int kProbeThreads = 512;
constexpr int kProbeDepth = 8;
__global__ __launch_bounds__(kProbeThreads) void read_probe_kernel(const u32x4* __restrict__ p, size_t n16,
                                                                   u32x4* __restrict__ sink) {
  const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const size_t beg = static_cast<size_t>(blockIdx.x) * per;
  const size_t end = beg + per < n16 ? beg + per : n16;
  u32x4 acc = u32x4{0u, 0u, 0u, 0u};
  for (size_t i = beg + threadIdx.x; i < end; i += static_cast<size_t>(kProbeThreads) * kProbeDepth) {
    u32x4 v[kProbeDepth];
#pragma unroll
    for (int u = 0; u < kProbeDepth; ++u) {
      const size_t j = i + static_cast<size_t>(u) * kProbeThreads;
      v[u] = j < end ? __builtin_nontemporal_load(p + j) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kProbeDepth; ++u) acc ^= v[u];
  }
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x9E3779B9u) sink[threadIdx.x] = acc;
}

__global__ __launch_bounds__(kThreads) void fill_u32_kernel(uint32_t* __restrict__ p, uint32_t v, size_t n) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride) p[i] = v;
}

}  // namespace

hipError_t launch_linear(int dtype_bf16, const ApplyArgs& a, const LinearArgs& l, hipStream_t stream) {
  // The shrink side is the kShrinkOnly split; the GEMM side needs whole
  // K-slices and column tiles, and token groups covering the rows.
  if (a.srows != kShrinkRowsFused || a.n_chunks < 1 || a.n_chunks > kMaxChunks || a.w.n_a != 1 ||
      a.w.mode != kStacked || a.tiles != 1 || l.n_out % kLinCols != 0 || a.d_model % kSliceK != 0 ||
      l.k_range % kSliceK != 0 || l.splits < 1 || static_cast<int64_t>(l.splits) * l.k_range < a.d_model ||
      static_cast<int64_t>(l.splits - 1) * l.k_range >= a.d_model || l.tokens < 1 ||
      static_cast<int64_t>(l.groups) * kLinTokens < l.tokens || (l.ldw % 8) != 0 || (a.ldx % 8) != 0)
    return hipErrorInvalidValue;
  const int32_t n_shrink = a.n_slots * a.n_chunks * a.n_rgroups;
  return dtype_bf16 ? launch_linear_t<__bf16>(a, l, n_shrink, stream) : launch_linear_t<_Float16>(a, l, n_shrink, stream);
}

hipError_t launch_fill_u32(uint32_t* p, uint32_t v, size_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const size_t blocks = std::min<size_t>((n + kThreads - 1) / kThreads, 2048);
  fill_u32_kernel<<<static_cast<unsigned>(blocks), kThreads, 0, stream>>>(p, v, n);
  return hipGetLastError();
}

hipError_t launch_read_probe(const void* p, size_t bytes, void* sink, int workgroups, hipStream_t stream) {
  const size_t n16 = bytes / 16;
  read_probe_kernel<<<static_cast<unsigned>(n16 == 0 ? 1 : workgroups), kProbeThreads, 0, stream>>>(
      static_cast<const u32x4*>(p), n16, static_cast<u32x4*>(sink));
  return hipGetLastError();
}

int expand_cols_per_workgroup() { return kOC; }
#ifdef WP_TRACE
int traced_build() { return 1; }
#else
int traced_build() { return 0; }
#endif
int shrink_small_waves_per_simd() { return waves_per_simd<0, kShrinkOnly, 1>(); }

int fused_waves_per_simd(int rank, int multi) {
  const bool wide = rank == 0 || rank == 64;
  if (multi) return wide ? waves_per_simd<64, kFusedMulti, 1>() : waves_per_simd<32, kFusedMulti, 1>();
  return wide ? waves_per_simd<64, kFused, 1>() : waves_per_simd<32, kFused, 1>();
}

hipError_t launch_fused(int dtype_bf16, const ApplyArgs& a, hipStream_t stream) {
  // The kernels' shrink split is fixed per role; the grid and the readers
  // follow a.srows, so the two must agree.
  if (a.srows != (a.n_sub > 1 ? kShrinkRowsFused : kShrinkRows)) return hipErrorInvalidValue;
  // The block's H rows live in LDS, sized for blocks of 16 tokens and at most
  // kMaxSlices A slices; the probe gate takes at most 64 x kProbesPerLane
  // shrink workgroups per block; the partial buffer holds kMaxChunks x
  // kMaxRank fp32 per plan position.
  if (a.tiles != 1) return hipErrorInvalidValue;
  if (a.w.n_a < 1 || a.w.n_a > kMaxSlices || (a.w.n_a > 1 && a.w.n_a != a.w.n_slices) ||
      a.hs != a.w.n_a * a.hs1 || a.n_chunks * a.n_rgroups * a.w.n_a > 64 * kProbesPerLane ||
      a.n_chunks * a.hs > kMaxChunks * kMaxRank ||
      (a.pad_rank && (a.w.n_a < 2 || a.rank != 0 || a.hs1 != kMaxRank)) || (a.rank == 0 && a.w.n_a > 1 && !a.pad_rank))
    return hipErrorInvalidValue;
  return a.n_sub > 1 ? launch_role<kFusedMulti>(dtype_bf16, a, stream) : launch_role<kFused>(dtype_bf16, a, stream);
}
hipError_t launch_shrink(int dtype_bf16, const ApplyArgs& a, hipStream_t stream) {
  if (a.n_chunks < 1 || a.n_chunks > kMaxChunks || a.w.n_a != 1) return hipErrorInvalidValue;
  return dtype_bf16 ? launch_shrink_t<__bf16>(a, stream) : launch_shrink_t<_Float16>(a, stream);
}
hipError_t launch_shrink_small(int dtype_bf16, const ApplyArgs& a, hipStream_t stream) {
  if (a.srows != kShrinkRowsFused || a.n_ochunks != 1 || a.n_sub != 1 || a.n_chunks < 1 || a.n_chunks > kMaxChunks ||
      a.w.n_a != 1)
    return hipErrorInvalidValue;
  return launch_role<kShrinkOnly>(dtype_bf16, a, stream);
}
hipError_t launch_expand(int dtype_bf16, const ApplyArgs& a, hipStream_t stream) {
  if (a.w.n_a < 1 || a.w.n_a > kMaxSlices) return hipErrorInvalidValue;
  return launch_role<kExpandOnly>(dtype_bf16, a, stream);
}

}  // namespace wp
