// wp_aux.hip -- small kernels around the apply path (gfx950):
//
//   * take_word_kernel: moves a device error word into caller memory and
//     clears it (one atomic exchange), so that errors can be read without a
//     host wait on the compute path;
//   * prep_kernel: the per-token work of vLLM V1's LoRA op surface that is
//     not a grouped GEMM -- the per-adapter bias add (PunicaWrapperGPU's
//     _apply_bias), the fp32 lora_shrink buffer rounded and packed into the
//     H rows the expand kernel reads, and zeroed output windows for an
//     expand that overwrites (add_inputs=False);
//   * barrier_probe_kernel: checks that lds_barrier() makes every wave's LDS
//     writes visible to every other wave of the workgroup (the property the
//     reference tests for its barrier wrappers, tests/unit/test_barrier_sync.cu:21-41);
//   * handoff_probe_kernel / handoff_split_kernel: measurements of what one
//     cross-workgroup dependency costs a launch that streams a call's bytes.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "wp_apply.h"
#include "wp_device.h"

namespace wp {
namespace {

constexpr int kAuxThreads = 256;

__global__ __launch_bounds__(64) void take_word_kernel(uint32_t* word, uint32_t* out) {
  if (threadIdx.x == 0) *out = __hip_atomic_exchange(word, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One workgroup per block slot of the plan: block b's tokens (one adapter).
template <typename T>
__global__ __launch_bounds__(kAuxThreads) void prep_kernel(PrepArgs p) {
  const int b = static_cast<int>(blockIdx.x);
  const int n_blocks = static_cast<int>(p.plan.header[kHdrNumBlocks]);
  if (b == p.n_slots - 1 && threadIdx.x == 0 && n_blocks > p.n_slots) flag_error(p.plan.header, kErrCapacity);
  if (b >= n_blocks) return;
  const Block blk = p.plan.blocks[b];
  if (blk.count <= 0) return;
  const int32_t* toks = p.plan.bperm + static_cast<int64_t>(b) * kBlockTokens;
  const int tid = static_cast<int>(threadIdx.x);
  // H rows: dst[t][s * rank + k] = rn(src[s][t][k]).
  if (p.h_src != nullptr) {
    const int per_tok = p.n_slices * p.rank;
    for (int u = tid; u < blk.count * per_tok; u += kAuxThreads) {
      const int j = u / per_tok;
      const int rem = u - j * per_tok;
      const int s = rem / p.rank;
      const int k = rem - s * p.rank;
      const int64_t t = toks[j];
      const int64_t at = s * p.h_slice_stride + t * p.h_row_stride + k;
      const float v = p.h_f32 ? static_cast<const float*>(p.h_src)[at] : static_cast<float>(static_cast<const T*>(p.h_src)[at]);
      static_cast<T*>(p.h_dst)[t * p.ldh_dst + rem] = static_cast<T>(v);
    }
  }
  // Output windows, 4 elements (8 bytes) per step: zeroed, or the adapter's
  // bias row added (y = rn(y + bias)).
  const bool id_ok = blk.adapter_id >= 0 && blk.adapter_id < p.num_ids;
  bool flagged = false;
  for (int s = 0; s < p.n_slices; ++s) {
    const bool bias = p.bias[s] != nullptr;
    if (!p.zero_y && !bias) continue;
    if (!p.zero_y && !id_ok) {
      flagged = true;
      continue;
    }
    const int q4 = p.o_size[s] / 4;
    const T* brow = bias ? static_cast<const T*>(p.bias[s]) + static_cast<int64_t>(blk.adapter_id) * p.bias_stride[s]
                         : nullptr;
    for (int u = tid; u < blk.count * q4; u += kAuxThreads) {
      const int j = u / q4;
      const int c = (u - j * q4) * 4;
      u32x2* yp = reinterpret_cast<u32x2*>(static_cast<T*>(p.y) + static_cast<int64_t>(toks[j]) * p.ldy + p.y_off[s] + c);
      if (p.zero_y) {
        *yp = u32x2{0u, 0u};
      } else {
        const f32x4 yv = unpack4f<T>(*yp);
        const f32x4 bv = unpack4f<T>(*reinterpret_cast<const u32x2*>(brow + c));
        *yp = __builtin_bit_cast(u32x2, round4<T>(yv + bv));
      }
    }
  }
  if (flagged && tid == 0) flag_error(p.plan.header, kErrIdRange);
}

// Each round, every thread writes a value that depends on a global load
// into its LDS slot, the workgroup passes lds_barrier(), and every thread
// reads all slots (its own wave's and the others') and counts those that do
// not hold this round's values; a second lds_barrier() keeps the next round's
// writes behind every read.  Waves are skewed by a few sleeps per round so
// that they reach the barrier at different times.
__device__ __forceinline__ uint32_t probe_value(uint32_t wg, uint32_t slot, uint32_t salt) {
  return (wg * 0x9E3779B1u) ^ (slot * 0x85EBCA77u) ^ salt;
}

template <int NT>
__global__ __launch_bounds__(NT) void barrier_probe_kernel(const uint32_t* __restrict__ salts, int rounds,
                                                           uint32_t* __restrict__ mismatches) {
  __shared__ uint32_t slot[NT];
  const uint32_t tid = threadIdx.x;
  const uint32_t wave = tid >> 6;
  const uint32_t wg = blockIdx.x;
  uint32_t bad = 0;
  for (int r = 0; r < rounds; ++r) {
    const uint32_t salt = salts[r];
    for (uint32_t i = 0; i < ((static_cast<uint32_t>(r) + wave) & 3u); ++i) __builtin_amdgcn_s_sleep(4);
    slot[tid] = probe_value(wg, tid, salt);
    lds_barrier();
    for (uint32_t k = 0; k < static_cast<uint32_t>(NT); ++k) {
      const uint32_t q = (tid + k) % static_cast<uint32_t>(NT);
      bad += slot[q] != probe_value(wg, q, salt) ? 1u : 0u;
    }
    lds_barrier();
  }
  if (bad != 0) atomicAdd(mismatches, bad);
}

// Handoff probe: each workgroup (512 threads, one per compute unit) streams
// its share of `a` (the call's A and X bytes), stores nothing until it has
// counted itself on its group's counter, and streams its share of `b` (B and
// Y read) -- the first batch before waiting for the rest of its group
// (mode 1) or after it (mode 2), or with no wait at all (mode 0) -- then
// writes its share of `y`.  The last workgroup of a group to pass the wait
// resets the group's counters for the next launch.
constexpr int kHandoffThreads = 512;
constexpr int kHandoffDepth = 8;

__device__ __forceinline__ u32x4 stream_share(const u32x4* __restrict__ p, size_t n16, u32x4 acc) {
  const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const size_t beg = static_cast<size_t>(blockIdx.x) * per;
  const size_t end = beg + per < n16 ? beg + per : n16;
  for (size_t i = beg + threadIdx.x; i < end; i += static_cast<size_t>(kHandoffThreads) * kHandoffDepth) {
    u32x4 v[kHandoffDepth];
#pragma unroll
    for (int u = 0; u < kHandoffDepth; ++u) {
      const size_t j = i + static_cast<size_t>(u) * kHandoffThreads;
      v[u] = j < end ? __builtin_nontemporal_load(p + j) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kHandoffDepth; ++u) acc ^= v[u];
  }
  return acc;
}

__global__ __launch_bounds__(kHandoffThreads) void handoff_probe_kernel(HandoffProbe p) {
  __shared__ int s_ok;
  const u32x4* a = static_cast<const u32x4*>(p.a);
  const u32x4* bsrc = static_cast<const u32x4*>(p.b);
  u32x4 acc = stream_share(a, p.a16, u32x4{0u, 0u, 0u, 0u});
  const int grp = static_cast<int>(blockIdx.x) / p.group;
  const int gsize = std::min<int>(p.group, static_cast<int>(gridDim.x) - grp * p.group);
  uint32_t* cnt = p.counters + static_cast<size_t>(grp) * 2 * kCounterStride;
  uint32_t* done = cnt + kCounterStride;
  // This workgroup's "partials": every load above has landed (the folds used
  // them) before the count goes out.
  __syncthreads();
  if (p.mode != 0 && threadIdx.x == 0) atomic_add_u(cnt, 1u);
  // The first batch of the b share (mode 1: before the wait).
  const size_t per = (p.b16 + gridDim.x - 1) / gridDim.x;
  const size_t beg = static_cast<size_t>(blockIdx.x) * per;
  const size_t end = beg + per < p.b16 ? beg + per : p.b16;
  u32x4 first[kHandoffDepth];
  if (p.mode == 1) {
#pragma unroll
    for (int u = 0; u < kHandoffDepth; ++u) {
      const size_t j = beg + threadIdx.x + static_cast<size_t>(u) * kHandoffThreads;
      first[u] = j < end ? __builtin_nontemporal_load(bsrc + j) : u32x4{0u, 0u, 0u, 0u};
    }
  }
  if (p.mode != 0) {
    if (threadIdx.x == 0) {
      int ok = 1;
      for (uint32_t spins = 0; atomic_load_u(cnt) < static_cast<uint32_t>(gsize); ++spins) {
        if (spins >= p.spin_limit) {
          ok = 0;
          atomicOr(p.err, 1u);
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      s_ok = ok;
    }
    __syncthreads();
    // Everyone in the group has passed the wait once `done` reaches the
    // group size: the last one resets both counters.
    if (threadIdx.x == 0 && s_ok != 0 && atomic_add_u(done, 1u) == static_cast<uint32_t>(gsize - 1)) {
      atomic_store_u(cnt, 0u);
      atomic_store_u(done, 0u);
    }
  }
  size_t rest = beg;
  if (p.mode == 1) {
#pragma unroll
    for (int u = 0; u < kHandoffDepth; ++u) acc ^= first[u];
    rest = beg + static_cast<size_t>(kHandoffThreads) * kHandoffDepth;
  }
  for (size_t i = rest + threadIdx.x; i < end; i += static_cast<size_t>(kHandoffThreads) * kHandoffDepth) {
    u32x4 v[kHandoffDepth];
#pragma unroll
    for (int u = 0; u < kHandoffDepth; ++u) {
      const size_t j = i + static_cast<size_t>(u) * kHandoffThreads;
      v[u] = j < end ? __builtin_nontemporal_load(bsrc + j) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kHandoffDepth; ++u) acc ^= v[u];
  }
  // The y share: written once, whatever the loads held.
  u32x4* y = static_cast<u32x4*>(p.y);
  const size_t yper = (p.y16 + gridDim.x - 1) / gridDim.x;
  const size_t ybeg = static_cast<size_t>(blockIdx.x) * yper;
  const size_t yend = ybeg + yper < p.y16 ? ybeg + yper : p.y16;
  for (size_t i = ybeg + threadIdx.x; i < yend; i += kHandoffThreads) __builtin_nontemporal_store(acc, y + i);
}

// Split-role handoff probe (mode 3): workgroups [0, group) stream the `a`
// share alone and count themselves on one counter; workgroups [group, grid)
// stream the whole `b` share first, then wait for every `a` workgroup's count
// and write the `y` share.  96 KB of LDS per workgroup keeps one workgroup on
// each compute unit, so a role is a compute unit's role: the `a` side's count
// never queues behind `b` loads in its compute unit's memory pipeline.  The
// last `b` workgroup past the wait resets the counters.
__device__ __forceinline__ u32x4 stream_part(const u32x4* __restrict__ p, size_t n16, int part, int parts, u32x4 acc) {
  const size_t per = (n16 + parts - 1) / parts;
  const size_t beg = static_cast<size_t>(part) * per;
  const size_t end = beg + per < n16 ? beg + per : n16;
  for (size_t i = beg + threadIdx.x; i < end; i += static_cast<size_t>(kHandoffThreads) * kHandoffDepth) {
    u32x4 v[kHandoffDepth];
#pragma unroll
    for (int u = 0; u < kHandoffDepth; ++u) {
      const size_t j = i + static_cast<size_t>(u) * kHandoffThreads;
      v[u] = j < end ? __builtin_nontemporal_load(p + j) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kHandoffDepth; ++u) acc ^= v[u];
  }
  return acc;
}

__global__ __launch_bounds__(kHandoffThreads) void handoff_split_kernel(HandoffProbe p) {
  __shared__ uint32_t s_pad[24 * 1024];
  __shared__ int s_ok;
  const int n_a = p.group;
  const int n_b = static_cast<int>(gridDim.x) - n_a;
  const int wg = static_cast<int>(blockIdx.x);
  uint32_t* cnt = p.counters;
  uint32_t* done = p.counters + kCounterStride;
  u32x4 acc{0u, 0u, 0u, 0u};
  if (wg < n_a) {
    acc = stream_part(static_cast<const u32x4*>(p.a), p.a16, wg, n_a, acc);
    s_pad[threadIdx.x] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    __syncthreads();
    if (threadIdx.x == 0) atomic_add_u(cnt, 1u);
    return;
  }
  acc = stream_part(static_cast<const u32x4*>(p.b), p.b16, wg - n_a, n_b, acc);
  if (threadIdx.x == 0) {
    int ok = 1;
    for (uint32_t spins = 0; atomic_load_u(cnt) < static_cast<uint32_t>(n_a); ++spins) {
      if (spins >= p.spin_limit) {
        ok = 0;
        atomicOr(p.err, 1u);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    s_ok = ok;
  }
  __syncthreads();
  if (threadIdx.x == 0 && s_ok != 0 && atomic_add_u(done, 1u) == static_cast<uint32_t>(n_b - 1)) {
    atomic_store_u(cnt, 0u);
    atomic_store_u(done, 0u);
  }
  u32x4* y = static_cast<u32x4*>(p.y);
  const size_t yper = (p.y16 + n_b - 1) / n_b;
  const size_t ybeg = static_cast<size_t>(wg - n_a) * yper;
  const size_t yend = ybeg + yper < p.y16 ? ybeg + yper : p.y16;
  acc[0] ^= s_pad[threadIdx.x];
  for (size_t i = ybeg + threadIdx.x; i < yend; i += kHandoffThreads) __builtin_nontemporal_store(acc, y + i);
}

}  // namespace

hipError_t launch_take_word(uint32_t* word, uint32_t* out, hipStream_t stream) {
  if (word == nullptr || out == nullptr) return hipErrorInvalidValue;
  take_word_kernel<<<1, 64, 0, stream>>>(word, out);
  return hipGetLastError();
}

hipError_t launch_prep(int dtype_bf16, const PrepArgs& p, hipStream_t stream) {
  if (p.n_slots <= 0) return hipSuccess;
  if (p.n_slices < 1 || p.n_slices > kMaxSlices || (p.h_src != nullptr && (p.rank < 1 || p.h_dst == nullptr)))
    return hipErrorInvalidValue;
  for (int s = 0; s < p.n_slices; ++s)
    if (p.o_size[s] % 4 != 0 || p.y_off[s] % 4 != 0) return hipErrorInvalidValue;
  if (dtype_bf16)
    prep_kernel<__bf16><<<p.n_slots, kAuxThreads, 0, stream>>>(p);
  else
    prep_kernel<_Float16><<<p.n_slots, kAuxThreads, 0, stream>>>(p);
  return hipGetLastError();
}

hipError_t launch_barrier_probe(const uint32_t* salts, int rounds, int threads, int workgroups, uint32_t* mismatches,
                                hipStream_t stream) {
  if (salts == nullptr || mismatches == nullptr || rounds < 1 || workgroups < 1) return hipErrorInvalidValue;
  if (threads == 256)
    barrier_probe_kernel<256><<<workgroups, 256, 0, stream>>>(salts, rounds, mismatches);
  else if (threads == 1024)
    barrier_probe_kernel<1024><<<workgroups, 1024, 0, stream>>>(salts, rounds, mismatches);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_handoff_probe(const HandoffProbe& p, int workgroups, hipStream_t stream) {
  if (workgroups < 1 || p.group < 1 || p.mode < 0 || p.mode > 3 || p.counters == nullptr || p.err == nullptr ||
      (p.a16 > 0 && p.a == nullptr) || (p.b16 > 0 && p.b == nullptr) || (p.y16 > 0 && p.y == nullptr) ||
      (p.mode == 3 && p.group >= workgroups))
    return hipErrorInvalidValue;
  if (p.mode == 3)
    handoff_split_kernel<<<workgroups, kHandoffThreads, 0, stream>>>(p);
  else
    handoff_probe_kernel<<<workgroups, kHandoffThreads, 0, stream>>>(p);
  return hipGetLastError();
}

}  // namespace wp
