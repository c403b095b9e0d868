/*
 * warppipe_mi355x.h -- C ABI of the MI355X (gfx950) grouped multi-LoRA apply.
 *
 * This is the drop-in boundary that replaces the reference's pybind11 class
 * `warp_pipe_ext.WarpPipeExtension` (csrc/pybind/warp_pipe_bindings.cpp:18-300).
 * Everything is plain C: opaque handle, raw device pointers, sizes, and a
 * hipStream_t passed as void*.  No torch types cross this boundary; the Python
 * engine (adapterslotsplusplus_amd/engine.py) binds it with ctypes.
 *
 * Conventions (reference: warp_pipe_bindings.cpp, engine.py):
 *   - Every call returns an int status.  WP_OK = 0.  WP_NOT_HANDLED = 1 is the
 *     reference's "return False / -1, caller falls back" convention.  Negative
 *     values are errors; the reference raises RuntimeError for these
 *     (TORCH_CHECK / std::runtime_error), and wp_last_error() returns the
 *     message of the last failing call on the calling thread.
 *   - Compute is enqueued on the caller's stream (the reference uses torch's
 *     current stream, bindings:135,145,167,211).  Nothing on the compute path
 *     synchronises the host.
 *   - Tensors are row-major.  X [T, d], H [T, rank], Y rows of `y_row_stride`
 *     elements.  A_seg is [rank, d] and B_seg is [o, rank] (bindings:114-115).
 *   - dtype: WP_DTYPE_F16 or WP_DTYPE_BF16 for X, A, B, H, Y alike; all
 *     accumulation is fp32.
 */
#ifndef WARPPIPE_MI355X_H
#define WARPPIPE_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WP_ABI_VERSION 2

enum wp_status {
  WP_OK = 0,
  WP_NOT_HANDLED = 1,
  WP_ERR_INVALID = -1,          /* bad argument (shape, dtype, alignment, rank) */
  WP_ERR_HIP = -2,              /* a HIP runtime call failed */
  WP_ERR_UNKNOWN_ADAPTER = -3,  /* adapter id not registered */
  WP_ERR_CAPACITY = -4,         /* a table or pool limit was exceeded */
  WP_ERR_NO_DEVICE = -5,        /* no usable GPU */
  WP_ERR_STATE = -6             /* call not valid in the engine's current state */
};

enum wp_dtype { WP_DTYPE_F16 = 0, WP_DTYPE_BF16 = 1 };

typedef struct wp_engine wp_engine;

typedef struct wp_config {
  int32_t device;             /* HIP device ordinal */
  int32_t num_staging_slots;  /* reference: WP_MAX_STAGING = 8 (warp_pipe_metadata.h:11) */
  int32_t max_tokens;         /* largest T accepted by build_seg_bounds (reference: 256) */
  int32_t max_rank;           /* largest adapter rank (64) */
  int32_t max_adapter_ids;    /* adapter table size: ids in [0, n) are usable with build_seg_bounds tables
                                 (others through build_segments only); 0 = 65536.  The table is sized once,
                                 so captured graphs never see it move. */
} wp_config;

/* ---- library ---------------------------------------------------------- */

/* Message of the last failing call on this thread ("" if none). */
const char* wp_last_error(void);

/* ABI version (WP_ABI_VERSION). */
int wp_abi_version(void);

/* 1 if rank has a compiled kernel specialisation (8, 16, 32, 64), else 0.
 * Replaces WarpPipeExtension::rank_supported (bindings:126) /
 * warp_pipe_rank_supported (csrc/dispatch/warp_pipe_dispatcher.cpp:18). */
int wp_rank_supported(int32_t rank);

/* Most tokens per work block in a plan over T tokens (16 for T <= 512, else
 * 64), as wp_read_plan reports the blocks.  No reference counterpart: the
 * by-adapter blocking is this library's own. */
int wp_block_tokens(int64_t T);

/* ---- engine lifetime ---------------------------------------------------- */

/* Replaces WarpPipeExtension::WarpPipeExtension (bindings:20-34): creates the
 * per-engine segment table, staging slots and prefetch stream.  cfg may be
 * NULL for the defaults.  Fails with WP_ERR_NO_DEVICE when no GPU is usable. */
int wp_create(const wp_config* cfg, wp_engine** out);

/* Replaces ~WarpPipeExtension (bindings:36-39). Synchronises the device. */
int wp_destroy(wp_engine* e);

/* ---- adapter store ------------------------------------------------------ */

/* Replaces WarpPipeExtension::register_adapter (bindings:110-119) and
 * AdapterStore::register_adapter (csrc/memory/adapter_store.h:21-27).
 * A is [rank, d], B is [o, rank], both contiguous.  The weights are copied into
 * engine-owned memory: device-resident (a stream-ordered pool allocation) when
 * `host_resident` is 0 and A/B are device pointers, or into the pinned host
 * store when `host_resident` is 1 and A/B are host pointers (such an adapter
 * is usable once prefetched).  Re-registering an id replaces it. */
int wp_register_adapter(wp_engine* e, int32_t adapter_id, const void* A, const void* B, int32_t rank,
                        int32_t d_model, int32_t out_features, float alpha_scale, int32_t dtype,
                        int32_t host_resident, void* stream);

/* AdapterStore::register_adapter as the reference keeps it (csrc/memory/
 * adapter_store.h:21-27: a registry of the caller's pointers, nothing copied):
 * A [rank, d] and B [o, rank] are device memory of the engine's device that
 * the caller keeps alive, unchanged in layout, until the id is evicted or
 * registered again and the work enqueued before that has finished; kernels
 * read them in place, so updates the caller makes to them are seen by later
 * calls.  Evicting such an id frees nothing.  Re-registering an id replaces it. */
int wp_register_adapter_ref(wp_engine* e, int32_t adapter_id, const void* A, const void* B, int32_t rank,
                            int32_t d_model, int32_t out_features, float alpha_scale, int32_t dtype, void* stream);

/* Replaces WarpPipeExtension::evict_adapter (bindings:121-124).  Silent for an
 * unknown id (adapter_store.h:29).  Also releases a staging slot held by the id. */
int wp_evict_adapter(wp_engine* e, int32_t adapter_id, void* stream);

/* 1 if the id is registered, 0 otherwise. */
int wp_has_adapter(wp_engine* e, int32_t adapter_id);

/* Multi-layer adapter store (no counterpart in the reference, whose store
 * holds one (A, B) per id, csrc/memory/adapter_store.h:12-19): a layer's
 * adapters are registered under ids offset by layer * stride.  After this
 * call, the per-token ids of a build_seg_bounds plan select the adapters
 * registered under offset + id in the shrink / expand calls that
 * follow on adapter-store weights; with count > 0, ids >= count are skipped
 * and flagged like unregistered ones (they would reach the next layer).
 * (0, 0) restores the plain ids.  Calls on a build_segments table require
 * offset 0. */
int wp_set_entry_offset(wp_engine* e, int32_t offset, int32_t count);

/* No reference counterpart (its registry has no capacity, adapter_store.h:12-19):
 * declares that at most n adapters will be registered at once (0: no
 * declaration).  Grids of adapter-store calls (shrink, expand, shrink_expand,
 * shrink_expand_slices on a build_seg_bounds table) hold a block slot per
 * possible block; an eager call counts the adapters registered when it is
 * enqueued, but a call captured into a graph is replayed after later
 * registrations, so without a declaration its grid holds up to T slots
 * (mostly empty at decode sizes).  With one, both use n, and registering an
 * (n+1)-th adapter fails with WP_ERR_CAPACITY.  WP_ERR_STATE if more than n
 * are registered already. */
int wp_set_max_adapters(wp_engine* e, int64_t n);

/* ---- segment tables ----------------------------------------------------- */

/* Replaces WarpPipeExtension::build_segments (bindings:128-130) /
 * build_segment_table (csrc/dispatch/segment_builder.cpp:5-50).  One segment
 * per (ids[k], offsets[k], offsets[k+1]-offsets[k]); n_offsets must be K+1 and
 * K at most max_segments.  The table is uploaded stream-ordered on `stream`. */
int wp_build_segments(wp_engine* e, const int32_t* sorted_adapter_ids, int32_t K, const int32_t* seg_offsets,
                      int32_t n_offsets, void* stream);

/* Replaces WarpPipeExtension::build_seg_bounds (bindings:162-170) and
 * build_seg_bounds_kernel (csrc/kernels/warp_pipe_r32.cu:461-512).  idx is a
 * device array of T token->adapter ids (int64 if idx_is_int64, else int32).
 * Builds, on the device, the run-length segment table (bit-exact with the
 * reference) and the by-adapter token grouping the apply kernels use.
 * Returns WP_NOT_HANDLED (reference: False, no launch) when T > max_tokens. */
int wp_build_seg_bounds(wp_engine* e, const void* idx, int32_t idx_is_int64, int64_t T, void* stream);

/* Test/debug readback (synchronous on `stream`): copies the current segment
 * table as int32 triples (adapter_id, token_start, token_count) into host
 * memory `out` (capacity cap triples) and the count into *num_segments. */
int wp_read_segments(wp_engine* e, int32_t* out, int64_t cap, int64_t* num_segments, void* stream);

/* Test/debug readback of the grouped plan (synchronous): perm[n_valid],
 * blocks as int32 quads (adapter_id, first, count, entry) and the counts. */
int wp_read_plan(wp_engine* e, int32_t* perm, int64_t perm_cap, int32_t* blocks, int64_t block_cap,
                 int64_t* n_valid, int64_t* n_blocks, void* stream);

/* Reads and clears the device error word (bit flags, see wp_types.h).
 * Synchronises `stream`.  Includes bits an earlier wp_poll_device_errors had
 * moved out of the word and not yet reported. */
int wp_read_device_errors(wp_engine* e, uint32_t* flags, void* stream);

/* No reference counterpart: the device error word without a host wait on
 * the compute path, for serving loops (the punica hook's update_metadata,
 * DraftLoRAContext.begin_step).  *flags gets the bits the previous poll moved
 * out of the word if that move has completed (0 otherwise: they come with a
 * later poll or with wp_read_device_errors); then, unless one is still in
 * flight, one kernel on `stream` moves the word (as of that point of the
 * stream) into a pinned host word and clears it.  Does nothing while
 * `stream` is capturing. */
int wp_poll_device_errors(wp_engine* e, uint32_t* flags, void* stream);

/* ---- apply ---------------------------------------------------------------- */

/* Replaces WarpPipeExtension::shrink (bindings:132-139) and
 * dispatch_bgmv_shrink (warp_pipe_dispatcher.cpp:33-42):
 *   H[t, :rank_a] = rn(alpha_a * X[t, :] . A_a^T) for every segment token.
 * H must be zero-initialised by the caller ([T, h_row_stride]).  rank = 0
 * selects mixed-rank mode (each adapter's own rank, h_row_stride >= 64). */
int wp_shrink(wp_engine* e, const void* X, void* H, int32_t d_model, int32_t rank, int64_t T,
              int64_t h_row_stride, int32_t dtype, void* stream);

/* Replaces WarpPipeExtension::expand (bindings:141-148):
 *   Y[t, off + o] = rn(Y[t, off + o] + H[t, :] . B_a[o, :]) for every segment token. */
int wp_expand(wp_engine* e, const void* H, void* Y, int32_t out_features, int32_t rank, int64_t T,
              int64_t h_row_stride, int64_t y_row_stride, int32_t y_col_offset, int32_t dtype, void* stream);

/* shrink() followed by expand() over the adapter store, as one call: no
 * counterpart in the reference (its callers run the two after each other,
 * bindings:132-148).  Decode-sized plans (at most 512 tokens) run both halves
 * in one launch with no H round trip (rank = 0: mixed ranks, each adapter's
 * own); larger plans run shrink then expand through the engine's own H.  Results
 * match the two calls within the fp tolerance (the d-range split, and so the
 * fp32 summation order of H, can differ). */
int wp_shrink_expand(wp_engine* e, const void* X, void* Y, int32_t d_model, int32_t out_features, int32_t rank,
                     int64_t T, int64_t y_row_stride, int32_t y_col_offset, int32_t dtype, void* stream);

/* A base linear and its per-token LoRA delta in one launch: replaces the
 * sequence the reference's draft-model wrapper runs per projection
 * (BGMVLoRALinear.forward, benchmarks/e2e/serve_multitenant.py:56-87: the
 * base F.linear, then bgmv_shrink and bgmv_expand into its output):
 *   y[T, d_out] = rn( rn(x . W^T + bias) + rn(scale . x . A_i^T) . B_i^T )
 * per token, i its adapter in the last build_seg_bounds table (tokens with
 * id -1: the base output alone).  W is [d_out, w_row_stride] (torch's Linear
 * layout), bias [d_out] or NULL; wa / wb are add_lora's stacked weights
 * (wa_t_all [num_loras, 1, rank, d_in], wb_t_all [num_loras, 1, d_out,
 * rank]); x [T, d_in] and y [T, d_out] contiguous.  WP_NOT_HANDLED (the
 * caller runs the linear and add_lora instead) for a rank without kernels,
 * T over 512, d_in not a multiple of 128 or d_out not a multiple of 16. */
int wp_linear_lora(wp_engine* e, void* y, const void* x, const void* w, int64_t w_row_stride, const void* bias,
                   const void* wa, int64_t wa_stride0, const void* wb, int64_t wb_stride0, int32_t num_loras,
                   float scale, int32_t rank, int32_t d_in, int32_t d_out, int64_t T, int32_t dtype, void* stream);

/* shrink_expand over several layers of a multi-layer store in one launch (no
 * reference counterpart): slice s applies, to every token of the last
 * build_seg_bounds table, the adapter registered under id_offsets[s] + the
 * token's id (ids >= ids_per_layer skipped and flagged; 0: no limit), into
 * columns [y_col_offsets[s], + out_features[s]) of Y.  X is read once; each
 * slice's adapter has its own A, B, alpha and (rank = 0) rank.  The packed
 * gate/up projections of a layer, for instance, as one call.  Plans over 512
 * tokens run one shrink_expand per slice. */
int wp_shrink_expand_slices(wp_engine* e, const void* X, void* Y, int32_t d_model, int32_t n_slices,
                            const int32_t* id_offsets, int32_t ids_per_layer, const int32_t* out_features,
                            const int32_t* y_col_offsets, int32_t rank, int64_t T, int64_t y_row_stride, int32_t dtype,
                            void* stream);

/* Replaces WarpPipeExtension::add_lora_packed (bindings:195-234) and the DSAK
 * kernels (warp_pipe_r32.cu:280-423), generalised to ranks 8/16/32/64, bf16,
 * and n_slices (1..4) output slices sharing one H:
 *   h = rn(scale * x[t] . wa[id]^T);  y[t, y_off[s] + o] = rn(y[...] + h . wb_s[id][o, :])
 * for every token t of the last build_seg_bounds table (ids < 0 untouched).
 * wa: [L, rank, d] with element stride wa_stride0 between adapters;
 * wb[s]: [L, o[s], rank] with element stride wb_stride0[s]. */
int wp_add_lora(wp_engine* e, void* y, const void* x, const void* wa, int64_t wa_stride0, int32_t num_loras,
                int32_t n_slices, const void* const* wb, const int64_t* wb_stride0, const int32_t* out_features,
                const int32_t* y_col_offsets, float scale, int32_t rank, int32_t d_model, int64_t T,
                int64_t y_row_stride, int32_t dtype, void* stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops or harnesses that forbid
 * hipMalloc): wp_build_seg_bounds followed by wp_add_lora as one call, with no
 * engine.  The step plan, the fp32 partials and the per-block counters live in
 * a static device array of this library, WP_STATIC_SCRATCH_BYTES per GPU, held
 * until the process ends; the call allocates and frees nothing.  Arguments and
 * results are wp_add_lora's on a table built from idx (T token -> adapter ids,
 * int64 if idx_is_int64, else int32).  Limits: T <= 256 (WP_ERR_CAPACITY
 * above), rank 8/16/32/64 (WP_NOT_HANDLED otherwise), 1..4 slices.  The first
 * call on a device sets its scratch up synchronously and must not be under
 * graph capture; later calls enqueue two kernels on `stream` and may be
 * captured.  Every call on a GPU shares that GPU's scratch: calls that overlap
 * (other streams, other threads) race and must be serialised by the caller. */
#define WP_STATIC_SCRATCH_BYTES 1189120
int wp_add_lora_static(void* y, const void* x, const void* idx, int32_t idx_is_int64, int64_t T, const void* wa,
                       int64_t wa_stride0, int32_t num_loras, int32_t n_slices, const void* const* wb,
                       const int64_t* wb_stride0, const int32_t* out_features, const int32_t* y_col_offsets,
                       float scale, int32_t rank, int32_t d_model, int64_t y_row_stride, int32_t dtype, void* stream);

/* No counterpart in the reference; for the callers of wp_add_lora_static
 * (those that cannot allocate).  The kernels of wp_add_lora_static skip
 * tokens they cannot serve and record why in the device error word of the
 * GPU's static scratch (bit flags as wp_read_device_errors reports them: 1
 * an id >= num_loras, 8 a wait on partials gave up, 16 more blocks than the
 * grid holds).  This enqueues, on `stream`, one kernel that copies that word
 * of device `device` into *out (4 bytes of device-accessible memory the
 * caller provides) and clears it; it allocates nothing and may be captured
 * once the device's scratch is set up (its first call on a device, or the
 * first wp_add_lora_static there, sets it up synchronously, outside capture).
 * The word is shared like the scratch: calls that overlap on one GPU race. */
int wp_read_static_errors(int32_t device, uint32_t* out, void* stream);

/* wp_add_lora with one A per output slice: vLLM's add_lora_packed_nslice
 * (packed q/k/v or gate/up layers, each slice with its own lora_a and lora_b;
 * the reference hook leaves this method to the stock path,
 * lora_warp_pipe/punica_wrapper.py:8-16).  In one launch, for every token t
 * of the last build_seg_bounds table and every slice s:
 *   h_s = rn(scale * x[t] . wa[s][id]^T);  y[t, y_off[s] + o] = rn(y[...] + h_s . wb[s][id][o, :])
 * x is read once per call; wa[s]: [L, rank, d] with element stride
 * wa_stride0[s]; wb[s]: [L, o[s], rank].  1..4 slices, one rank for all. */
int wp_add_lora_nslice(wp_engine* e, void* y, const void* x, int32_t n_slices, const void* const* wa,
                       const int64_t* wa_stride0, const void* const* wb, const int64_t* wb_stride0,
                       const int32_t* out_features, const int32_t* y_col_offsets, int32_t num_loras, float scale,
                       int32_t rank, int32_t d_model, int64_t T, int64_t y_row_stride, int32_t dtype, void* stream);

/* ---- vLLM V1 LoRA ops ------------------------------------------------------ */
/* No reference counterpart: the reference hooks only vLLM 0.6's add_lora and
 * scopes the V1 op surface out (lora_warp_pipe/punica_wrapper.py:8-16).  These
 * are the grouped ops behind V1's PunicaWrapperGPU (add_shrink, add_expand,
 * add_lora_embedding, add_lora_linear) on the last build_seg_bounds table and
 * vLLM's stacked weights: lora_a_stacked[s] [L, 1, rank, d], lora_b_stacked[s]
 * [L, 1, o_s, rank], lora_bias_stacked[s] [L, 1, o_s] (element strides between
 * adapters given).  add_lora_linear itself is wp_add_bias (if biases) then
 * wp_add_lora_nslice: no H round trip. */

/* add_shrink: out[s][t][k] += scale * x[t] . wa[s][id_t][k, :] for k < rank,
 * fp32, unrounded (V1's lora_shrink buffer), for every token t of the table
 * and slice s; slice s of out starts out_slice_stride floats after slice 0,
 * rows out_row_stride floats apart (both multiples of 4; out 16-byte
 * aligned).  WP_NOT_HANDLED for a rank without kernels. */
int wp_lora_shrink(wp_engine* e, float* out, int64_t out_slice_stride, int64_t out_row_stride, const void* x,
                   int32_t n_slices, const void* const* wa, const int64_t* wa_stride0, int32_t num_loras, float scale,
                   int32_t rank, int32_t d_model, int64_t T, int32_t dtype, void* stream);

/* add_expand / add_lora_embedding: for every token t of the table and slice s,
 *   y[t, off_s + o] = rn((add_inputs ? y'[t, off_s + o] : 0) + rn(h[s][t][:]) . wb[s][id_t][o, :])
 * with y' = rn(y + bias[s][id_t]) where bias[s] is given (add_inputs only,
 * as V1 applies the bias before an expand that adds).  h is fp32 (h_is_f32;
 * rounded to the I/O type first, as V1's lora_expand casts it) or the I/O
 * type; slice s at h + s * h_slice_stride, rows h_row_stride apart.  Two
 * launches.  WP_NOT_HANDLED for a rank without kernels. */
int wp_lora_expand(wp_engine* e, void* y, int64_t y_row_stride, const void* h, int32_t h_is_f32, int64_t h_slice_stride,
                   int64_t h_row_stride, int32_t n_slices, const void* const* wb, const int64_t* wb_stride0,
                   const int32_t* out_features, const int32_t* y_col_offsets, const void* const* bias,
                   const int64_t* bias_stride0, int32_t num_loras, int32_t rank, int64_t T, int32_t add_inputs,
                   int32_t dtype, void* stream);

/* V1's _apply_bias: y[t, off_s + o] = rn(y[t, off_s + o] + bias[s][id_t][o]) for
 * every token of the table and every slice whose bias is not NULL (ids >=
 * num_loras are skipped and flagged, device error 1). */
int wp_add_bias(wp_engine* e, void* y, int64_t y_row_stride, int32_t n_slices, const void* const* bias,
                const int64_t* bias_stride0, const int32_t* out_features, const int32_t* y_col_offsets,
                int32_t num_loras, int64_t T, int32_t dtype, void* stream);

/* ---- staging / prefetch ---------------------------------------------------- */

/* Replaces WarpPipeExtension::prefetch_adapter (bindings:46-57): copies the
 * adapter's A and B into a staging slot on the engine's prefetch stream (H2D
 * from the pinned host store, which the copy kernel reads directly, or D2D).
 * Writes the slot index, or -1 when the id is unknown or every slot is taken
 * (*slot_out); an id that already holds a slot keeps it (nothing is copied).  Once the copy has landed
 * the slot is published on the device; the next build_seg_bounds (captured or
 * not) puts it into the adapter table, and an eager call on a table built
 * before that picks it up when it finds the copy complete. */
int wp_prefetch_adapter(wp_engine* e, int32_t adapter_id, int32_t* slot_out);

/* prefetch_adapter for n ids in one call (no reference counterpart): one copy
 * kernel for the batch.  slots_out[k] as wp_prefetch_adapter's *slot_out. */
int wp_prefetch_adapters(wp_engine* e, const int32_t* adapter_ids, int32_t n, int32_t* slots_out);

/* Replaces is_prefetch_ready (bindings:59-62): *ready = 1 once the copy completed. */
int wp_is_prefetch_ready(wp_engine* e, int32_t adapter_id, int32_t* ready);

/* Replaces release_prefetch (bindings:64): frees the id's slot (no-op without one).
 * In stream order on `stream`: kernels enqueued on it before the release
 * (graph replays included) still read the slot; kernels enqueued after it use
 * the adapter's registered weights (or skip a host-resident adapter), and the
 * slot's next copy waits for this point.  The reference frees the slot at
 * once (staging_buffer.h:75-79). */
int wp_release_prefetch(wp_engine* e, int32_t adapter_id, void* stream);

/* wp_release_prefetch for n ids in one call (no reference counterpart). */
int wp_release_prefetches(wp_engine* e, const int32_t* adapter_ids, int32_t n, void* stream);

/* No reference counterpart: makes `stream` wait (on the device, no host
 * wait) until the id's prefetch copy has landed, so that a plan built next on
 * it uses the staged copy.  WP_NOT_HANDLED when the id holds no slot. */
int wp_wait_prefetch(wp_engine* e, int32_t adapter_id, void* stream);

/* wp_wait_prefetch for n ids in one call; WP_NOT_HANDLED when any holds no slot
 * (the others are still waited for). */
int wp_wait_prefetches(wp_engine* e, const int32_t* adapter_ids, int32_t n, void* stream);

/* Test and debug: polls a wait on partials makes before it gives up (device
 * error 8, kErrSpin); 0xFFFFFFFF restores the default (131072, about 0.1 s).
 * After a give-up, calls that use the partial buffer skip their work until
 * the next build_seg_bounds / build_segments (or wp_read_device_errors) has
 * repaired the buffer. */
int wp_set_spin_limit(wp_engine* e, uint32_t polls);

/* Measurement, no reference counterpart: reads `bytes` (a multiple of 16) of
 * device memory at `buffer` once, with 16-byte non-temporal loads over two
 * workgroups per compute unit, on `stream`; `sink` is 8 KiB of device memory
 * the kernel may write.  bytes == 0 launches an empty kernel.  bench.py times
 * it to state the floor of a call: the time one launch takes to read that
 * call's bytes, and the launch cost alone. */
int wp_read_probe(wp_engine* e, const void* buffer, int64_t bytes, void* sink, void* stream);

/* Measurement, no reference counterpart: what one cross-workgroup dependency
 * costs a launch that streams a call's bytes.  `workgroups` workgroups of 512
 * threads each stream their share of `a` (a call's A and X bytes), count
 * themselves on their group's counter (`group` consecutive workgroups wait
 * for each other), stream their share of `b` (B, and Y read) -- the first
 * batch of it before waiting for the group (mode 1), all of it after (mode
 * 2), or with no wait (mode 0) -- and write their share of `y`.  Mode 3
 * splits the roles over compute units instead (one workgroup per compute
 * unit): workgroups [0, group) stream `a` and count themselves, the others
 * stream all of `b`, wait for every count and write `y`.  counters:
 * 2 x 64 words per group, zero before the first launch (each launch leaves
 * them zero); *err gets bit 0 if a wait gave up (about 0.1 s; the counters
 * must then be zeroed again).  All pointers are device memory. */
int wp_handoff_probe(const void* a, int64_t a_bytes, const void* b, int64_t b_bytes, void* y, int64_t y_bytes,
                     uint32_t* counters, uint32_t* err, int32_t group, int32_t mode, int32_t workgroups, void* stream);

/* Test of lds_barrier(), the LDS-only workgroup barrier of every kernel here
 * (the property the reference checks for its barrier wrappers,
 * tests/unit/test_barrier_sync.cu:21-41): `workgroups` workgroups of `threads`
 * (256 = 4 wave64 waves, or 1024) run `rounds` rounds in which every thread
 * writes a value built from salts[round] (a device array) into its LDS slot,
 * passes the barrier, and checks every slot of the workgroup; mismatches are
 * added to *mismatches (device memory, zeroed by the caller). */
int wp_barrier_probe(const uint32_t* salts, int32_t rounds, int32_t threads, int32_t workgroups, uint32_t* mismatches,
                     void* stream);

/* Diagnostics: in a library built with WP_TRACE (adapterslotsplusplus_amd.build
 * --trace), fused launches whose grid fits record 8 timestamps per workgroup
 * into the device buffer (n_words 64-bit words; NULL stops tracing).  In a
 * normal build: WP_ERR_STATE. */
int wp_set_trace(wp_engine* e, void* buffer, int64_t n_words);

#ifdef __cplusplus
}
#endif

#endif /* WARPPIPE_MI355X_H */
