/*
 * seg_oracle.c -- CPU restatement of the reference's segment-table rules.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP segment
 * builder is compared against.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product library never links,
 * loads or calls it, and has no CPU fallback that could route through it.
 *
 * Functions and the reference code each one restates:
 *
 *   wpo_seg_bounds      build_seg_bounds_kernel, csrc/kernels/warp_pipe_r32.cu:461-512
 *                       (run detection :482-489, ids < 0 skipped :485, split into
 *                       pieces of WP_MAX_SEGMENT_TOKENS=32 :488/:506-511 with the
 *                       constant from csrc/bridge/warp_pipe_metadata.h:22, slots in
 *                       token-start order from the exclusive scan :494-503).
 *                       The reference caps the input at 256 tokens
 *                       (csrc/pybind/warp_pipe_bindings.cpp:165-166); the rule
 *                       itself is length-independent and is applied to any T here.
 *   wpo_segment_table   build_segment_table, csrc/dispatch/segment_builder.cpp:5-50
 *                       ((ids[K], offsets[K+1]) -> one segment per id, in the order
 *                       given, no split; K+1 check :9-11; K > 256 check :12-14).
 *   wpo_group_tokens    no reference counterpart: the stable grouping of tokens by
 *                       adapter id that the MI355X builder uses internally so that
 *                       every touched adapter's weights stream once per call.  It
 *                       is checked here so the device sort is checked bit-exactly.
 *
 * Parity pinning (see tests/test_oracle_segments.py): the known-answer index
 * lists held by the reference's own tests (test_add_lora_packed.py:78-125,
 * test_warp_pipe_graph_capture.py:54-55, test_segment_builder.py:35-75), an
 * independent itertools.groupby restatement on random inputs, and invariants
 * (coverage, maximality, <=32 per piece, token order) on random inputs up to
 * T = 8192.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define WPO_MAX_SEGMENT_TOKENS 32

/* Status codes mirror the product library's: 0 ok, <0 error. */
#define WPO_OK 0
#define WPO_ERR_INVALID (-1)
#define WPO_ERR_CAPACITY (-4)

/*
 * Run-length segment table over token_lora_indices in token order.
 * out: 3 int32 per segment (adapter_id, token_start, token_count), capacity
 * `cap` segments.  *num_segments receives the total count even when it
 * exceeds cap (then WPO_ERR_CAPACITY is returned and out holds the first cap).
 */
int wpo_seg_bounds(const int64_t* idx, int64_t T, int32_t* out, int64_t cap, int64_t* num_segments) {
  int64_t n = 0;
  int64_t i = 0;
  while (i < T) {
    const int64_t id = idx[i];
    int64_t j = i + 1;
    while (j < T && idx[j] == id) j++;
    if (id >= 0) {
      const int64_t run_len = j - i;
      const int64_t pieces = (run_len + WPO_MAX_SEGMENT_TOKENS - 1) / WPO_MAX_SEGMENT_TOKENS;
      for (int64_t s = 0; s < pieces; s++) {
        if (n < cap) {
          const int64_t rem = run_len - s * WPO_MAX_SEGMENT_TOKENS;
          out[3 * n + 0] = (int32_t)id;
          out[3 * n + 1] = (int32_t)(i + s * WPO_MAX_SEGMENT_TOKENS);
          out[3 * n + 2] = (int32_t)(rem < WPO_MAX_SEGMENT_TOKENS ? rem : WPO_MAX_SEGMENT_TOKENS);
        }
        n++;
      }
    }
    i = j;
  }
  *num_segments = n;
  return n > cap ? WPO_ERR_CAPACITY : WPO_OK;
}

/*
 * Host segment table from (sorted_adapter_ids[K], seg_offsets[K+1]).
 * max_segments is the table capacity (256 in the reference).
 */
int wpo_segment_table(const int32_t* ids, int64_t K, const int32_t* offsets, int64_t n_offsets,
                      int64_t max_segments, int32_t* out) {
  if (n_offsets != K + 1) return WPO_ERR_INVALID;
  if (K > max_segments) return WPO_ERR_CAPACITY;
  for (int64_t k = 0; k < K; k++) {
    out[3 * k + 0] = ids[k];
    out[3 * k + 1] = offsets[k];
    out[3 * k + 2] = offsets[k + 1] - offsets[k];
  }
  return WPO_OK;
}

/*
 * Stable grouping of tokens by adapter id (ids < 0 dropped).
 * perm[]     : token indices, grouped by ascending adapter id, token order kept
 *              inside a group (length = number of tokens with id >= 0).
 * group_id[] : adapter id of each group, ascending.
 * group_off[]: start of each group in perm (length num_groups + 1).
 * Returns the number of groups, or <0 on error.
 */
static int cmp_pair(const void* a, const void* b) {
  const int64_t* x = (const int64_t*)a;
  const int64_t* y = (const int64_t*)b;
  if (x[0] != y[0]) return x[0] < y[0] ? -1 : 1;
  if (x[1] != y[1]) return x[1] < y[1] ? -1 : 1;
  return 0;
}

int64_t wpo_group_tokens(const int64_t* idx, int64_t T, int32_t* perm, int64_t* group_id, int32_t* group_off,
                         int64_t* num_valid) {
  int64_t* pairs = (int64_t*)malloc(sizeof(int64_t) * 2 * (T > 0 ? T : 1));
  if (!pairs) return WPO_ERR_INVALID;
  int64_t m = 0;
  for (int64_t i = 0; i < T; i++) {
    if (idx[i] >= 0) {
      pairs[2 * m + 0] = idx[i];
      pairs[2 * m + 1] = i;
      m++;
    }
  }
  qsort(pairs, (size_t)m, sizeof(int64_t) * 2, cmp_pair);
  int64_t g = 0;
  for (int64_t k = 0; k < m; k++) {
    perm[k] = (int32_t)pairs[2 * k + 1];
    if (k == 0 || pairs[2 * k] != pairs[2 * (k - 1)]) {
      group_id[g] = pairs[2 * k];
      group_off[g] = (int32_t)k;
      g++;
    }
  }
  group_off[g] = (int32_t)m;
  *num_valid = m;
  free(pairs);
  return g;
}
