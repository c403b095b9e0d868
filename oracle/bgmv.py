"""torch fp32 CPU restatement of the reference's shrink / expand / add_lora --
TEST INFRASTRUCTURE ONLY (the checker, never the thing measured or shipped).

Math and rounding points, restated from the reference:
  shrink  H[t, :] = rn_io(alpha_seg * sum_d X[t, d] * A_seg[:, d])   fp32 accumulation
          tests/correctness/reference_bgmv.py:4-12 (alpha applied once, in shrink);
          rounding to the I/O dtype after alpha: csrc/kernels/warp_pipe_r32.cu:129, :360;
          rows outside every segment stay 0: csrc/pybind/warp_pipe_bindings.cpp:134.
  expand  Y[t, o] = rn_io(Y[t, o] + sum_r H[t, r] * B_seg[o, r])      fp32 accumulation, no alpha
          tests/correctness/reference_bgmv.py:15-18; rounding once: warp_pipe_r32.cu:194, :417.
  add_lora  the same two steps per segment of the build_seg_bounds table, with
          A = wa_t_all[adapter_id], B = wb_t_all[adapter_id] and the call's scale
          (warp_pipe_r32.cu:292, :377; warp_pipe_bindings.cpp:195-234); rows whose
          id is < 0 are untouched (tests/correctness/test_add_lora_packed.py:35-45).

Deliberate differences from the reference kernels (the reference is defective
there; both are documented in the product code too):
  * a host-built segment longer than 32 tokens is applied to all of its tokens
    (the reference's fixed grid silently drops tokens past 32);
  * y_offset / multi-slice expand writes into a column window of a wider Y (the
    reference hook falls back to the stock path for these,
    lora_warp_pipe/punica_wrapper.py:147-155).

Parity pinning for this module: tests/test_oracle_bgmv.py checks it against a
float64 brute-force triple loop with the same rounding points on random tiny
cases, against structural special cases (one-hot A/B select columns, alpha=0,
ids < 0), and shows that dropping the H rounding point is detected.
"""
from __future__ import annotations

from typing import Dict, Iterable, Sequence, Tuple

import torch


def shrink_rows(x_rows: torch.Tensor, A: torch.Tensor, alpha: float) -> torch.Tensor:
    """rn_io(alpha * x_rows @ A^T) with fp32 accumulation; A is [r, d]."""
    return ((x_rows.float() @ A.float().T) * alpha).to(x_rows.dtype)


def expand_rows(h_rows: torch.Tensor, B: torch.Tensor, y_rows: torch.Tensor) -> torch.Tensor:
    """rn_io(y_rows + h_rows @ B^T) with fp32 accumulation; B is [o, r]."""
    return (y_rows.float() + h_rows.float() @ B.float().T).to(y_rows.dtype)


def shrink(X: torch.Tensor, segments: Iterable[Sequence[int]], adapters: Dict[int, Tuple], rank: int,
           total_tokens: int | None = None) -> torch.Tensor:
    """Per-segment shrink. adapters[id] = (A [r_a, d], B [o, r_a], alpha).
    H is [T, rank] and zero outside the segments; an adapter of rank r_a < rank
    fills only the first r_a columns of its rows (mixed-rank calls)."""
    T = X.shape[0] if total_tokens is None else total_tokens
    H = torch.zeros(T, rank, dtype=X.dtype)
    for aid, ts, tc in segments:
        if tc <= 0:
            continue
        A, _, alpha = adapters[int(aid)]
        H[ts:ts + tc, :A.shape[0]] = shrink_rows(X[ts:ts + tc], A, alpha)
    return H


def expand(H: torch.Tensor, Y: torch.Tensor, segments: Iterable[Sequence[int]], adapters: Dict[int, Tuple],
           y_offset: int = 0) -> torch.Tensor:
    """Per-segment expand into columns [y_offset, y_offset + o) of a copy of Y."""
    Yn = Y.clone()
    for aid, ts, tc in segments:
        if tc <= 0:
            continue
        _, B, _ = adapters[int(aid)]
        r, o = B.shape[1], B.shape[0]
        Yn[ts:ts + tc, y_offset:y_offset + o] = expand_rows(H[ts:ts + tc, :r], B, Yn[ts:ts + tc, y_offset:y_offset + o])
    return Yn


def add_lora(y: torch.Tensor, x: torch.Tensor, wa_t_all: torch.Tensor, wb_t_all, scale: float,
             segments: Iterable[Sequence[int]], y_offsets: Sequence[int] | int = 0) -> torch.Tensor:
    """add_lora over the build_seg_bounds table; returns the updated copy of y.

    wa_t_all: [L, 1, r, d] (or [L, r, d]); wb_t_all: one [L, 1, o, r] tensor or a
    list of them (slices sharing one H, written at y_offsets[i])."""
    wbs = list(wb_t_all) if isinstance(wb_t_all, (list, tuple)) else [wb_t_all]
    offs = [y_offsets] * len(wbs) if isinstance(y_offsets, int) else list(y_offsets)
    x2 = x.reshape(-1, x.shape[-1])
    yn = y.reshape(-1, y.shape[-1]).clone()
    L = wa_t_all.shape[0]
    for aid, ts, tc in segments:
        if tc <= 0:
            continue
        a = wa_t_all[int(aid)].reshape(-1, wa_t_all.shape[-1])
        h = shrink_rows(x2[ts:ts + tc], a, scale)
        for wb, off in zip(wbs, offs):
            assert wb.shape[0] == L
            b = wb[int(aid)].reshape(-1, wb.shape[-1])
            o = b.shape[0]
            yn[ts:ts + tc, off:off + o] = expand_rows(h, b, yn[ts:ts + tc, off:off + o])
    return yn.reshape(y.shape)


def add_lora_nslice(y: torch.Tensor, x: torch.Tensor, wa_t_alls: Sequence[torch.Tensor],
                    wb_t_alls: Sequence[torch.Tensor], scale: float, segments: Iterable[Sequence[int]],
                    y_offsets: Sequence[int]) -> torch.Tensor:
    """add_lora over the build_seg_bounds table with one A per slice: slice i
    is an independent add_lora with (wa_t_alls[i], wb_t_alls[i]) into columns
    [y_offsets[i], + o_i) of y -- vLLM's PunicaWrapper.add_lora_packed_nslice
    is that loop over slices (one add_lora per slice, offsets accumulated from
    output_slices), named by the reference at lora_warp_pipe/punica_wrapper.py:8-16.
    Each slice's H is rounded after scale and y once per slice, as in add_lora
    (warp_pipe_r32.cu:129, :194).  Returns the updated copy of y."""
    yn = y
    for wa, wb, off in zip(wa_t_alls, wb_t_alls, y_offsets):
        yn = add_lora(yn, x, wa, wb, scale, segments, off)
    return yn

