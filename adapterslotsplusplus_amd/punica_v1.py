"""vLLM V1's LoRA op surface (PunicaWrapperGPU) on the MI355X engine.

The reference hooks only vLLM 0.6's PunicaWrapper.add_lora and scopes the V1
op interface out (lora_warp_pipe/punica_wrapper.py:8-16).  V1's LoRA layers
call four methods of their punica wrapper instead:

  add_shrink(y, x, lora_a_stacked, scale)
      for each slice s: y[s] += scale * x . lora_a_stacked[s][id]^T
      (y: fp32 [n_slices, T, r]);
  add_expand(y, x, lora_b_stacked, lora_bias_stacked, output_slices,
             offset_start=0, add_inputs=True)
      y[:, off_s : off_s + o_s] += x[s] . lora_b_stacked[s][id]^T (+ bias[s][id]),
      windows consecutive from offset_start (V1 adds whatever add_inputs says);
  add_lora_embedding(y, x, lora_b_stacked, add_inputs=True)
      y (+)= x . lora_b_stacked[id]^T;
  add_lora_linear(y, x, lora_a_stacked, lora_b_stacked, lora_bias_stacked,
                  scale, output_slices, *, buffer=None)
      bias, then shrink into an fp32 buffer, then expand, for every slice.

WarpPipeV1Mixin overrides those four (add_lora_logits, on the sampler's
indices, stays with the parent) and update_metadata, which after the parent's
bookkeeping builds the step's segment table from token_lora_indices with the
engine's build_seg_bounds (prefill and decode alike: the engine takes up to
WarpPipeConfig.max_tokens tokens) and reports tokens an earlier step had to
skip.  add_lora_linear runs the bias (if any) and then all slices' shrink and
expand in ONE launch with no fp32 buffer round trip (the caller's `buffer`,
if given, is left untouched); add_shrink / add_expand keep V1's fp32 buffer
contract.  Rounding points are V1's: the fp32 shrink result is rounded to the
activation dtype before the expand, which accumulates in fp32 and rounds once
with y.

Fallbacks (the parent's method runs): AS_WARP_PIPE != "1", CPU tensors, a
step whose table could not be built (more tokens than max_tokens), fewer rows
than the table covers, slices of different ranks, more than 4 slices, or a
rank without kernels.
"""
from __future__ import annotations

from typing import Optional, Sequence, Tuple, Union

import torch

from .punica_wrapper import _WARP_PIPE_IMPORT_OK, _get_engine, report_device_errors, warp_pipe_available


def _ranks(ws: Sequence[torch.Tensor], axis: int) -> set:
    return {int(w.size(axis)) for w in ws}


class WarpPipeV1Mixin:
    """update_metadata / add_shrink / add_expand / add_lora_embedding /
    add_lora_linear overrides; combine with vLLM V1's PunicaWrapperGPU."""

    _wp_step_ok: bool = False
    _wp_tokens: int = 0

    def update_metadata(self, mapping, lora_index_to_id, max_loras, vocab_size, extra_vocab_size, *args,
                        **kwargs) -> None:
        super().update_metadata(mapping, lora_index_to_id, max_loras, vocab_size, extra_vocab_size,  # type: ignore[misc]
                                *args, **kwargs)
        self._wp_step_ok = False
        if warp_pipe_available():
            engine = _get_engine()
            report_device_errors(engine.poll_device_errors(), "update_metadata")
            idx = self.token_lora_indices  # type: ignore[attr-defined]
            self._wp_tokens = int(idx.numel())
            self._wp_step_ok = bool(engine.build_seg_bounds(idx))

    def _wp_ok(self, x: torch.Tensor, rows: int) -> bool:
        return self._wp_step_ok and warp_pipe_available() and x.is_cuda and rows >= self._wp_tokens

    def add_shrink(self, y: Union[Tuple[torch.Tensor, ...], torch.Tensor], x: torch.Tensor,
                   lora_a_stacked: Tuple[torch.Tensor, ...], scale: float, **kwargs):
        x2 = x.view(-1, x.shape[-1])
        if (not self._wp_ok(x2, int(x2.size(0))) or len(lora_a_stacked) > 4 or len(_ranks(lora_a_stacked, -2)) != 1
                or not _get_engine().lora_shrink(y, x2, lora_a_stacked, float(scale))):
            return super().add_shrink(y, x, lora_a_stacked, scale, **kwargs)  # type: ignore[misc]
        return None

    def add_expand(self, y: torch.Tensor, x: Union[Tuple[torch.Tensor, ...], torch.Tensor],
                   lora_b_stacked: Tuple[torch.Tensor, ...], lora_bias_stacked: Optional[Tuple[torch.Tensor, ...]],
                   output_slices: Tuple[int, ...], offset_start: int = 0, add_inputs=True, **kwargs) -> None:
        h = torch.stack(list(x)) if isinstance(x, (list, tuple)) else x
        rows = int(y.numel() // y.shape[-1])
        if (not self._wp_ok(h, rows) or len(lora_b_stacked) > 4 or len(_ranks(lora_b_stacked, -1)) != 1
                or h.dim() != 3 or int(h.size(0)) != len(output_slices)
                or not _get_engine().lora_expand(y, h, lora_b_stacked, output_slices, offset_start, True,
                                                 lora_bias_stacked)):
            return super().add_expand(y, x, lora_b_stacked, lora_bias_stacked, output_slices,  # type: ignore[misc]
                                      offset_start, add_inputs, **kwargs)
        return None

    def add_lora_embedding(self, y: torch.Tensor, x: torch.Tensor, lora_b_stacked: torch.Tensor, add_inputs: bool = True,
                           **kwargs) -> None:
        rows = int(y.numel() // y.shape[-1])
        if (not self._wp_ok(x, rows)
                or not _get_engine().lora_expand(y, x.view(1, -1, x.shape[-1]), (lora_b_stacked,),
                                                 (int(lora_b_stacked.size(-2)),), 0, bool(add_inputs))):
            return super().add_lora_embedding(y, x, lora_b_stacked, add_inputs, **kwargs)  # type: ignore[misc]
        return None

    def add_lora_linear(self, y: torch.Tensor, x: torch.Tensor, lora_a_stacked: Tuple[torch.Tensor, ...],
                        lora_b_stacked: Tuple[torch.Tensor, ...], lora_bias_stacked: Optional[Tuple[torch.Tensor, ...]],
                        scale: float, output_slices: Tuple[int, ...], *, buffer=None, **kwargs) -> None:
        x2 = x.view(-1, x.shape[-1])
        n = len(output_slices)
        engine = _get_engine() if self._wp_ok(x2, int(x2.size(0))) else None
        ranks = _ranks(lora_b_stacked, -1) | _ranks(lora_a_stacked, -2)
        if (engine is None or n > 4 or len(lora_a_stacked) != n or len(lora_b_stacked) != n or len(ranks) != 1
                or not engine._rank_ok(ranks.pop())):
            return super().add_lora_linear(y, x, lora_a_stacked, lora_b_stacked,  # type: ignore[misc]
                                           lora_bias_stacked, scale, output_slices, buffer=buffer, **kwargs)
        y2 = y.view(-1, y.shape[-1])
        if lora_bias_stacked is not None:
            engine.add_bias(y2, lora_bias_stacked, output_slices, int(lora_b_stacked[0].size(0)))
        if not engine.add_lora_packed_nslice(y2, x2, lora_a_stacked, lora_b_stacked, float(scale), output_slices):
            raise RuntimeError("WarpPipe add_lora_linear: the kernels refused a call they had accepted")
        return None


_CLASS_CACHE: dict = {}


def warp_pipe_v1_class_for(base: type) -> type:
    """The WarpPipe subclass of a V1 PunicaWrapper class (cached)."""
    if issubclass(base, WarpPipeV1Mixin):
        return base
    cls = _CLASS_CACHE.get(base)
    if cls is None:
        cls = type(f"{base.__name__}WarpPipeV1", (WarpPipeV1Mixin, base), {})
        _CLASS_CACHE[base] = cls
    return cls


def install_warp_pipe_v1(lora_manager) -> bool:
    """Reassigns the live V1 wrapper's __class__ to its WarpPipe subclass (the
    same lora_manager._adapter_manager.punica_wrapper chain as
    install_warp_pipe_add_lora).  False (no-op) if lora_manager is None, the
    library is missing, there is no wrapper, or it is already switched."""
    if lora_manager is None or not _WARP_PIPE_IMPORT_OK:
        return False
    adapter_manager = getattr(lora_manager, "_adapter_manager", None)
    wrapper = getattr(adapter_manager, "punica_wrapper", None) if adapter_manager is not None else None
    if wrapper is None or isinstance(wrapper, WarpPipeV1Mixin):
        return False
    wrapper.__class__ = warp_pipe_v1_class_for(type(wrapper))
    return True
