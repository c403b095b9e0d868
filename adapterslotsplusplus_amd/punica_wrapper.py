"""Routes vLLM-style PunicaWrapper.add_lora() calls to the MI355X engine.

Reference: lora_warp_pipe/punica_wrapper.py:100-159 (FusedPunicaWrapperWarpPipe)
and :219-238 (install_warp_pipe_add_lora).  Same contract:

  * update_metadata(...) runs the parent first, then -- outside any graph
    capture and once per decode step -- builds the segment table from
    self.token_lora_indices with the engine's build_seg_bounds;
  * add_lora(y, x, wa_t_all, wb_t_all, scale, y_offset, y_slice_size, *, buffer)
    runs the grouped HIP kernels, or falls back to the parent's add_lora for
    prefill, when AS_WARP_PIPE != "1", for CPU tensors, or for a rank without
    kernels;
  * install_warp_pipe_add_lora(lora_manager) switches the live wrapper's class
    with __class__ reassignment and returns False when there is nothing to do.

Added: add_lora_packed_nslice (vLLM's packed q/k/v and gate/up layers, one
lora_a / lora_b per slice) runs every slice in one launch; the reference
leaves it to its parent class (punica_wrapper.py:8-16).  update_metadata
also reports tokens an earlier step's kernels had to skip (the engine's
device error word, polled without a host wait): a logged warning, or
RuntimeError with AS_WARP_PIPE_STRICT=1.

Differences: the reference can only subclass AdapterSlots' FusedPunicaWrapper
(an absent dependency here), so the overrides live in a mixin that is combined
with whatever class the live wrapper has; sliced outputs (y_offset /
y_slice_size) run on the kernels instead of falling back; and a step whose
build_seg_bounds returned False (more tokens than the engine's capacity) falls
back for that step instead of reusing the previous step's table.
"""
from __future__ import annotations

import logging
import os
from typing import Optional

import torch

try:
    from .engine import WarpPipeEngine

    _WARP_PIPE_IMPORT_OK = True
except ImportError:  # library not built: every entry point falls back
    WarpPipeEngine = None  # type: ignore[assignment,misc]
    _WARP_PIPE_IMPORT_OK = False

_engine: Optional["WarpPipeEngine"] = None


def _get_engine() -> "WarpPipeEngine":
    """Lazy process-wide engine (needs a live GPU context, so never at import)."""
    global _engine
    if _engine is None:
        _engine = WarpPipeEngine()
    return _engine


def warp_pipe_available() -> bool:
    return _WARP_PIPE_IMPORT_OK and os.environ.get("AS_WARP_PIPE", "0") == "1"


_log = logging.getLogger(__name__)
_ERROR_NAMES = ((1, "adapter id outside the stacked weights"), (2, "adapter id not registered"),
                (4, "adapter shape does not match the call"), (8, "a wait on partial results gave up"),
                (16, "more adapter blocks than the call's grid"))
# Every device error bit reported so far in this process (OR of them).
device_errors_seen = 0


def describe_device_errors(bits: int) -> str:
    return ", ".join(name for bit, name in _ERROR_NAMES if bits & bit) or "none"


def report_device_errors(bits: int, where: str) -> int:
    """Records device error bits that an earlier step's kernels set (tokens
    they skipped, leaving those rows without their LoRA delta): ORs them into
    `device_errors_seen`, logs a warning, and raises RuntimeError instead when
    AS_WARP_PIPE_STRICT=1.  Returns `bits`."""
    global device_errors_seen
    if bits:
        device_errors_seen |= bits
        msg = (f"WarpPipe: an earlier step skipped tokens (device errors 0x{bits:x}: "
               f"{describe_device_errors(bits)}); reported at {where}")
        if os.environ.get("AS_WARP_PIPE_STRICT", "0") == "1":
            raise RuntimeError(msg)
        _log.warning(msg)
    return bits


class WarpPipeAddLoraMixin:
    """update_metadata / add_lora overrides; combine with a PunicaWrapper class."""

    _wp_step_ok: bool = False

    def update_metadata(self, mapping, lora_index_to_id, max_loras, vocab_size, extra_vocab_size,
                        long_lora_context=None) -> None:
        super().update_metadata(mapping, lora_index_to_id, max_loras, vocab_size, extra_vocab_size,  # type: ignore[misc]
                                long_lora_context)
        self._wp_step_ok = False
        if not self.is_prefill and warp_pipe_available():  # type: ignore[attr-defined]
            engine = _get_engine()
            # Errors of earlier steps, without a host wait: the bits a
            # previous poll moved to host memory, once that move has landed.
            report_device_errors(engine.poll_device_errors(), "update_metadata")
            self._wp_step_ok = bool(engine.build_seg_bounds(self.token_lora_indices))  # type: ignore[attr-defined]

    def add_lora(self, y: torch.Tensor, x: torch.Tensor, wa_t_all: torch.Tensor, wb_t_all: torch.Tensor,
                 scale: float, y_offset: Optional[int] = None, y_slice_size: Optional[int] = None, *,
                 buffer: Optional[torch.Tensor] = None) -> None:
        # No capture guard: the segment table is built on the device and the
        # kernels read it on every replay with fixed launch parameters.
        if (self.is_prefill  # type: ignore[attr-defined]
                or not self._wp_step_ok
                or not warp_pipe_available()
                or not x.is_cuda
                or not _get_engine()._ext.rank_supported(int(wb_t_all.size(-1)))):
            return super().add_lora(y, x, wa_t_all, wb_t_all, scale, y_offset, y_slice_size,  # type: ignore[misc]
                                    buffer=buffer)
        handled = _get_engine().add_lora_packed(y, x, wa_t_all, wb_t_all, float(scale), y_offset, y_slice_size)
        if not handled:
            return super().add_lora(y, x, wa_t_all, wb_t_all, scale, y_offset, y_slice_size,  # type: ignore[misc]
                                    buffer=buffer)
        return None

    def add_lora_packed_nslice(self, y: torch.Tensor, x: torch.Tensor, lora_a_stacked, lora_b_stacked, scale: float,
                               output_slices) -> None:
        """vLLM's packed layers (q/k/v, gate/up): 2-3 slices that share x, each
        with its own lora_a / lora_b.  All slices run in one launch on the
        kernels; the same fallbacks as add_lora, plus slices of different
        ranks.  The reference leaves this method to its parent
        (punica_wrapper.py:8-16)."""
        ranks = {int(b.size(-1)) for b in lora_b_stacked}
        if (self.is_prefill  # type: ignore[attr-defined]
                or not self._wp_step_ok
                or not warp_pipe_available()
                or not x.is_cuda
                or len(ranks) != 1
                or len(output_slices) > 4
                or not _get_engine()._ext.rank_supported(ranks.pop())):
            return super().add_lora_packed_nslice(y, x, lora_a_stacked, lora_b_stacked, scale,  # type: ignore[misc]
                                                  output_slices)
        if not _get_engine().add_lora_packed_nslice(y, x, lora_a_stacked, lora_b_stacked, float(scale), output_slices):
            return super().add_lora_packed_nslice(y, x, lora_a_stacked, lora_b_stacked, scale,  # type: ignore[misc]
                                                  output_slices)
        return None


_CLASS_CACHE: dict = {}


def warp_pipe_class_for(base: type) -> type:
    """The WarpPipe subclass of a PunicaWrapper class (cached)."""
    if issubclass(base, WarpPipeAddLoraMixin):
        return base
    cls = _CLASS_CACHE.get(base)
    if cls is None:
        cls = type(f"{base.__name__}WarpPipe", (WarpPipeAddLoraMixin, base), {})
        _CLASS_CACHE[base] = cls
    return cls


try:  # the reference's concrete class, when AdapterSlots is installed
    from adapter_slots.kernel.fused_punica_wrapper import FusedPunicaWrapper  # type: ignore

    FusedPunicaWrapperWarpPipe = warp_pipe_class_for(FusedPunicaWrapper)
except ImportError:
    FusedPunicaWrapperWarpPipe = None


def install_warp_pipe_add_lora(lora_manager) -> bool:
    """Reassigns the live wrapper's __class__ to its WarpPipe subclass.
    Returns False (no-op) if lora_manager is None, the library is missing,
    there is no wrapper, or it is already switched."""
    if lora_manager is None or not _WARP_PIPE_IMPORT_OK:
        return False
    adapter_manager = getattr(lora_manager, "_adapter_manager", None)
    if adapter_manager is None:
        return False
    wrapper = getattr(adapter_manager, "punica_wrapper", None)
    if wrapper is None or isinstance(wrapper, WarpPipeAddLoraMixin):
        return False
    wrapper.__class__ = warp_pipe_class_for(type(wrapper))
    return True
