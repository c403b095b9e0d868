"""Engine configuration (reference: lora_warp_pipe/config.py:4-9)."""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional


@dataclass
class WarpPipeConfig:
    enabled: bool = True
    # Rank used by register_adapter when none is given (reference default 32).
    rank: int = 32
    # Staging slots of the prefetch pool.  The reference declares this field
    # but hard-codes 8 slots (warp_pipe_bindings.cpp:20); here it is honoured.
    num_staging_slots: int = 8
    # Kept for API compatibility; like the reference, nothing reads it.
    min_segment_tokens: int = 4
    # Largest T build_seg_bounds accepts before returning False.  The
    # reference's limit is 256 (WP_MAX_SEGMENTS, bindings:165-166); 8192 covers
    # the 512-token mixed-rank and 8192-token prefill workloads.
    max_tokens: int = 8192
    # HIP device ordinal; None = torch.cuda.current_device() at construction.
    device: Optional[int] = None
    # Multi-layer adapter store (not in the reference, whose store holds one
    # (A, B) per id): with a stride S > 0, register_adapter(..., layer=l)
    # keeps adapter ids 0..S-1 of layer l apart from every other layer's, and
    # shrink / expand(..., layer=l) on a build_seg_bounds table apply layer
    # l's weights to each token's adapter id.  0: one layer, plain ids.
    layer_stride: int = 0
    # Size of the device adapter table: ids (layer * layer_stride + id with a
    # multi-layer store) in [0, max_adapter_ids) are usable with
    # build_seg_bounds tables; others through build_segments only.
    max_adapter_ids: int = 65536
