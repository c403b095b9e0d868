"""AdapterSlots++ grouped multi-LoRA apply, MI355X (gfx950) native.

WarpPipeEngine is the drop-in for the reference's lora_warp_pipe.WarpPipeEngine;
the compute runs in libwarppipe_mi355x.so (hand-written HIP kernels, C ABI in
include/warppipe_mi355x.h).
"""
from .config import WarpPipeConfig
from .engine import WarpPipeEngine

__all__ = ["WarpPipeConfig", "WarpPipeEngine"]
