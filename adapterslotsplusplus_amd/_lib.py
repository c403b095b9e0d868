"""ctypes binding of libwarppipe_mi355x.so (C ABI: include/warppipe_mi355x.h).

The library is the only compute path.  There is no CPU fallback: if the
library is missing the import of the engine raises, and if no GPU is present
engine creation raises RuntimeError.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# WP_LIB_PATH selects another build of the library (the traced one, for
# adapterslotsplusplus_amd.trace_phases).
LIB_PATH = os.environ.get("WP_LIB_PATH") or os.path.join(HERE, "libwarppipe_mi355x.so")

WP_OK = 0
WP_NOT_HANDLED = 1
WP_ERR_INVALID = -1
WP_ERR_HIP = -2
WP_ERR_UNKNOWN_ADAPTER = -3
WP_ERR_CAPACITY = -4
WP_ERR_NO_DEVICE = -5
WP_ERR_STATE = -6

WP_DTYPE_F16 = 0
WP_DTYPE_BF16 = 1

# Bits of the device error word (wp_types.h DeviceError).
DEVICE_ERR_ID_RANGE = 1
DEVICE_ERR_UNREGISTERED = 2
DEVICE_ERR_SHAPE = 4
DEVICE_ERR_SPIN = 8
DEVICE_ERR_CAPACITY = 16

# Every entry point include/warppipe_mi355x.h declares.
EXPORTED = (
    "wp_last_error", "wp_abi_version", "wp_rank_supported", "wp_block_tokens", "wp_create", "wp_destroy",
    "wp_register_adapter", "wp_register_adapter_ref", "wp_evict_adapter", "wp_has_adapter", "wp_set_entry_offset", "wp_build_segments",
    "wp_build_seg_bounds", "wp_read_segments", "wp_read_plan", "wp_read_device_errors",
    "wp_shrink", "wp_expand", "wp_shrink_expand", "wp_add_lora", "wp_prefetch_adapter", "wp_is_prefetch_ready",
    "wp_release_prefetch", "wp_add_lora_static", "wp_wait_prefetch", "wp_set_spin_limit",
    "wp_add_lora_nslice", "wp_prefetch_adapters", "wp_release_prefetches", "wp_wait_prefetches", "wp_set_trace",
    "wp_shrink_expand_slices", "wp_linear_lora", "wp_read_probe",
    "wp_set_max_adapters", "wp_read_static_errors", "wp_poll_device_errors", "wp_lora_shrink", "wp_lora_expand",
    "wp_add_bias", "wp_handoff_probe", "wp_barrier_probe",
)


class WpConfig(ctypes.Structure):
    _fields_ = [
        ("device", ctypes.c_int32),
        ("num_staging_slots", ctypes.c_int32),
        ("max_tokens", ctypes.c_int32),
        ("max_rank", ctypes.c_int32),
        ("max_adapter_ids", ctypes.c_int32),
    ]


_lib = None


def load():
    """Loads the library (once) and declares every signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m adapterslotsplusplus_amd.build` "
            "(there is no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    p = ctypes.c_void_p
    i32 = ctypes.c_int32
    i64 = ctypes.c_int64
    f32 = ctypes.c_float
    P = ctypes.POINTER
    sig = {
        "wp_last_error": ([], ctypes.c_char_p),
        "wp_abi_version": ([], ctypes.c_int),
        "wp_rank_supported": ([i32], ctypes.c_int),
        "wp_block_tokens": ([i64], ctypes.c_int),
        "wp_create": ([P(WpConfig), P(p)], ctypes.c_int),
        "wp_destroy": ([p], ctypes.c_int),
        "wp_register_adapter": ([p, i32, p, p, i32, i32, i32, f32, i32, i32, p], ctypes.c_int),
        "wp_register_adapter_ref": ([p, i32, p, p, i32, i32, i32, f32, i32, p], ctypes.c_int),
        "wp_evict_adapter": ([p, i32, p], ctypes.c_int),
        "wp_has_adapter": ([p, i32], ctypes.c_int),
        "wp_set_entry_offset": ([p, i32, i32], ctypes.c_int),
        "wp_shrink_expand": ([p, p, p, i32, i32, i32, i64, i64, i32, i32, p], ctypes.c_int),
        "wp_build_segments": ([p, p, i32, p, i32, p], ctypes.c_int),
        "wp_build_seg_bounds": ([p, p, i32, i64, p], ctypes.c_int),
        "wp_read_segments": ([p, p, i64, P(i64), p], ctypes.c_int),
        "wp_read_plan": ([p, p, i64, p, i64, P(i64), P(i64), p], ctypes.c_int),
        "wp_read_device_errors": ([p, P(ctypes.c_uint32), p], ctypes.c_int),
        "wp_shrink": ([p, p, p, i32, i32, i64, i64, i32, p], ctypes.c_int),
        "wp_expand": ([p, p, p, i32, i32, i64, i64, i64, i32, i32, p], ctypes.c_int),
        "wp_add_lora": ([p, p, p, p, i64, i32, i32, p, p, p, p, f32, i32, i32, i64, i64, i32, p], ctypes.c_int),
        "wp_prefetch_adapter": ([p, i32, P(i32)], ctypes.c_int),
        "wp_is_prefetch_ready": ([p, i32, P(i32)], ctypes.c_int),
        "wp_release_prefetch": ([p, i32, p], ctypes.c_int),
        "wp_wait_prefetch": ([p, i32, p], ctypes.c_int),
        "wp_prefetch_adapters": ([p, p, i32, p], ctypes.c_int),
        "wp_release_prefetches": ([p, p, i32, p], ctypes.c_int),
        "wp_wait_prefetches": ([p, p, i32, p], ctypes.c_int),
        "wp_set_trace": ([p, p, i64], ctypes.c_int),
        "wp_shrink_expand_slices": ([p, p, p, i32, i32, p, i32, p, p, i32, i64, i64, i32, p], ctypes.c_int),
        "wp_linear_lora": ([p, p, p, p, i64, p, p, i64, p, i64, i32, f32, i32, i32, i32, i64, i32, p], ctypes.c_int),
        "wp_add_lora_nslice": ([p, p, p, i32, p, p, p, p, p, p, i32, f32, i32, i32, i64, i64, i32, p], ctypes.c_int),
        "wp_set_spin_limit": ([p, ctypes.c_uint32], ctypes.c_int),
        "wp_read_probe": ([p, p, i64, p, p], ctypes.c_int),
        "wp_add_lora_static": ([p, p, p, i32, i64, p, i64, i32, i32, p, p, p, p, f32, i32, i32, i64, i32, p],
                               ctypes.c_int),
        "wp_set_max_adapters": ([p, i64], ctypes.c_int),
        "wp_read_static_errors": ([i32, p, p], ctypes.c_int),
        "wp_poll_device_errors": ([p, P(ctypes.c_uint32), p], ctypes.c_int),
        "wp_lora_shrink": ([p, p, i64, i64, p, i32, p, p, i32, f32, i32, i32, i64, i32, p], ctypes.c_int),
        "wp_lora_expand": ([p, p, i64, p, i32, i64, i64, i32, p, p, p, p, p, p, i32, i32, i64, i32, i32, p],
                           ctypes.c_int),
        "wp_add_bias": ([p, p, i64, i32, p, p, p, p, i32, i64, i32, p], ctypes.c_int),
        "wp_handoff_probe": ([p, i64, p, i64, p, i64, p, p, i32, i32, i32, p], ctypes.c_int),
        "wp_barrier_probe": ([p, i32, i32, i32, p, p], ctypes.c_int),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def last_error() -> str:
    return load().wp_last_error().decode("utf-8", "replace")


def check(rc: int, what: str = "") -> int:
    """Maps an error status to RuntimeError (the reference's TORCH_CHECK /
    std::runtime_error convention); returns WP_OK / WP_NOT_HANDLED unchanged."""
    if rc < 0:
        msg = last_error()
        raise RuntimeError(f"{what}: {msg}" if what and not msg.startswith(what) else (msg or what))
    return rc
