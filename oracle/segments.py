"""ctypes front end of oracle/seg_oracle.c -- TEST INFRASTRUCTURE ONLY.

Restates (see seg_oracle.c for line-level citations):
  seg_bounds     -- build_seg_bounds_kernel, csrc/kernels/warp_pipe_r32.cu:461-512
  segment_table  -- build_segment_table, csrc/dispatch/segment_builder.cpp:5-50
  group_tokens   -- the stable by-adapter grouping the MI355X builder adds (no
                    reference counterpart)
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libwpo.so")
_lib = None

MAX_SEGMENT_TOKENS = 32  # csrc/bridge/warp_pipe_metadata.h:22
REFERENCE_MAX_SEGMENTS = 256  # csrc/bridge/warp_pipe_metadata.h:10


def build() -> str:
    """Compile seg_oracle.c with gcc (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH) or os.path.getmtime(_LIB_PATH) < os.path.getmtime(
                os.path.join(_HERE, "seg_oracle.c")):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        lib.wpo_seg_bounds.argtypes = [p, i64, p, i64, ctypes.POINTER(i64)]
        lib.wpo_seg_bounds.restype = ctypes.c_int
        lib.wpo_segment_table.argtypes = [p, i64, p, i64, i64, p]
        lib.wpo_segment_table.restype = ctypes.c_int
        lib.wpo_group_tokens.argtypes = [p, i64, p, p, p, ctypes.POINTER(i64)]
        lib.wpo_group_tokens.restype = ctypes.c_int64
        _lib = lib
    return _lib


def seg_bounds(idx) -> np.ndarray:
    """Run-length segment table of token_lora_indices -> int32 array [n, 3]
    of (adapter_id, token_start, token_count), in token order."""
    lib = _load()
    a = np.ascontiguousarray(np.asarray(idx, dtype=np.int64).reshape(-1))
    T = a.shape[0]
    cap = max(T, 1)
    out = np.zeros((cap, 3), dtype=np.int32)
    n = ctypes.c_int64(0)
    rc = lib.wpo_seg_bounds(a.ctypes.data, T, out.ctypes.data, cap, ctypes.byref(n))
    if rc != 0:
        raise RuntimeError(f"wpo_seg_bounds failed rc={rc}")
    return out[: n.value].copy()


def segment_table(sorted_adapter_ids, seg_offsets, max_segments: int = REFERENCE_MAX_SEGMENTS) -> np.ndarray:
    """Host table (adapter_id, token_start, token_count) per given segment.
    Raises RuntimeError on the reference's two error conditions."""
    lib = _load()
    ids = np.ascontiguousarray(np.asarray(sorted_adapter_ids, dtype=np.int32).reshape(-1))
    off = np.ascontiguousarray(np.asarray(seg_offsets, dtype=np.int32).reshape(-1))
    K = ids.shape[0]
    out = np.zeros((max(K, 1), 3), dtype=np.int32)
    rc = lib.wpo_segment_table(ids.ctypes.data, K, off.ctypes.data, off.shape[0], max_segments, out.ctypes.data)
    if rc == -1:
        raise RuntimeError("seg_offsets must have K+1 entries")
    if rc == -4:
        raise RuntimeError("K exceeds the segment-table capacity")
    if rc != 0:
        raise RuntimeError(f"wpo_segment_table failed rc={rc}")
    return out[:K].copy()


def group_tokens(idx):
    """Stable grouping of tokens by ascending adapter id.
    Returns (perm int32 [n_valid], group_ids int64 [G], group_off int32 [G+1])."""
    lib = _load()
    a = np.ascontiguousarray(np.asarray(idx, dtype=np.int64).reshape(-1))
    T = a.shape[0]
    perm = np.zeros(max(T, 1), dtype=np.int32)
    gid = np.zeros(max(T, 1), dtype=np.int64)
    goff = np.zeros(max(T, 1) + 1, dtype=np.int32)
    nv = ctypes.c_int64(0)
    g = lib.wpo_group_tokens(a.ctypes.data, T, perm.ctypes.data, gid.ctypes.data, goff.ctypes.data,
                             ctypes.byref(nv))
    if g < 0:
        raise RuntimeError("wpo_group_tokens failed")
    return perm[: nv.value].copy(), gid[:g].copy(), goff[: g + 1].copy()
