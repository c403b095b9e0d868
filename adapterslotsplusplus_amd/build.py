"""Builds libwarppipe_mi355x.so (the C-ABI library) with hipcc for gfx950.

    python -m adapterslotsplusplus_amd.build

Sources are in csrc/; objects go to csrc/_build/ and the library next to this
file, where the engine loads it.  Every HIP file is compiled with packed-fp32
instructions disabled (the compiler still emits plain fp32 FMA / MFMA).
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ_DIR = os.path.join(CSRC, "_build")
LIB_NAME = "libwarppipe_mi355x.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
SOURCES = ["wp_plan.hip", "wp_apply.hip", "wp_aux.hip", "wp_engine.hip"]
ARCH = os.environ.get("WP_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# apply_kernel's first six arguments (plan pointers and grid split) are
# preloaded into SGPRs at wave launch (gfx950 kernarg preloading); kernels
# whose first argument is a struct preload nothing.
EXTRA = {"wp_apply.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=6"]}


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(line for line in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in line)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


TRACE_LIB_PATH = os.path.join(HERE, "libwarppipe_mi355x_trace.so")


def build(verbose: bool = False, trace: bool = False) -> str:
    """Compiles every source (always) and links the shared library.  trace:
    the diagnostic build (-DWP_TRACE, per-workgroup phase timestamps of the
    fused kernels; see trace_phases.py) as libwarppipe_mi355x_trace.so."""
    obj_dir = OBJ_DIR + ("_trace" if trace else "")
    lib_path = TRACE_LIB_PATH if trace else LIB_PATH
    flags = ["-DWP_TRACE=1"] if trace else []
    os.makedirs(obj_dir, exist_ok=True)
    objs = [os.path.join(obj_dir, s.rsplit(".", 1)[0] + ".o") for s in SOURCES]
    cmds = [[HIPCC, *COMMON, *flags, *EXTRA.get(s, []), "-c", os.path.join(CSRC, s), "-o", o]
            for s, o in zip(SOURCES, objs)]
    with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        outs = list(ex.map(_run, cmds))
    tmp = lib_path + ".tmp"
    outs.append(_run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", tmp, *objs]))
    os.replace(tmp, lib_path)
    if verbose:
        for o in outs:
            if o.strip():
                print(o)
    return lib_path


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv, trace="--trace" in sys.argv)
    print(path)
