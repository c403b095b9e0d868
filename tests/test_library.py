"""CPU tier for the C-ABI library: it loads, exports every entry point the
public header declares, and behaves correctly without a GPU (no compute calls
are made here)."""
import ctypes
import os
import re

import pytest
import torch

from adapterslotsplusplus_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "warppipe_mi355x.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(wp_[a-z0-9_]+)\s*\(", src)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    declared = declared_functions()
    assert len(declared) >= 19
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
    assert sorted(_lib.EXPORTED) == declared


def test_abi_version_and_rank_table():
    lib = _lib.load()
    assert lib.wp_abi_version() == 2
    # reference: test_rank_variants.py:97-103
    for r in (8, 16, 32, 64):
        assert lib.wp_rank_supported(r) == 1
    for r in (0, 4, 24, 48, 128, -32):
        assert lib.wp_rank_supported(r) == 0


def test_block_size_rule():
    lib = _lib.load()
    for T, bt in ((0, 16), (1, 16), (256, 16), (512, 16), (513, 64), (2048, 64), (8192, 64)):
        assert lib.wp_block_tokens(T) == bt, T


def test_library_contains_gfx950_code():
    data = open(_lib.LIB_PATH, "rb").read()
    assert b"gfx950" in data


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU behaviour")
def test_create_without_gpu_fails_loudly():
    lib = _lib.load()
    h = ctypes.c_void_p(None)
    rc = lib.wp_create(None, ctypes.byref(h))
    assert rc == _lib.WP_ERR_NO_DEVICE
    assert "no HIP device" in _lib.last_error()
    from adapterslotsplusplus_amd import WarpPipeEngine
    with pytest.raises(RuntimeError, match="GPU"):
        WarpPipeEngine()


def test_null_engine_arguments_are_errors_not_crashes():
    lib = _lib.load()
    assert lib.wp_destroy(None) == 0
    assert lib.wp_build_seg_bounds(None, None, 1, 4, None) == _lib.WP_ERR_INVALID
    assert lib.wp_shrink(None, None, None, 64, 32, 1, 32, 1, None) == _lib.WP_ERR_INVALID
    assert lib.wp_has_adapter(None, 0) == 0
    assert lib.wp_shrink_expand(None, None, None, 64, 64, 32, 1, 64, 0, 1, None) == _lib.WP_ERR_INVALID
    assert lib.wp_set_entry_offset(None, 0, 0) == _lib.WP_ERR_INVALID
    slot = ctypes.c_int32(5)
    assert lib.wp_prefetch_adapter(None, 0, ctypes.byref(slot)) == _lib.WP_ERR_INVALID
    with pytest.raises(RuntimeError, match="engine is NULL"):
        _lib.check(lib.wp_evict_adapter(None, 0, None), "evict_adapter")
    assert lib.wp_read_probe(None, None, 0, None, None) == _lib.WP_ERR_INVALID


@pytest.mark.parametrize("compiler,std", [("gcc", "-std=c99"), ("g++", "-std=c++17")])
def test_header_is_plain_c_and_cpp(tmp_path, compiler, std):
    """The public header compiles on its own as C99 and as C++17 with every
    warning an error (no HIP or torch headers needed by a caller)."""
    import shutil
    import subprocess

    if shutil.which(compiler) is None:
        pytest.skip(f"{compiler} not found")
    src = tmp_path / ("use.c" if compiler == "gcc" else "use.cc")
    src.write_text('#include "warppipe_mi355x.h"\n'
                   "int probe(void) { return wp_rank_supported(32) + wp_abi_version(); }\n")
    r = subprocess.run([compiler, std, "-Wall", "-Wextra", "-pedantic", "-Werror", "-fsyntax-only",
                        "-I", os.path.join(ROOT, "include"), str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
