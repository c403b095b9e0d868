"""GPU: wp_add_lora_static, the entry point that allocates nothing, against the
engine's wp_build_seg_bounds + wp_add_lora on the same inputs (and both
against the CPU oracle).  Called through the C ABI with ctypes."""
import ctypes

import pytest
import torch

from adapterslotsplusplus_amd import WarpPipeEngine, _lib
from oracle import bgmv
from oracle import segments as so
from tests.helpers import announce, assert_close, randn

pytestmark = pytest.mark.gpu


def static_call(y, x, idx, wa, wbs, offs, scale, rank):
    """wp_add_lora_static through ctypes; returns the status."""
    lib = _lib.load()
    n = len(wbs)
    wb_ptrs = (ctypes.c_void_p * n)(*[w.data_ptr() for w in wbs])
    wb_strides = (ctypes.c_int64 * n)(*[int(w.stride(0)) for w in wbs])
    outs = (ctypes.c_int32 * n)(*[int(w.size(-2)) for w in wbs])
    off_arr = (ctypes.c_int32 * n)(*[int(v) for v in offs])
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return lib.wp_add_lora_static(ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                                  ctypes.c_void_p(idx.data_ptr()), 1 if idx.dtype == torch.int64 else 0,
                                  int(idx.numel()), ctypes.c_void_p(wa.data_ptr()), int(wa.stride(0)),
                                  int(wa.size(0)), n, wb_ptrs, wb_strides, outs, off_arr, float(scale), int(rank),
                                  int(x.size(1)), int(y.size(1)), _lib.WP_DTYPE_BF16 if y.dtype == torch.bfloat16
                                  else _lib.WP_DTYPE_F16, stream)


def case(T, L, rank, d, widths, dtype, seed, idx_dtype=torch.int64):
    g = torch.Generator().manual_seed(seed)
    idx = torch.randint(-1, L, (T,), generator=g).to(idx_dtype)
    x = randn((T, d), seed + 1, dtype)
    wa = randn((L, 1, rank, d), seed + 2, dtype, 0.02)
    wbs = [randn((L, 1, o, rank), seed + 3 + i, dtype, 0.02) for i, o in enumerate(widths)]
    offs = [sum(widths[:i]) for i in range(len(widths))]
    y0 = randn((T, sum(widths)), seed + 9, dtype)
    return idx, x, wa, wbs, offs, y0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_static_matches_engine_two_calls(dtype):
    """Two calls in a row, the second smaller: each equals the engine's result
    bit for bit and the oracle within the tolerance."""
    engine = WarpPipeEngine()
    for k, (T, L, rank, d, widths, idt) in enumerate([(256, 64, 32, 4096, [4096, 1024, 1024], torch.int64),
                                                       (37, 5, 16, 512, [384], torch.int32)]):
        announce(f"add_lora_static call {k}: T={T} L={L} r={rank} d={d} widths={widths} {dtype} idx {idt}")
        idx, x, wa, wbs, offs, y0 = case(T, L, rank, d, widths, dtype, 100 + k, idt)
        xd, wad, wbd, idxd = x.cuda(), wa.cuda(), [w.cuda() for w in wbs], idx.cuda()
        y_static = y0.cuda()
        assert static_call(y_static, xd, idxd, wad, wbd, offs, 0.5, rank) == _lib.WP_OK, _lib.last_error()
        y_engine = y0.cuda()
        assert engine.build_seg_bounds(idxd)
        assert engine.add_lora_slices(y_engine, xd, wad, wbd, 0.5, offs)
        torch.cuda.synchronize()
        assert torch.equal(y_static.cpu(), y_engine.cpu()), f"call {k}: static and engine results differ"
        segs = so.seg_bounds(idx.tolist()).tolist()
        assert_close(y_static, bgmv.add_lora(y0, x, wa, wbs, 0.5, segs, offs), f"call {k} vs oracle")
        assert engine.device_errors() == 0


def test_static_rejects_oversize_and_unsupported_rank():
    announce("add_lora_static: limits")
    for T, rank, expect in [(257, 32, _lib.WP_ERR_CAPACITY), (16, 24, _lib.WP_NOT_HANDLED)]:
        idx, x, wa, wbs, offs, y0 = case(T, 4, rank, 256, [256], torch.bfloat16, 7 + T)
        y = y0.cuda()
        assert static_call(y, x.cuda(), idx.cuda(), wa.cuda(), [w.cuda() for w in wbs], offs, 1.0, rank) == expect
        if expect == _lib.WP_ERR_CAPACITY:
            assert "static scratch" in _lib.last_error()
        torch.cuda.synchronize()
        assert torch.equal(y.cpu(), y0), f"a rejected call (T={T}, rank {rank}) wrote y"


def test_static_in_captured_graph_replays():
    """Captured once (after an uncaptured first call), replayed with new
    routings copied into the index buffer: every replay matches the oracle."""
    announce("add_lora_static: graph replays")
    T, L, rank, d, o = 128, 32, 32, 2048, 2048
    idx, x, wa, wbs, offs, y0 = case(T, L, rank, d, [o], torch.bfloat16, 21)
    xd, wad, wbd = x.cuda(), wa.cuda(), [w.cuda() for w in wbs]
    idx_buf = idx.cuda()
    y = y0.cuda()
    assert static_call(y, xd, idx_buf, wad, wbd, offs, 2.0, rank) == _lib.WP_OK
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = static_call(y, xd, idx_buf, wad, wbd, offs, 2.0, rank)
    assert rc == _lib.WP_OK, _lib.last_error()
    g = torch.Generator().manual_seed(5)
    for rep in range(4):
        new_idx = torch.randint(-1, L, (T,), generator=g)
        idx_buf.copy_(new_idx)
        y.copy_(y0.cuda())
        graph.replay()
        torch.cuda.synchronize()
        segs = so.seg_bounds(new_idx.tolist()).tolist()
        assert_close(y, bgmv.add_lora(y0, x, wa, wbs, 2.0, segs, offs), f"replay {rep}")


def read_static_errors(out):
    lib = _lib.load()
    return lib.wp_read_static_errors(torch.cuda.current_device(), ctypes.c_void_p(out.data_ptr()),
                                     ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def test_static_errors_are_readable_and_cleared():
    """An id >= num_loras makes the static call skip its tokens (device error
    1); wp_read_static_errors copies the word into caller memory and clears
    it, so the next read is 0."""
    announce("add_lora_static: error word")
    idx, x, wa, wbs, offs, y0 = case(64, 4, 16, 256, [256], torch.bfloat16, 31)
    idx[7] = 9
    word = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    assert read_static_errors(word) == _lib.WP_OK, _lib.last_error()  # clears what earlier tests left
    y = y0.cuda()
    assert static_call(y, x.cuda(), idx.cuda(), wa.cuda(), [w.cuda() for w in wbs], offs, 1.0, 16) == _lib.WP_OK
    assert read_static_errors(word) == _lib.WP_OK
    torch.cuda.synchronize()
    assert int(word.item()) & 1
    assert read_static_errors(word) == _lib.WP_OK
    torch.cuda.synchronize()
    assert int(word.item()) == 0
    # The rows of valid ids are still applied.
    keep = [s for s in so.seg_bounds(idx.tolist()).tolist() if s[0] < 4]
    assert_close(y, bgmv.add_lora(y0, x, wa, wbs, 1.0, keep, offs), "valid rows")
    assert _lib.load().wp_read_static_errors(0, None, None) == _lib.WP_ERR_INVALID


def test_static_at_capacity_allocates_nothing():
    """T=256 (the static scratch's capacity) against the engine and the
    oracle; after a first call, further calls of any size leave the device's
    free memory and torch's allocator untouched."""
    announce("add_lora_static: T=256 and device memory")
    engine = WarpPipeEngine()
    idx, x, wa, wbs, offs, y0 = case(256, 16, 32, 1024, [1024, 512], torch.float16, 41)
    xd, wad, wbd, idxd = x.cuda(), wa.cuda(), [w.cuda() for w in wbs], idx.cuda()
    y = y0.cuda()
    assert static_call(y, xd, idxd, wad, wbd, offs, 0.75, 32) == _lib.WP_OK
    torch.cuda.synchronize()
    ref = bgmv.add_lora(y0, x, wa, wbs, 0.75, so.seg_bounds(idx.tolist()).tolist(), offs)
    assert_close(y, ref, "T=256")
    ye = y0.cuda()
    assert engine.build_seg_bounds(idxd)
    assert engine.add_lora_slices(ye, xd, wad, wbd, 0.75, offs)
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), ye.cpu())
    sizes = (256, 17, 128)
    ys = [y0[:T].cuda() for T in sizes]
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    alloc0 = torch.cuda.memory_allocated()
    for T, y2 in zip(sizes, ys):
        assert static_call(y2, xd[:T], idxd[:T], wad, wbd, offs, 0.75, 32) == _lib.WP_OK
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0, f"device free memory moved by {free0 - free1} bytes"
    assert torch.cuda.memory_allocated() == alloc0
