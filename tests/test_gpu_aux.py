"""GPU: the library's small pieces around the apply path --
  * lds_barrier(), the LDS-only workgroup barrier of every kernel, through
    wp_barrier_probe (the property the reference tests for its barrier
    wrappers, tests/unit/test_barrier_sync.cu:21-41: every wave's LDS writes
    are visible to every other wave after the barrier), at 4 and 16 wave64
    waves per workgroup, many workgroups per launch;
  * the handoff probe bench.py times for its per-call floor;
  * the device error word polled without a host wait (wp_poll_device_errors);
  * grid bounds of captured adapter-store calls when adapters are registered
    after capture, with and without wp_set_max_adapters."""
import ctypes

import pytest
import torch

from adapterslotsplusplus_amd import WarpPipeEngine, _lib
from oracle import bgmv
from oracle import segments as so
from tests.helpers import announce, assert_close, randn

pytestmark = pytest.mark.gpu


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("threads", [256, 1024])
def test_lds_barrier_makes_every_waves_writes_visible(threads):
    announce(f"barrier probe {threads} threads")
    lib = _lib.load()
    rounds, workgroups = 64, 4096
    salts = torch.randint(0, 2 ** 31 - 1, (rounds,), generator=torch.Generator().manual_seed(threads),
                          dtype=torch.int64).to(torch.int32).cuda()
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    for _ in range(2):
        assert lib.wp_barrier_probe(ctypes.c_void_p(salts.data_ptr()), rounds, threads, workgroups,
                                    ctypes.c_void_p(bad.data_ptr()), _stream()) == _lib.WP_OK, _lib.last_error()
    torch.cuda.synchronize()
    assert int(bad.item()) == 0, f"{int(bad.item())} LDS slots read before their writes were visible"


def test_barrier_probe_rejects_bad_arguments():
    lib = _lib.load()
    salts = torch.zeros(4, dtype=torch.int32, device="cuda")
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    for rounds, threads, wgs in [(0, 256, 1), (4, 512, 1), (4, 256, 0)]:
        assert lib.wp_barrier_probe(ctypes.c_void_p(salts.data_ptr()), rounds, threads, wgs,
                                    ctypes.c_void_p(bad.data_ptr()), _stream()) == _lib.WP_ERR_INVALID


@pytest.mark.parametrize("mode,group", [(0, 8), (1, 8), (2, 8), (3, 64)])
def test_handoff_probe_runs_clean(mode, group):
    """Every wait ends (no give-up), the group counters are left at zero for
    the next launch, and y is written."""
    announce(f"handoff probe mode {mode} group {group}")
    lib = _lib.load()
    a = torch.randint(0, 255, (4 << 20,), dtype=torch.uint8, device="cuda")
    b = torch.randint(0, 255, (8 << 20,), dtype=torch.uint8, device="cuda")
    y = torch.zeros(2 << 20, dtype=torch.uint8, device="cuda")
    workgroups = 256
    counters = torch.zeros(workgroups // group * 2 * 64, dtype=torch.int32, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    for _ in range(3):
        rc = lib.wp_handoff_probe(ctypes.c_void_p(a.data_ptr()), a.numel(), ctypes.c_void_p(b.data_ptr()), b.numel(),
                                  ctypes.c_void_p(y.data_ptr()), y.numel(), ctypes.c_void_p(counters.data_ptr()),
                                  ctypes.c_void_p(err.data_ptr()), group, mode, workgroups, _stream())
        assert rc == _lib.WP_OK, _lib.last_error()
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    assert int(counters.abs().sum().item()) == 0
    assert int(y.ne(0).sum().item()) > 0
    bad = lib.wp_handoff_probe(ctypes.c_void_p(a.data_ptr()), 24, ctypes.c_void_p(b.data_ptr()), 0,
                               ctypes.c_void_p(y.data_ptr()), 0, ctypes.c_void_p(counters.data_ptr()),
                               ctypes.c_void_p(err.data_ptr()), group, mode, workgroups, _stream())
    assert bad == _lib.WP_ERR_INVALID


def register(engine, ids, rank, d, o, dtype, seed):
    adapters = {}
    for aid in ids:
        A = randn((rank, d), seed + 2 * aid, dtype, 0.02)
        B = randn((o, rank), seed + 2 * aid + 1, dtype, 0.02)
        engine.register_adapter(aid, A.cuda(), B.cuda(), 0.5, rank=rank)
        adapters[aid] = (A, B, 0.5)
    return adapters


def test_poll_reports_skipped_tokens_without_a_wait():
    """An unregistered id in a store call (device error 2): a poll moves the
    word to host memory, a later poll (once that move has landed) returns
    the bit; device_errors() then reads a clean word."""
    announce("poll_device_errors")
    dtype = torch.bfloat16
    engine = WarpPipeEngine()
    assert engine.poll_device_errors() == 0
    register(engine, [0, 1], 16, 256, 256, dtype, 300)
    T = 32
    idx = torch.tensor([0] * 12 + [7] * 8 + [1] * 12)
    X = randn((T, 256), 301, dtype).cuda()
    Y = torch.zeros(T, 256, dtype=dtype, device="cuda")
    assert engine.build_seg_bounds(idx.cuda())
    engine.shrink_expand(X, Y, 256, 16)
    seen = 0
    for _ in range(3):
        seen |= engine.poll_device_errors()
        torch.cuda.synchronize()
    assert seen & 2, f"0x{seen:x}"
    torch.cuda.synchronize()
    engine.poll_device_errors()
    assert engine.device_errors() == 0
    # Bits a poll moved but did not return come back through device_errors().
    engine.shrink_expand(X, Y, 256, 16)
    engine.poll_device_errors()
    assert engine.device_errors() & 2


def store_step(engine, X, Y, H):
    engine.shrink(X, X.size(1), 16, X.size(0), out=H)
    engine.expand(H, Y, Y.size(1), 16)


@pytest.mark.parametrize("declare", [False, True])
def test_captured_store_calls_cover_adapters_registered_later(declare):
    """Store calls captured with 2 adapters registered; 30 more registered
    after capture; a replay routed over all 32 matches the oracle with a clean
    error word.  Declared (set_max_adapters(32)), the grid is sized for 32
    and a 33rd registration is refused."""
    announce(f"captured store calls, adapters registered later, declare={declare}")
    dtype = torch.bfloat16
    engine = WarpPipeEngine()
    if declare:
        engine.set_max_adapters(32)
    T, d, o = 256, 512, 384
    adapters = register(engine, [0, 1], 16, d, o, dtype, 400)
    X0 = randn((T, d), 401, dtype)
    Y0 = randn((T, o), 402, dtype)
    X, Y = X0.cuda(), Y0.cuda()
    H = torch.zeros(T, 16, dtype=dtype, device="cuda")
    idx_buf = torch.randint(0, 2, (T,), generator=torch.Generator().manual_seed(3)).cuda()
    assert engine.build_seg_bounds(idx_buf)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        store_step(engine, X, Y, H)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        engine.build_seg_bounds(idx_buf)
        store_step(engine, X, Y, H)
    adapters.update(register(engine, list(range(2, 32)), 16, d, o, dtype, 400))
    torch.cuda.synchronize()
    # Every id 0..31 at least 4 times, in a shuffled order.
    ids = torch.arange(T) % 32
    ids = ids[torch.randperm(T, generator=torch.Generator().manual_seed(4))]
    idx_buf.copy_(ids.cuda())
    Y.copy_(Y0.cuda())
    g.replay()
    torch.cuda.synchronize()
    segs = so.seg_bounds(ids.numpy()).tolist()
    ref = bgmv.expand(bgmv.shrink(X0, segs, adapters, 16, T), Y0, segs, adapters)
    assert_close(Y, ref, "replay over 32 adapters")
    assert engine.device_errors() == 0
    if declare:
        with pytest.raises(RuntimeError, match="declared maximum"):
            register(engine, [40], 16, d, o, dtype, 400)
        with pytest.raises(RuntimeError, match="registered already"):
            engine.set_max_adapters(8)
