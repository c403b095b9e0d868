"""GPU parity of shrink / expand / add_lora against the CPU oracle.

Each test mirrors a reference test (cited) on identical seeded inputs drawn on
the CPU, at the north-star tolerance |dev - ref| <= 1e-3 + 1e-2 |ref|
(bf16 / fp16 I/O, fp32 accumulation)."""
import numpy as np
import pytest
import torch

from adapterslotsplusplus_amd import WarpPipeEngine
from oracle import bgmv
from oracle import segments as so
from tests.helpers import announce, assert_close, h_tie_flips, randn, seeds

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16]


def register(engine, K, rank, d, o, dtype, seed, alpha, ids=None):
    A = randn((K, rank, d), seed, dtype, 0.02)
    B = randn((K, o, rank), seed + 1, dtype, 0.02)
    ids = list(range(K)) if ids is None else ids
    adapters = {}
    for i, aid in enumerate(ids):
        engine.register_adapter(aid, A[i].cuda().contiguous(), B[i].cuda().contiguous(), alpha, rank=rank)
        adapters[aid] = (A[i], B[i], alpha)
    return adapters


def run_host_path(engine, adapters, ids, offsets, X, Y0, d, o, rank):
    engine.build_segments(ids, offsets)
    T = X.shape[0]
    H = engine.shrink(X.cuda(), d, rank, T)
    Y = Y0.cuda().clone()
    engine.expand(H, Y, o, rank)
    torch.cuda.synchronize()
    segs = so.segment_table(ids, offsets).tolist()
    H_ref = bgmv.shrink(X, segs, adapters, rank if rank else 64, T)
    Y_ref = bgmv.expand(H_ref, Y0, segs, adapters)
    return H, Y, H_ref, Y_ref


@pytest.mark.parametrize("dtype", DTYPES)
def test_bgmv_correctness_grid(dtype):
    """tests/correctness/test_bgmv_correctness.py:17-60: K x T grid, r=32, d=o=4096."""
    for K in [1, 2, 4, 8]:
        for T in [1, 4, 8, 16]:
            announce(f"bgmv grid K={K} T={T} {dtype}")
            engine = WarpPipeEngine()
            adapters = register(engine, K, 32, 4096, 4096, dtype, K * 1000 + T, 16.0 / 32)
            X = randn((K * T, 4096), K * 7 + T, dtype, 0.1)
            Y0 = randn((K * T, 4096), K * 11 + T, dtype, 0.1)
            H, Y, H_ref, Y_ref = run_host_path(engine, adapters, list(range(K)), [i * T for i in range(K + 1)],
                                               X, Y0, 4096, 4096, 32)
            assert_close(H, H_ref, f"H K={K} T={T}")
            assert_close(Y, Y_ref, f"Y K={K} T={T}")
            assert engine.device_errors() == 0


@pytest.mark.parametrize("rank", [8, 16, 32, 64])
@pytest.mark.parametrize("dtype", DTYPES)
def test_rank_variants(rank, dtype):
    """tests/unit/test_rank_variants.py:30-95: d=o=512, K=3, 17 tokens each (tails)."""
    announce(f"rank variants r={rank} {dtype}")
    engine = WarpPipeEngine()
    K, n = 3, 17
    adapters = register(engine, K, rank, 512, 512, dtype, 5, 16.0 / rank)
    X = randn((K * n, 512), 6, dtype, 0.1)
    Y0 = randn((K * n, 512), 7, dtype, 0.1)
    H, Y, H_ref, Y_ref = run_host_path(engine, adapters, list(range(K)), [i * n for i in range(K + 1)],
                                       X, Y0, 512, 512, rank)
    assert_close(H, H_ref, "H")
    assert_close(Y, Y_ref, "Y")


@pytest.mark.parametrize("rank", [8, 16, 32, 64])
def test_pipeline_full_size(rank):
    """tests/unit/test_pipeline_output.py:36-82: d=o=4096, K=4 x 32 tokens, per-chunk check."""
    announce(f"pipeline full size r={rank}")
    dtype = torch.float16
    engine = WarpPipeEngine()
    K, n = 4, 32
    adapters = register(engine, K, rank, 4096, 4096, dtype, 100 + rank, 16.0 / rank)
    X = randn((K * n, 4096), 8, dtype, 0.1)
    Y0 = randn((K * n, 4096), 9, dtype, 0.1)
    H, Y, H_ref, Y_ref = run_host_path(engine, adapters, list(range(K)), [i * n for i in range(K + 1)],
                                       X, Y0, 4096, 4096, rank)
    assert_close(H, H_ref, "H")
    for lo in range(0, K * n, 4):
        assert_close(Y[lo:lo + 4], Y_ref[lo:lo + 4], f"Y chunk {lo}")


def test_segment_builder_shapes():
    """tests/unit/test_segment_builder.py:35-75: 1/31/2 tokens; K=256 one token each."""
    announce("segment builder shapes")
    dtype = torch.float16
    engine = WarpPipeEngine()
    adapters = register(engine, 256, 32, 4096, 4096, dtype, 21, 0.5)
    X = randn((34, 4096), 22, dtype, 0.1)
    Y0 = randn((34, 4096), 23, dtype, 0.1)
    H, Y, H_ref, Y_ref = run_host_path(engine, adapters, [0, 1, 2], [0, 1, 32, 34], X, Y0, 4096, 4096, 32)
    assert_close(H, H_ref, "H 1/31/2")
    assert_close(Y, Y_ref, "Y 1/31/2")
    X = randn((256, 4096), 24, dtype, 0.1)
    Y0 = randn((256, 4096), 25, dtype, 0.1)
    H, Y, H_ref, Y_ref = run_host_path(engine, adapters, list(range(256)), list(range(257)), X, Y0, 4096, 4096, 32)
    assert_close(H, H_ref, "H K=256")
    assert_close(Y, Y_ref, "Y K=256")


def test_long_host_segment_is_fully_applied():
    """A 100-token host segment: all tokens are applied (the reference's grid
    drops tokens past 32, Appendix-B defect)."""
    announce("long host segment")
    dtype = torch.bfloat16
    engine = WarpPipeEngine()
    adapters = register(engine, 2, 16, 1024, 768, dtype, 31, 1.0)
    X = randn((140, 1024), 32, dtype)
    Y0 = randn((140, 768), 33, dtype)
    H, Y, H_ref, Y_ref = run_host_path(engine, adapters, [1, 0], [0, 100, 140], X, Y0, 1024, 768, 16)
    assert_close(H, H_ref, "H")
    assert_close(Y, Y_ref, "Y")


ADD_LORA_CASES = [
    [0, 0, 0, 0, -1, -1, 2, 2, 2, 1, 1, 1, 1, 1, 1, 1],   # test_add_lora_packed.py:78
    [3] * 32,                                             # :81
    [-1] * 8,                                             # :84
    [5] * 33,                                             # :93
    list(range(8)) * 4,                                   # :102
    [4] * 8,                                              # :108
    [4] * 9,                                              # :109
]


def add_lora_case(engine, idx_list, rank, dtype, seed, L=8, d=4096, o=4096, scale=16.0 / 32):
    T = len(idx_list)
    wa = randn((L, 1, rank, d), seed, dtype, 0.02)
    wb = randn((L, 1, o, rank), seed + 1, dtype, 0.02)
    x = randn((T, d), seed + 2, dtype, 0.1)
    y0 = randn((T, o), seed + 3, dtype, 0.1)
    idx = torch.tensor(idx_list, dtype=torch.int64)
    y = y0.cuda()
    assert engine.build_seg_bounds(idx.cuda())
    assert engine.add_lora_packed(y, x.cuda(), wa.cuda(), wb.cuda(), scale)
    torch.cuda.synchronize()
    y_ref = bgmv.add_lora(y0, x, wa, wb, scale, so.seg_bounds(idx_list).tolist())
    return y, y_ref


@pytest.mark.parametrize("dtype", DTYPES)
def test_add_lora_packed_cases(dtype):
    """tests/correctness/test_add_lora_packed.py:48-112, all seven index lists."""
    engine = WarpPipeEngine()
    for n, lst in enumerate(ADD_LORA_CASES):
        announce(f"add_lora case {n} {dtype}")
        y, y_ref = add_lora_case(engine, lst, 32, dtype, 40 + n)
        assert_close(y, y_ref, f"case {n}")
    assert engine.device_errors() == 0


@pytest.mark.parametrize("rank", [8, 16, 64])
def test_add_lora_other_ranks(rank):
    """add_lora at the ranks the reference's DSAK path rejects (bindings:197-198)."""
    engine = WarpPipeEngine()
    for n, lst in enumerate(ADD_LORA_CASES[:2] + ADD_LORA_CASES[4:5]):
        announce(f"add_lora r={rank} case {n}")
        y, y_ref = add_lora_case(engine, lst, rank, torch.bfloat16, 60 + n, scale=16.0 / rank)
        assert_close(y, y_ref, f"r={rank} case {n}")


def test_add_lora_unsupported_rank_returns_false():
    engine = WarpPipeEngine()
    idx = torch.zeros(4, dtype=torch.int64, device="cuda")
    assert engine.build_seg_bounds(idx)
    y = torch.zeros(4, 64, dtype=torch.float16, device="cuda")
    x = torch.zeros(4, 64, dtype=torch.float16, device="cuda")
    wa = torch.zeros(1, 1, 24, 64, dtype=torch.float16, device="cuda")
    wb = torch.zeros(1, 1, 64, 24, dtype=torch.float16, device="cuda")
    assert engine.add_lora_packed(y, x, wa, wb, 1.0) is False


def test_segment_reuse_across_layers():
    """test_add_lora_packed.py:116-146: one table, four layers with their own weights."""
    engine = WarpPipeEngine()
    idx_list = [0, 0, 0, -1, 1, 1, 1, 1, 1, 2, 2]
    T = len(idx_list)
    x = randn((T, 4096), 70, torch.float16, 0.1)
    assert engine.build_seg_bounds(torch.tensor(idx_list, device="cuda"))
    segs = so.seg_bounds(idx_list).tolist()
    for layer in range(4):
        announce(f"reuse across layers layer={layer}")
        wa = randn((8, 1, 32, 4096), 71 + layer, torch.float16, 0.02)
        wb = randn((8, 1, 4096, 32), 81 + layer, torch.float16, 0.02)
        y0 = randn((T, 4096), 91 + layer, torch.float16, 0.1)
        y = y0.cuda()
        assert engine.add_lora_packed(y, x.cuda(), wa.cuda(), wb.cuda(), 0.5)
        torch.cuda.synchronize()
        assert_close(y, bgmv.add_lora(y0, x, wa, wb, 0.5, segs), f"layer {layer}")


def test_graph_capture_replay_uses_replay_time_indices():
    """tests/correctness/test_warp_pipe_graph_capture.py:39-129: capture with one
    routing, rebuild the table outside the graph, replay with another; several
    replays with eager work and synchronisation in between, each checked."""
    dtype = torch.float16
    T = 16
    wa = randn((8, 1, 32, 4096), 100, dtype, 0.02)
    wb = randn((8, 1, 4096, 32), 101, dtype, 0.02)
    x = randn((T, 4096), 102, dtype, 0.1)
    y0 = randn((T, 4096), 103, dtype, 0.1)
    cap = [0, 0, 0, 0, 1, 1, 1, 1, -1, -1, 2, 2, 2, 2, 2, 2]
    rep = [3, 3, 5, 5, 5, 5, 5, 5, 5, 5, 5, 5, 5, 5, -1, 6]
    engine = WarpPipeEngine()
    wa_d, wb_d, x_d, y0_d = wa.cuda(), wb.cuda(), x.cuda(), y0.cuda()
    idx_buf = torch.zeros(T, dtype=torch.int64, device="cuda")
    y_buf = torch.zeros(T, 4096, dtype=dtype, device="cuda")
    idx_buf.copy_(torch.tensor(cap))
    assert engine.build_seg_bounds(idx_buf)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            y_buf.copy_(y0_d)
            engine.add_lora_packed(y_buf, x_d, wa_d, wb_d, 0.5)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    y_buf.copy_(y0_d)
    announce("graph capture")
    with torch.cuda.graph(g):
        assert engine.add_lora_packed(y_buf, x_d, wa_d, wb_d, 0.5)
    torch.cuda.synchronize()
    ref_cap = bgmv.add_lora(y0, x, wa, wb, 0.5, so.seg_bounds(cap).tolist())
    ref_rep = bgmv.add_lora(y0, x, wa, wb, 0.5, so.seg_bounds(rep).tolist())
    for it, (lst, ref) in enumerate([(cap, ref_cap), (rep, ref_rep), (cap, ref_cap), (rep, ref_rep)]):
        announce(f"graph replay {it}")
        idx_buf.copy_(torch.tensor(lst))
        assert engine.build_seg_bounds(idx_buf)
        y_buf.copy_(y0_d)
        _ = (x_d.float() * 2).sum()  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert_close(y_buf, ref, f"replay {it}")
    # Negative control: the replay-routing result differs from the capture-routing one.
    assert not torch.allclose(ref_rep.float(), ref_cap.float(), rtol=1e-2, atol=1e-3)


def test_seg_bounds_with_registered_adapters():
    """build_seg_bounds + shrink/expand through the adapter store (the reference
    reads stale descriptor pointers on this pairing)."""
    announce("seg_bounds + store shrink/expand")
    dtype = torch.bfloat16
    engine = WarpPipeEngine()
    adapters = register(engine, 6, 32, 2048, 1536, dtype, 110, 0.25, ids=[3, 7, 11, 2, 5, 0])
    rng = np.random.default_rng(3)
    idx = rng.choice([3, 7, 11, 2, 5, 0, -1], size=200)
    X = randn((200, 2048), 111, dtype)
    Y0 = randn((200, 1536), 112, dtype)
    assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
    H = engine.shrink(X.cuda(), 2048, 32, 200)
    Y = Y0.cuda()
    engine.expand(H, Y, 1536, 32)
    torch.cuda.synchronize()
    segs = so.seg_bounds(idx).tolist()
    H_ref = bgmv.shrink(X, segs, adapters, 32, 200)
    assert_close(H, H_ref, "H")
    assert_close(Y, bgmv.expand(H_ref, Y0, segs, adapters), "Y")
    assert engine.device_errors() == 0


@pytest.mark.parametrize("d,rank", [(1032, 16), (1032, 64), (20480, 32), (20480, 0)])
def test_shrink_unaligned_and_wide_d(d, rank):
    """shrink()/expand() with d not a multiple of the 128-column slice (the
    last slice is clamped and zeroed) and d past 16 d-ranges of 1024 columns
    (each workgroup streams several 1024-column groups); rank 0 = mixed."""
    announce(f"shrink d={d} rank={rank}")
    dtype = torch.bfloat16
    engine = WarpPipeEngine()
    ranks = [rank] * 5 if rank else [8, 16, 32, 64, 32]
    adapters = {}
    for i, r in enumerate(ranks):
        A = randn((r, d), 300 + i, dtype, 0.02)
        B = randn((640, r), 310 + i, dtype, 0.02)
        engine.register_adapter(i, A.cuda(), B.cuda(), 16.0 / r, rank=r)
        adapters[i] = (A, B, 16.0 / r)
    rng = np.random.default_rng(d + rank)
    idx = rng.integers(-1, 5, size=150)
    X = randn((150, d), 320, dtype)
    Y0 = randn((150, 640), 321, dtype)
    assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
    H = engine.shrink(X.cuda(), d, rank, 150)
    Y = Y0.cuda()
    engine.expand(H, Y, 640, rank)
    torch.cuda.synchronize()
    segs = so.seg_bounds(idx).tolist()
    H_ref = bgmv.shrink(X, segs, adapters, rank if rank else 64, 150)
    assert_close(H, H_ref, "H")
    assert_close(Y, bgmv.expand(H_ref, Y0, segs, adapters), "Y")
    assert engine.device_errors() == 0


@pytest.mark.parametrize("T", [40, 700])
def test_add_lora_unaligned_d(T):
    """add_lora with d = 1032 on a decode-sized (fused) and a large plan."""
    announce(f"add_lora d=1032 T={T}")
    engine = WarpPipeEngine()
    rng = np.random.default_rng(T)
    idx = rng.integers(-1, 6, size=T).tolist()
    y, y_ref = add_lora_case(engine, idx, 32, torch.float16, 330, L=6, d=1032, o=1032)
    assert_close(y, y_ref, f"T={T}")
    assert engine.device_errors() == 0


def test_mixed_rank_store():
    """Mixed ranks in one grouped call (configuration 3's shape, reduced)."""
    announce("mixed rank")
    dtype = torch.bfloat16
    engine = WarpPipeEngine()
    ranks = [8, 16, 32, 64] * 3
    adapters = {}
    for i, r in enumerate(ranks):
        A = randn((r, 1280), 120 + i, dtype, 0.02)
        B = randn((2048, r), 140 + i, dtype, 0.02)
        engine.register_adapter(i, A.cuda(), B.cuda(), 16.0 / r, rank=r)
        adapters[i] = (A, B, 16.0 / r)
    rng = np.random.default_rng(5)
    idx = rng.integers(-1, 12, size=300)
    X = randn((300, 1280), 160, dtype)
    Y0 = randn((300, 2048), 161, dtype)
    assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
    H = engine.shrink(X.cuda(), 1280, 0, 300)
    Y = Y0.cuda()
    engine.expand(H, Y, 2048, 0)
    torch.cuda.synchronize()
    segs = so.seg_bounds(idx).tolist()
    H_ref = bgmv.shrink(X, segs, adapters, 64, 300)
    assert_close(H, H_ref, "H")
    assert_close(Y, bgmv.expand(H_ref, Y0, segs, adapters), "Y")
    assert engine.device_errors() == 0


def test_plan_entry_copies_follow_table_writes():
    """A build_seg_bounds plan copies each block's adapter-table entry for the
    mixed-rank store kernels; a table write after the build (an adapter
    evicted and registered again with other weights, another evicted) must
    make the calls read the table itself until the next build.  shrink +
    expand and shrink_expand against the oracle at every stage."""
    announce("plan entry copies vs table writes")
    dtype = torch.bfloat16
    T, d, o = 200, 1024, 1536
    ranks = [8, 16, 32, 64, 32, 16]
    engine = WarpPipeEngine()
    adapters = {}

    def register(i, seed):
        r = ranks[i]
        A = randn((r, d), seed, dtype, 0.02)
        B = randn((o, r), seed + 1, dtype, 0.02)
        engine.register_adapter(i, A.cuda(), B.cuda(), 8.0 / r, rank=r)
        adapters[i] = (A, B, 8.0 / r)

    for i in range(len(ranks)):
        register(i, 500 + 10 * i)
    idx = np.random.default_rng(11).integers(-1, len(ranks), size=T)
    X = randn((T, d), 600, dtype)
    Y0 = randn((T, o), 601, dtype)
    segs = so.seg_bounds(idx).tolist()

    def check(stage, errors_expected=False):
        H = engine.shrink(X.cuda(), d, 0, T)
        Y = Y0.cuda()
        engine.expand(H, Y, o, 0)
        Y1 = Y0.cuda()
        engine.shrink_expand(X.cuda(), Y1, o, 0)
        torch.cuda.synchronize()
        live = [sg for sg in segs if int(sg[0]) in adapters]  # an evicted id's tokens are left alone
        H_ref = bgmv.shrink(X, live, adapters, 64, T)
        Y_ref = bgmv.expand(H_ref, Y0, live, adapters)
        assert_close(H, H_ref, f"{stage}: H")
        assert_close(Y, Y_ref, f"{stage}: Y")
        assert_close(Y1, Y_ref, f"{stage}: Y, shrink_expand")
        assert (engine.device_errors() != 0) == errors_expected, stage

    assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
    check("as built")
    # New weights under id 3, after the build.
    engine.evict_adapter(3)
    register(3, 700)
    check("id 3 replaced after the build")
    # Id 1 gone: its tokens are skipped (and flagged), the others applied.
    engine.evict_adapter(1)
    del adapters[1]
    check("id 1 evicted after the build", errors_expected=True)
    # The next build copies the current table.
    assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
    check("rebuilt", errors_expected=True)


@pytest.mark.parametrize("dtype", DTYPES)
def test_packed_slices_and_offsets(dtype):
    """One shared H expanded into q/k/v slices of a wider y, and a single
    y_offset slice (the reference hook falls back for these)."""
    announce(f"slices {dtype}")
    engine = WarpPipeEngine()
    T, d, L, r = 96, 1024, 6, 32
    rng = np.random.default_rng(7)
    idx = rng.integers(-1, L, size=T)
    wa = randn((L, 1, r, d), 170, dtype, 0.02)
    wbs = [randn((L, 1, o, r), 171 + i, dtype, 0.02) for i, o in enumerate([1024, 256, 256])]
    x = randn((T, d), 175, dtype)
    y0 = randn((T, 1536 + 8), 176, dtype)
    offs = [0, 1024, 1280]
    assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
    y = y0.cuda()
    assert engine.add_lora_slices(y, x.cuda(), wa.cuda(), [w.cuda() for w in wbs], 0.5, offs)
    torch.cuda.synchronize()
    segs = so.seg_bounds(idx).tolist()
    assert_close(y, bgmv.add_lora(y0, x, wa, wbs, 0.5, segs, offs), "q/k/v slices")
    y = y0.cuda()
    assert engine.add_lora_packed(y, x.cuda(), wa.cuda(), wbs[1].cuda(), 0.5, y_offset=1288, y_slice_size=256)
    torch.cuda.synchronize()
    assert_close(y, bgmv.add_lora(y0, x, wa, [wbs[1]], 0.5, segs, [1288]), "y_offset slice")


def test_out_of_range_ids_are_skipped_and_flagged():
    """Ids >= L are not read (the reference indexes past wa_t_all, Appendix B
    item 4): those rows stay untouched and the device error word says so."""
    announce("out of range ids")
    dtype = torch.float16
    engine = WarpPipeEngine()
    idx_list = [0, 0, 9, 9, 1, -1, 12, 1]
    assert engine.device_errors() == 0
    T = len(idx_list)
    wa = randn((4, 1, 32, 512), 191, dtype, 0.02)
    wb = randn((4, 1, 512, 32), 192, dtype, 0.02)
    x = randn((T, 512), 193, dtype)
    y0 = randn((T, 512), 194, dtype)
    assert engine.build_seg_bounds(torch.tensor(idx_list, device="cuda"))
    y = y0.cuda()
    assert engine.add_lora_packed(y, x.cuda(), wa.cuda(), wb.cuda(), 1.0)
    torch.cuda.synchronize()
    segs = [s for s in so.seg_bounds(idx_list).tolist() if s[0] < 4]
    assert_close(y, bgmv.add_lora(y0, x, wa, wb, 1.0, segs), "valid rows")
    assert engine.device_errors() & 1


def test_store_calls_flag_routing_past_the_block_bound():
    """shrink()/expand() on a build_seg_bounds plan size their grid for the
    registered adapters (T/16 + 2 blocks here).  A routing that names 48
    unregistered ids has more blocks than that: the call skips what it does
    not cover and says so (unregistered 2, capacity 16); registered-only
    routing of the same length is complete."""
    announce("block bound of store calls")
    dtype = torch.bfloat16
    engine = WarpPipeEngine()
    adapters = register(engine, 2, 16, 512, 256, dtype, 290, 0.5, ids=[50, 51])
    T = 64
    X = randn((T, 512), 291, dtype)
    idx = np.concatenate([np.arange(48), np.full(8, 50), np.full(8, 51)])
    assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
    engine.shrink(X.cuda(), 512, 16, T)
    torch.cuda.synchronize()
    err = engine.device_errors()
    assert err & 16 and err & 2
    idx = np.random.default_rng(4).choice([50, 51], size=T)
    assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
    H = engine.shrink(X.cuda(), 512, 16, T)
    torch.cuda.synchronize()
    assert_close(H, bgmv.shrink(X, so.seg_bounds(idx).tolist(), adapters, 16, T), "H")
    assert engine.device_errors() == 0


def test_plan_token_count_must_fit_call():
    engine = WarpPipeEngine()
    assert engine.build_seg_bounds(torch.zeros(32, dtype=torch.int64, device="cuda"))
    x = torch.zeros(16, 256, dtype=torch.float16, device="cuda")
    y = torch.zeros(16, 256, dtype=torch.float16, device="cuda")
    wa = torch.zeros(1, 1, 32, 256, dtype=torch.float16, device="cuda")
    wb = torch.zeros(1, 1, 256, 32, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="segments reach token"):
        engine.add_lora_packed(y, x, wa, wb, 1.0)


@pytest.mark.parametrize("T,rank", [(513, 16), (1000, 64), (2049, 32)])
def test_add_lora_large_plans(T, rank):
    """Plans over more than 512 tokens (64-token blocks, shrink + expand
    launches with several token tiles in flight): random routings with ids < 0
    and ragged blocks, three output slices with offsets."""
    announce(f"large plan T={T} r={rank}")
    dtype = torch.bfloat16
    engine = WarpPipeEngine()
    L, d = 9, 1024
    rng = np.random.default_rng(T)
    idx = np.repeat(rng.integers(-1, L, size=T // 3 + 1), 3)[:T]
    rng.shuffle(idx[: T // 2])
    wa = randn((L, 1, rank, d), 200, dtype, 0.02)
    wbs = [randn((L, 1, o, rank), 201 + i, dtype, 0.02) for i, o in enumerate([1024, 512, 512])]
    x = randn((T, d), 205, dtype)
    y0 = randn((T, 2048), 206, dtype)
    offs = [0, 1024, 1536]
    assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
    y = y0.cuda()
    assert engine.add_lora_slices(y, x.cuda(), wa.cuda(), [w.cuda() for w in wbs], 16.0 / rank, offs)
    torch.cuda.synchronize()
    segs = so.seg_bounds(idx).tolist()
    assert_close(y, bgmv.add_lora(y0, x, wa, wbs, 16.0 / rank, segs, offs), f"T={T} r={rank}")
    assert engine.device_errors() == 0


def test_registered_adapters_large_plan():
    """shrink / expand through the adapter store on a 64-token-block plan."""
    announce("store shrink/expand T=1500")
    dtype = torch.float16
    engine = WarpPipeEngine()
    adapters = register(engine, 5, 64, 1536, 1024, dtype, 210, 0.25, ids=[4, 1, 9, 6, 2])
    rng = np.random.default_rng(11)
    idx = np.sort(rng.choice([4, 1, 9, 6, 2, -1], size=1500))
    X = randn((1500, 1536), 211, dtype)
    Y0 = randn((1500, 1024), 212, dtype)
    assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
    H = engine.shrink(X.cuda(), 1536, 64, 1500)
    Y = Y0.cuda()
    engine.expand(H, Y, 1024, 64)
    torch.cuda.synchronize()
    segs = so.seg_bounds(idx).tolist()
    H_ref = bgmv.shrink(X, segs, adapters, 64, 1500)
    assert_close(H, H_ref, "H")
    assert_close(Y, bgmv.expand(H_ref, Y0, segs, adapters), "Y")
    assert engine.device_errors() == 0


@pytest.mark.parametrize("case", ["rank32_device_plan", "rank16_host_plan_window", "mixed", "mixed_wide", "large_plan"])
def test_shrink_expand_matches_oracle(case):
    """shrink_expand(): one launch for decode-sized single-rank plans, shrink +
    expand through the engine's H otherwise; each against the oracle."""
    announce(f"shrink_expand {case}")
    dtype = torch.bfloat16
    engine = WarpPipeEngine()
    # mixed_wide: 19 output chunks of 256 (the last one 12 columns), more
    # than one chunk per expand workgroup.
    d, o = 2048, (4620 if case == "mixed_wide" else 1536)
    if case in ("mixed", "mixed_wide"):
        rng = np.random.default_rng(8)
        ranks = [8, 16, 32, 64, 16, 32]
        ids = [4, 9, 1, 7, 3, 12]
        adapters = {}
        for i, (aid, r) in enumerate(zip(ids, ranks)):
            A = randn((r, d), 300 + i, dtype, 0.02)
            B = randn((o, r), 310 + i, dtype, 0.02)
            engine.register_adapter(aid, A.cuda(), B.cuda(), 16.0 / r, rank=r)
            adapters[aid] = (A, B, 16.0 / r)
        rank = 0
    else:
        rank = 16 if case == "rank16_host_plan_window" else 32
        ids = [4, 9, 1, 7, 3, 12]
        adapters = register(engine, 6, rank, d, o, dtype, 320, 0.5, ids=ids)
    T = 700 if case == "large_plan" else 200
    X = randn((T, d), 330, dtype)
    width, off = (o + 256, 128) if case == "rank16_host_plan_window" else (o, 0)
    Y0 = randn((T, width), 331, dtype)
    if case == "rank16_host_plan_window":
        sorted_ids = [1, 3, 4, 7, 9, 12]
        offsets = [0, 30, 55, 90, 140, 170, 200]
        engine.build_segments(sorted_ids, offsets)
        segs = so.segment_table(sorted_ids, offsets).tolist()
    else:
        idx = np.random.default_rng(T).choice(ids + [-1], size=T)
        assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
        segs = so.seg_bounds(idx).tolist()
    Y = Y0.cuda()
    engine.shrink_expand(X.cuda(), Y, o, rank, y_offset=off)
    torch.cuda.synchronize()
    H_ref = bgmv.shrink(X, segs, adapters, rank if rank else 64, T)
    ref = Y0.clone()
    ref[:, off:off + o] = bgmv.expand(H_ref, Y0[:, off:off + o].contiguous(), segs, adapters)
    assert_close(Y, ref, "Y")
    assert engine.device_errors() == 0


def _random_case(seed):
    """Seeded add_lora shape: T across the 512-token switch between the
    one-launch and the two-launch paths, 1-3 slices (one of them wider than
    4096 columns in some cases), every rank, column offsets, runs of -1."""
    rng = np.random.default_rng(1000 + seed)
    T = int(rng.choice([1, 3, 16, 17, 100, 255, 256, 300, 511, 512, 513, 640]))
    d = int(rng.choice([64, 520, 1024, 2056, 4096]))
    rank = int(rng.choice([8, 16, 32, 64]))
    L = int(rng.choice([1, 2, 7, 33]))
    n_sl = int(rng.integers(1, 4))
    if seed % 5 == 0:
        widths = [4620]
    else:
        widths = [int(rng.integers(1, 1025)) * 4 for _ in range(n_sl)]
    offs, col = [], int(rng.integers(0, 3)) * 4
    for w in widths:
        offs.append(col)
        col += w + int(rng.integers(0, 3)) * 4
    # Runs of equal ids (decode batches group by request), some -1.
    idx = np.repeat(rng.integers(-1, L, size=T), rng.integers(1, 6, size=T))[:T]
    dtype = DTYPES[seed % 2]
    scale = float(rng.uniform(0.25, 2.0))
    return T, d, rank, L, widths, offs, col, idx, dtype, scale


@pytest.mark.parametrize("seed", seeds(16))
def test_add_lora_random_shapes(seed):
    T, d, rank, L, widths, offs, width, idx, dtype, scale = _random_case(seed)
    announce(f"random add_lora seed {seed}: T={T} d={d} r={rank} L={L} slices={widths} offs={offs} {dtype}")
    engine = WarpPipeEngine()
    wa = randn((L, 1, rank, d), 2000 + seed, dtype, 0.02)
    wbs = [randn((L, 1, o, rank), 2100 + 7 * seed + i, dtype, 0.02) for i, o in enumerate(widths)]
    x = randn((T, d), 2200 + seed, dtype)
    y0 = randn((T, width), 2300 + seed, dtype)
    assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
    y = y0.cuda()
    if len(widths) == 1:
        assert engine.add_lora_packed(y, x.cuda(), wa.cuda(), wbs[0].cuda(), scale, y_offset=offs[0],
                                      y_slice_size=widths[0])
    else:
        assert engine.add_lora_slices(y, x.cuda(), wa.cuda(), [w.cuda() for w in wbs], scale, offs)
    torch.cuda.synchronize()
    segs = so.seg_bounds(idx).tolist()
    # H is rounded to the I/O type before the expand; where an element's exact
    # value ties with a rounding midpoint within fp32 summation error, either
    # neighbour is a correct H, and the output may move by that step times |B|.
    slack = torch.zeros(y0.shape, dtype=torch.float32)
    for lid in np.unique(idx[(idx >= 0) & (idx < L)]):
        rows = torch.from_numpy(np.nonzero(idx == lid)[0])
        flips = h_tie_flips(x[rows], wa[lid, 0], scale, dtype)
        for wb, off in zip(wbs, offs):
            slack[rows, off:off + wb.shape[2]] += (flips @ wb[lid, 0].double().abs().T).float()
    assert_close(y, bgmv.add_lora(y0, x, wa, wbs, scale, segs, offs), f"seed {seed}", slack=slack)
    assert engine.device_errors() == 0


@pytest.mark.parametrize("seed", seeds(8))
def test_store_random_shapes(seed):
    """Seeded adapter-store calls: registered adapters of random ranks (mixed,
    rank=0, on device-built plans; one rank on host-built plans), random ids,
    T across the 512-token switch; shrink + expand and shrink_expand against
    the oracle."""
    rng = np.random.default_rng(3000 + seed)
    dtype = DTYPES[seed % 2]
    host_plan = seed % 3 == 0
    T = int(rng.choice([1, 40, 200, 512, 513, 700]))
    d = int(rng.choice([64, 1032, 2048]))
    o = int(rng.integers(1, 1300)) * 4
    K = int(rng.integers(1, 12))
    ids = sorted(int(v) for v in rng.choice(200, size=K, replace=False))
    one_rank = int(rng.choice([8, 16, 32, 64]))
    ranks = [one_rank] * K if host_plan else [int(rng.choice([8, 16, 32, 64])) for _ in ids]
    announce(f"random store seed {seed}: T={T} d={d} o={o} K={K} ranks={ranks} host_plan={host_plan} {dtype}")
    engine = WarpPipeEngine()
    adapters = {}
    for i, (aid, r) in enumerate(zip(ids, ranks)):
        A = randn((r, d), 3100 + 10 * seed + i, dtype, 0.02)
        B = randn((o, r), 3200 + 10 * seed + i, dtype, 0.02)
        alpha = float(rng.uniform(0.25, 2.0))
        engine.register_adapter(aid, A.cuda(), B.cuda(), alpha, rank=r)
        adapters[aid] = (A, B, alpha)
    if host_plan:
        cuts = np.sort(rng.choice(np.arange(1, T), size=min(K - 1, T - 1), replace=False)) if T > 1 else []
        offsets = [0] + [int(c) for c in cuts] + [T]
        sorted_ids = ids[: len(offsets) - 1]
        engine.build_segments(sorted_ids, offsets)
        segs = so.segment_table(sorted_ids, offsets).tolist()
        rank = one_rank
    else:
        idx = np.repeat(rng.choice(ids + [-1], size=T), rng.integers(1, 9, size=T))[:T]
        assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
        segs = so.seg_bounds(idx).tolist()
        rank = 0
    X = randn((T, d), 3300 + seed, dtype)
    Y0 = randn((T, o), 3400 + seed, dtype)
    H = engine.shrink(X.cuda(), d, rank, T)
    Y = Y0.cuda()
    engine.expand(H, Y, o, rank)
    Y1 = Y0.cuda()
    engine.shrink_expand(X.cuda(), Y1, o, rank)
    torch.cuda.synchronize()
    H_ref = bgmv.shrink(X, segs, adapters, rank if rank else 64, T)
    Y_ref = bgmv.expand(H_ref, Y0, segs, adapters)
    # Rounding ties of H (see test_add_lora_random_shapes): per segment, the
    # steps its H elements may take either way, times |B|.
    slack = torch.zeros(Y0.shape, dtype=torch.float32)
    for aid, start, count in ((g[0], g[1], g[2]) for g in segs):
        if aid in adapters:
            A, B, alpha = adapters[aid]
            flips = h_tie_flips(X[start:start + count], A, alpha, dtype)
            slack[start:start + count] += (flips @ B.double().abs().T).float()
    assert_close(H, H_ref, f"seed {seed} H")
    assert_close(Y, Y_ref, f"seed {seed} Y", slack=slack)
    assert_close(Y1, Y_ref, f"seed {seed} Y, shrink_expand", slack=slack)
    assert engine.device_errors() == 0


def test_shrink_expand_graph_replays_with_new_routing():
    """The adapter-store path in a captured step: build_seg_bounds and a
    mixed-rank shrink_expand captured once, replayed with other routings
    copied into the captured index tensor; eager work and synchronisation
    between the replays, every replay against the oracle."""
    dtype = torch.bfloat16
    T, d, o = 48, 1024, 768
    engine = WarpPipeEngine()
    ids, ranks = [3, 8, 5, 11], [16, 32, 64, 8]
    adapters = {}
    for i, (aid, r) in enumerate(zip(ids, ranks)):
        A = randn((r, d), 400 + i, dtype, 0.02)
        B = randn((o, r), 410 + i, dtype, 0.02)
        engine.register_adapter(aid, A.cuda(), B.cuda(), 16.0 / r, rank=r)
        adapters[aid] = (A, B, 16.0 / r)
    X = randn((T, d), 420, dtype)
    Y0 = randn((T, o), 421, dtype)
    rng = np.random.default_rng(42)
    routings = [rng.choice(ids + [-1], size=T) for _ in range(3)]
    x_d, y0_d = X.cuda(), Y0.cuda()
    idx_buf = torch.from_numpy(routings[0]).cuda()
    y_buf = y0_d.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            assert engine.build_seg_bounds(idx_buf)
            y_buf.copy_(y0_d)
            engine.shrink_expand(x_d, y_buf, o, 0)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    announce("shrink_expand graph capture")
    with torch.cuda.graph(g):
        engine.build_seg_bounds(idx_buf)
        engine.shrink_expand(x_d, y_buf, o, 0)
    torch.cuda.synchronize()
    refs = []
    for idx in routings:
        segs = so.seg_bounds(idx).tolist()
        refs.append(bgmv.expand(bgmv.shrink(X, segs, adapters, 64, T), Y0, segs, adapters))
    for it, k in enumerate([1, 2, 0, 1]):
        announce(f"shrink_expand graph replay {it}")
        idx_buf.copy_(torch.from_numpy(routings[k]))
        y_buf.copy_(y0_d)
        _ = (x_d.float() * 2).sum()  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert_close(y_buf, refs[k], f"replay {it} (routing {k})")
    assert engine.device_errors() == 0
    assert not torch.allclose(refs[1].float(), refs[2].float(), rtol=1e-2, atol=1e-3)


def test_shrink_expand_shape_errors():
    """A call whose out_features do not match the registered adapters: raised
    on a host-built table (checked when enqueued); on a device-built plan the
    blocks are skipped, Y is left as it was and the shape bit (4) is set."""
    dtype = torch.float16
    engine = WarpPipeEngine()
    register(engine, 2, 16, 256, 512, dtype, 500, 1.0, ids=[1, 2])
    X = randn((32, 256), 501, dtype).cuda()
    Y = randn((32, 256), 502, dtype).cuda()
    engine.build_segments([1, 2], [0, 10, 32])
    with pytest.raises(RuntimeError, match="shrink_expand"):
        engine.shrink_expand(X, Y, 256, 16)
    assert engine.build_seg_bounds(torch.tensor([1] * 16 + [2] * 16).cuda())
    before = Y.clone()
    engine.shrink_expand(X, Y, 256, 16)
    torch.cuda.synchronize()
    assert torch.equal(Y, before)
    assert engine.device_errors() & 4
    with pytest.raises(RuntimeError, match="2-D"):
        engine.shrink_expand(X.view(2, 16, 256), Y, 256, 16)
