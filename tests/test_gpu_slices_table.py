"""GPU: shrink_expand_slices -- several layers of the multi-layer adapter store
(WarpPipeConfig.layer_stride) applied in one launch, each layer's adapter of
a token's id into its own columns of Y (a packed gate/up projection, for
instance).  Reference: per slice, the oracle's shrink then expand over that
layer's adapters alone (oracle.bgmv.shrink / expand), on the same seeded
inputs."""
import numpy as np
import pytest
import torch

from adapterslotsplusplus_amd import WarpPipeConfig, WarpPipeEngine
from adapterslotsplusplus_amd import workloads as wl
from oracle import bgmv
from oracle import segments as so
from tests.helpers import announce, assert_close, randn

pytestmark = pytest.mark.gpu

STRIDE = 256


def register(engine, layer, ids, ranks, d, o, dtype, seed):
    """Registers adapter i of `ids` at rank ranks[i] under `layer`; returns the
    oracle's {id: (A, B, alpha)}."""
    adapters = {}
    for k, aid in enumerate(ids):
        r = ranks[k]
        A = randn((r, d), seed + 3 * k, dtype, 0.02)
        B = randn((o, r), seed + 3 * k + 1, dtype, 0.02)
        alpha = 16.0 / r
        engine.register_adapter(aid, A.cuda(), B.cuda(), alpha, rank=r, layer=layer)
        adapters[aid] = (A, B, alpha)
    return adapters


def reference(X, Y0, segs, per_slice, widths, offs, rank, T):
    """Per slice, shrink then expand over the segments whose id that slice's
    layer holds (tokens of other ids are left as they are)."""
    Y = Y0.clone()
    for ad, o, off in zip(per_slice, widths, offs):
        ss = [sg for sg in segs if sg[0] in ad]
        H = bgmv.shrink(X, ss, ad, rank, T)
        Y = bgmv.expand(H, Y, ss, ad, off)
    return Y


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rank_mode", ["fixed", "mixed"])
def test_gate_up_one_launch(dtype, rank_mode):
    """Two layers (gate, up) of 128-adapter stores, Zipf decode routing: one
    launch against two oracle shrink/expand passes."""
    T, L, d, o = 256, 64, 2048, 2816
    announce(f"slices gate/up {rank_mode} {dtype}")
    engine = WarpPipeEngine(WarpPipeConfig(layer_stride=STRIDE))
    g = torch.Generator().manual_seed(4)
    if rank_mode == "fixed":
        ranks = [[16] * L, [16] * L]
        call_rank = 16
    else:
        ranks = [[int(v) for v in torch.tensor([8, 16, 32, 64])[torch.randint(0, 4, (L,), generator=g)]]
                 for _ in range(2)]
        call_rank = 0
    per_slice = [register(engine, lay, range(L), ranks[lay], d, o, dtype, 100 + 50 * lay) for lay in range(2)]
    idx = wl.zipf_indices(T, L, 1.1, 3)
    X = randn((T, d), 7, dtype)
    Y0 = randn((T, 2 * o), 8, dtype)
    assert engine.build_seg_bounds(idx.cuda())
    Y = Y0.cuda()
    engine.shrink_expand_slices(X.cuda(), Y, [0, 1], [o, o], [0, o], rank=call_rank)
    torch.cuda.synchronize()
    segs = so.seg_bounds(idx.tolist()).tolist()
    ref = reference(X, Y0, segs, per_slice, [o, o], [0, o], 64 if call_rank == 0 else call_rank, T)
    assert_close(Y, ref, "gate/up")
    assert engine.device_errors() == 0


def test_three_layers_ragged_windows_mixed_ranks():
    """Three slices of different widths at gapped offsets, each layer with its
    own ranks per adapter; the columns between windows stay untouched."""
    T, L, d = 93, 9, 1032
    widths, offs = [516, 132, 260], [4, 524, 660]
    dtype = torch.bfloat16
    announce("slices ragged three layers")
    engine = WarpPipeEngine(WarpPipeConfig(layer_stride=STRIDE))
    rng = np.random.default_rng(11)
    per_slice = []
    for s, lay in enumerate([5, 2, 7]):
        ranks = [int(v) for v in rng.choice([8, 16, 32, 64], size=L)]
        per_slice.append(register(engine, lay, range(L), ranks, d, widths[s], dtype, 300 + 40 * s))
    idx = rng.integers(-1, L, size=T)
    X = randn((T, d), 12, dtype)
    Y0 = randn((T, 940), 13, dtype)
    assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
    Y = Y0.cuda()
    engine.shrink_expand_slices(X.cuda(), Y, [5, 2, 7], widths, offs)
    torch.cuda.synchronize()
    segs = so.seg_bounds(idx).tolist()
    assert_close(Y, reference(X, Y0, segs, per_slice, widths, offs, 64, T), "ragged")
    assert engine.device_errors() == 0


@pytest.mark.parametrize("rank", [8, 16, 32, 64])
def test_fixed_ranks_four_layers(rank):
    T, L, d, o = 64, 4, 512, 256
    dtype = torch.float16
    announce(f"slices four layers r={rank}")
    engine = WarpPipeEngine(WarpPipeConfig(layer_stride=STRIDE))
    per_slice = [register(engine, lay, range(L), [rank] * L, d, o, dtype, 500 + 30 * lay) for lay in range(4)]
    idx = np.random.default_rng(rank).integers(0, L, size=T)
    X = randn((T, d), 14, dtype)
    Y0 = randn((T, 4 * o), 15, dtype)
    assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
    Y = Y0.cuda()
    offs = [3 * o, 0, 2 * o, o]  # slice order need not follow column order
    engine.shrink_expand_slices(X.cuda(), Y, [0, 1, 2, 3], [o] * 4, offs, rank=rank)
    torch.cuda.synchronize()
    segs = so.seg_bounds(idx).tolist()
    assert_close(Y, reference(X, Y0, segs, per_slice, [o] * 4, offs, rank, T), f"r={rank}")
    assert engine.device_errors() == 0


def test_four_layers_mixed_ranks_wide_d():
    """Four zero-padded 64-column slices over d = 4096 (the d-range count is
    capped so the partial rows fit the partial buffer)."""
    T, L, d, o = 256, 16, 4096, 768
    dtype = torch.bfloat16
    announce("slices four layers mixed d=4096")
    engine = WarpPipeEngine(WarpPipeConfig(layer_stride=STRIDE))
    rng = np.random.default_rng(40)
    per_slice = [register(engine, lay, range(L), [int(v) for v in rng.choice([8, 16, 32, 64], size=L)], d, o, dtype,
                          1200 + 60 * lay) for lay in range(4)]
    idx = wl.zipf_indices(T, L, 1.1, 5)
    X = randn((T, d), 22, dtype)
    Y0 = randn((T, 4 * o), 23, dtype)
    assert engine.build_seg_bounds(idx.cuda())
    Y = Y0.cuda()
    offs = [k * o for k in range(4)]
    engine.shrink_expand_slices(X.cuda(), Y, [0, 1, 2, 3], [o] * 4, offs)
    torch.cuda.synchronize()
    segs = so.seg_bounds(idx.tolist()).tolist()
    assert_close(Y, reference(X, Y0, segs, per_slice, [o] * 4, offs, 64, T), "4 layers d=4096")
    assert engine.device_errors() == 0


@pytest.mark.parametrize("o,layers", [(256, [0, 1]), (2560, [1, 0])])
def test_adapter_missing_in_one_layer_is_skipped_and_flagged(o, layers):
    """An id registered in one slice's layer but not the other's: that slice
    skips its tokens (and the call is flagged), the other applies them.  At
    o = 2560 each expand workgroup has one chunk of each slice, the first in
    the slice that misses the id."""
    T, L, d = 48, 4, 512
    dtype = torch.bfloat16
    announce(f"slices missing adapter o={o} layers={layers}")
    engine = WarpPipeEngine(WarpPipeConfig(layer_stride=STRIDE))
    per_layer = [register(engine, 0, range(L), [16] * L, d, o, dtype, 700),
                 register(engine, 1, [0, 1, 3], [32] * 3, d, o, dtype, 720)]
    idx = np.random.default_rng(3).integers(0, L, size=T)
    idx[:4] = 2
    X = randn((T, d), 16, dtype)
    Y0 = randn((T, 2 * o), 17, dtype)
    assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
    Y = Y0.cuda()
    engine.shrink_expand_slices(X.cuda(), Y, layers, [o, o], [0, o])
    torch.cuda.synchronize()
    assert engine.device_errors() != 0
    segs = so.seg_bounds(idx).tolist()
    ref = reference(X, Y0, segs, [per_layer[l] for l in layers], [o, o], [0, o], 64, T)
    assert_close(Y, ref, "missing id")


def test_large_plan_runs_per_slice():
    """Over 512 tokens: one shrink_expand per slice, same results."""
    T, L, d, o = 900, 6, 1024, 512
    dtype = torch.bfloat16
    announce("slices large plan T=900")
    engine = WarpPipeEngine(WarpPipeConfig(layer_stride=STRIDE))
    per_slice = [register(engine, lay, range(L), [32] * L, d, o, dtype, 800 + 40 * lay) for lay in range(2)]
    idx = np.sort(np.random.default_rng(8).integers(0, L, size=T))
    X = randn((T, d), 18, dtype)
    Y0 = randn((T, 2 * o), 19, dtype)
    assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
    Y = Y0.cuda()
    engine.shrink_expand_slices(X.cuda(), Y, [0, 1], [o, o], [0, o], rank=0)
    torch.cuda.synchronize()
    segs = so.seg_bounds(idx).tolist()
    assert_close(Y, reference(X, Y0, segs, per_slice, [o, o], [0, o], 64, T), "large plan")
    assert engine.device_errors() == 0


def test_captured_replays_follow_routing():
    """A graph holding build_seg_bounds and a two-layer call, replayed with
    other routings (eager work between replays), matches the oracle each time."""
    T, L, d, o = 40, 5, 512, 384
    dtype = torch.bfloat16
    engine = WarpPipeEngine(WarpPipeConfig(layer_stride=STRIDE))
    rng = np.random.default_rng(21)
    per_slice = [register(engine, lay, range(L), [int(v) for v in rng.choice([8, 16, 32, 64], size=L)], d, o, dtype,
                          900 + 40 * lay) for lay in range(2)]
    X = randn((T, d), 20, dtype)
    Y0 = randn((T, 2 * o), 21, dtype)
    routings = [rng.integers(-1, L, size=T) for _ in range(2)]
    x_d, y0_d = X.cuda(), Y0.cuda()
    y = y0_d.clone()
    idx_buf = torch.from_numpy(routings[0]).cuda()

    def step():
        engine.build_seg_bounds(idx_buf)
        engine.shrink_expand_slices(x_d, y, [0, 1], [o, o], [0, o])

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    announce("slices graph capture")
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    for it, k in enumerate([1, 0, 1]):
        announce(f"slices graph replay {it}")
        idx_buf.copy_(torch.from_numpy(routings[k]))
        y.copy_(y0_d)
        g.replay()
        torch.cuda.synchronize()
        segs = so.seg_bounds(routings[k]).tolist()
        assert_close(y, reference(X, Y0, segs, per_slice, [o, o], [0, o], 64, T), f"replay {it}")
        _ = (x_d.float() * 2).sum().item()  # eager work between replays
    assert engine.device_errors() == 0


def test_arguments_are_checked():
    engine = WarpPipeEngine(WarpPipeConfig(layer_stride=STRIDE))
    d, o, T = 256, 128, 16
    register(engine, 0, range(2), [16, 16], d, o, torch.bfloat16, 1000)
    X = torch.zeros(T, d, dtype=torch.bfloat16, device="cuda")
    Y = torch.zeros(T, 2 * o, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="build_seg_bounds"):
        engine.shrink_expand_slices(X, Y, [0, 1], [o, o], [0, o])
    assert engine.build_seg_bounds(torch.zeros(T, dtype=torch.int64, device="cuda"))
    with pytest.raises(RuntimeError, match="does not fit"):
        engine.shrink_expand_slices(X, Y, [0, 1], [o, o], [0, o + 4])
    with pytest.raises(RuntimeError, match="one width"):
        engine.shrink_expand_slices(X, Y, [0, 1], [o], [0, o])
    with pytest.raises(RuntimeError, match="slices"):
        engine.shrink_expand_slices(X, torch.zeros(T, 5 * o, dtype=torch.bfloat16, device="cuda"),
                                    [0, 1, 2, 3, 4], [o] * 5, [k * o for k in range(5)])
    with pytest.raises(RuntimeError, match="rank"):
        engine.shrink_expand_slices(X, Y, [0, 1], [o, o], [0, o], rank=12)
    assert engine.device_errors() == 0
