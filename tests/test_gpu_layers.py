"""Multi-layer adapter store (WarpPipeConfig.layer_stride) on the GPU.

The reference's store keeps one (A, B) per adapter id (csrc/bridge/
adapter_store.h:12-19), so a model with L LoRA'd layers needs L engines or
re-registration per layer.  Here one engine holds every layer's weights under
ids layer * stride + adapter_id, and one build_seg_bounds table routes all
layers: shrink / expand(..., layer=l) apply layer l's weights to each token's
adapter id.  Reference: the oracle's bgmv over that layer's adapters alone."""
import numpy as np
import pytest
import torch

from adapterslotsplusplus_amd import WarpPipeConfig, WarpPipeEngine
from oracle import bgmv
from oracle import segments as so
from tests.helpers import announce, assert_close, randn

pytestmark = pytest.mark.gpu

LAYERS, K, STRIDE = 3, 4, 8


def register_layers(engine, rank, d, o, dtype, seed):
    per_layer = []
    for lay in range(LAYERS):
        A = randn((K, rank, d), seed + 2 * lay, dtype, 0.02)
        B = randn((K, o, rank), seed + 2 * lay + 1, dtype, 0.02)
        adapters = {}
        for aid in range(K):
            alpha = 0.25 * (lay + 1)
            engine.register_adapter(aid, A[aid].cuda().contiguous(), B[aid].cuda().contiguous(), alpha,
                                    rank=rank, layer=lay)
            adapters[aid] = (A[aid], B[aid], alpha)
        per_layer.append(adapters)
    return per_layer


@pytest.mark.parametrize("T,rank", [(48, 16), (700, 32)])
def test_layers_share_one_table(T, rank):
    announce(f"multi-layer store T={T} rank={rank}")
    dtype = torch.bfloat16
    d, o = 1024, 768
    engine = WarpPipeEngine(WarpPipeConfig(layer_stride=STRIDE))
    per_layer = register_layers(engine, rank, d, o, dtype, 500)
    idx = np.random.default_rng(T).integers(-1, K, size=T)
    assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
    segs = so.seg_bounds(idx).tolist()
    for lay in (2, 0, 1):
        X = randn((T, d), 600 + lay, dtype)
        Y0 = randn((T, o), 700 + lay, dtype)
        H = engine.shrink(X.cuda(), d, rank, T, layer=lay)
        Y = Y0.cuda()
        engine.expand(H, Y, o, rank, layer=lay)
        torch.cuda.synchronize()
        H_ref = bgmv.shrink(X, segs, per_layer[lay], rank, T)
        assert_close(H, H_ref, f"H layer {lay}")
        assert_close(Y, bgmv.expand(H_ref, Y0, segs, per_layer[lay]), f"Y layer {lay}")
        # Negative control: another layer's weights give a different H.
        other = bgmv.shrink(X, segs, per_layer[(lay + 1) % LAYERS], rank, T)
        assert not torch.allclose(H.cpu().float(), other.float(), rtol=1e-2, atol=1e-3)
    # Calls without a layer read layer 0 again.
    X = randn((T, d), 800, dtype)
    H = engine.shrink(X.cuda(), d, rank, T)
    torch.cuda.synchronize()
    assert_close(H, bgmv.shrink(X, segs, per_layer[0], rank, T), "H default layer")
    assert engine.device_errors() == 0


def test_evicted_layer_is_skipped_and_flagged():
    announce("multi-layer store eviction")
    dtype = torch.float16
    d, o, rank, T = 512, 512, 16, 64
    engine = WarpPipeEngine(WarpPipeConfig(layer_stride=STRIDE))
    per_layer = register_layers(engine, rank, d, o, dtype, 900)
    idx = np.random.default_rng(5).integers(0, K, size=T)
    assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
    segs = so.seg_bounds(idx).tolist()
    engine.evict_adapter(1, layer=1)
    X = randn((T, d), 901, dtype)
    # Layer 2 keeps adapter 1.
    H = engine.shrink(X.cuda(), d, rank, T, layer=2)
    torch.cuda.synchronize()
    assert_close(H, bgmv.shrink(X, segs, per_layer[2], rank, T), "H layer 2")
    assert engine.device_errors() == 0
    # Layer 1 has lost it: its tokens are skipped and the call is flagged.
    H1 = engine.shrink(X.cuda(), d, rank, T, layer=1).cpu()
    torch.cuda.synchronize()
    assert engine.device_errors() != 0
    kept = {a: w for a, w in per_layer[1].items() if a != 1}
    mask = torch.from_numpy(idx != 1)
    ref = bgmv.shrink(X, [s for s in segs if s[0] != 1], kept, rank, T)
    assert_close(H1[mask], ref[mask], "H layer 1 kept tokens")
    # An id >= the stride would address the next layer's adapters: skipped.
    idx2 = idx.copy()
    idx2[: T // 2] = STRIDE
    assert engine.build_seg_bounds(torch.from_numpy(idx2).cuda())
    H0 = engine.shrink(X.cuda(), d, rank, T, layer=0).cpu()
    torch.cuda.synchronize()
    assert engine.device_errors() != 0
    assert torch.count_nonzero(H0[: T // 2]) == 0
    assert_close(H0[T // 2:], bgmv.shrink(X, segs, per_layer[0], rank, T)[T // 2:], "H layer 0 in-range tokens")
    # Evicting without a layer drops every layer of the id.
    engine.evict_adapter(2)
    for lay in range(LAYERS):
        assert engine.prefetch_adapter(2, layer=lay) == -1


def test_layer_arguments_are_checked():
    engine = WarpPipeEngine()
    with pytest.raises(RuntimeError, match="layer_stride"):
        engine.shrink(torch.zeros(4, 64, dtype=torch.float16, device="cuda"), 64, 16, 4, layer=1)
    engine = WarpPipeEngine(WarpPipeConfig(layer_stride=4))
    A = torch.zeros(16, 64, dtype=torch.float16, device="cuda")
    B = torch.zeros(64, 16, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="adapter ids must be"):
        engine.register_adapter(4, A, B, 1.0, rank=16, layer=0)
    engine.register_adapter(1, A, B, 1.0, rank=16, layer=0)
    engine.register_adapter(1, A, B, 1.0, rank=16, layer=3)
    # Host-built tables route layer 0 only.
    engine.build_segments([1], [0, 4])
    with pytest.raises(RuntimeError, match="build_seg_bounds"):
        engine.shrink(torch.zeros(4, 64, dtype=torch.float16, device="cuda"), 64, 16, 4, layer=3)


def test_layers_in_one_captured_step():
    """One graph holds build_seg_bounds and every layer's shrink_expand; each
    call's layer offset is recorded with it, so replays with other routings
    apply each layer's own adapters."""
    dtype = torch.bfloat16
    d, o, rank, T = 512, 384, 16, 40
    engine = WarpPipeEngine(WarpPipeConfig(layer_stride=STRIDE))
    per_layer = register_layers(engine, rank, d, o, dtype, 950)
    X = randn((T, d), 960, dtype)
    Y0 = randn((T, o), 961, dtype)
    rng = np.random.default_rng(9)
    routings = [rng.integers(-1, K, size=T) for _ in range(2)]
    x_d, y0_d = X.cuda(), Y0.cuda()
    idx_buf = torch.from_numpy(routings[0]).cuda()
    ys = [y0_d.clone() for _ in range(LAYERS)]

    def step():
        engine.build_seg_bounds(idx_buf)
        for lay in range(LAYERS):
            engine.shrink_expand(x_d, ys[lay], o, rank, layer=lay)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    announce("layers graph capture")
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    for it, k in enumerate([1, 0, 1]):
        announce(f"layers graph replay {it}")
        idx_buf.copy_(torch.from_numpy(routings[k]))
        for y in ys:
            y.copy_(y0_d)
        g.replay()
        torch.cuda.synchronize()
        segs = so.seg_bounds(routings[k]).tolist()
        for lay in range(LAYERS):
            ref = bgmv.expand(bgmv.shrink(X, segs, per_layer[lay], rank, T), Y0, segs, per_layer[lay])
            assert_close(ys[lay], ref, f"replay {it} layer {lay}")
    assert engine.device_errors() == 0
