"""GPU: add_lora with one A per output slice (wp_add_lora_nslice, vLLM's
add_lora_packed_nslice: packed q/k/v and gate/up layers), the hook's
override of it, and the packed draft-model linear -- all against the CPU
oracle (oracle.bgmv.add_lora_nslice: one independent add_lora per slice) on
the same seeded inputs."""
import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from adapterslotsplusplus_amd import WarpPipeEngine, workloads as wl
from adapterslotsplusplus_amd import punica_wrapper as pw
from adapterslotsplusplus_amd.lora_linear import DraftLoRAContext, WarpPipeLoRAPackedLinear
from oracle import bgmv
from oracle import segments as so
from tests.helpers import announce, assert_close, randn, seeds

pytestmark = pytest.mark.gpu


def inputs(T, L, rank, d, widths, dtype, seed, idx=None):
    if idx is None:
        idx = torch.randint(-1, L, (T,), generator=torch.Generator().manual_seed(seed))
    x = randn((T, d), seed + 1, dtype)
    was = [randn((L, 1, rank, d), seed + 10 + i, dtype, 0.02) for i in range(len(widths))]
    wbs = [randn((L, 1, o, rank), seed + 20 + i, dtype, 0.02) for i, o in enumerate(widths)]
    y0 = randn((T, sum(widths)), seed + 2, dtype)
    return idx, x, was, wbs, y0


def run(engine, idx, x, was, wbs, y0, scale, offs):
    assert engine.build_seg_bounds(idx.cuda())
    y = y0.cuda()
    assert engine.add_lora_slices(y, x.cuda(), [w.cuda() for w in was], [w.cuda() for w in wbs], scale, offs)
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("name,T,L,widths", [
    ("cfg2 qkv", 256, 64, [4096, 4096, 4096]),
    ("cfg2 gqa", 256, 64, [4096, 1024, 1024]),
    ("cfg5 qkv", 128, 32, [2048, 2048, 2048]),
    ("gate/up", 256, 64, [4096, 4096]),
])
def test_nslice_decode_shapes(name, T, L, widths, dtype):
    d = 4096 if T == 256 else 2048
    idx = wl.zipf_indices(T, L, 1.1, 1) if T == 256 else torch.repeat_interleave(torch.arange(L), T // L)
    announce(f"nslice {name}: T={T} L={L} d={d} widths={widths} {dtype}")
    idx, x, was, wbs, y0 = inputs(T, L, 32, d, widths, dtype, 5, idx)
    offs = [sum(widths[:i]) for i in range(len(widths))]
    engine = WarpPipeEngine()
    y = run(engine, idx, x, was, wbs, y0, 0.5, offs)
    segs = so.seg_bounds(idx.tolist()).tolist()
    assert_close(y, bgmv.add_lora_nslice(y0, x, was, wbs, 0.5, segs, offs), name)
    assert engine.device_errors() == 0


@pytest.mark.parametrize("seed", seeds(8))
def test_nslice_random_shapes(seed):
    """Seeded one-A-per-slice calls: 2-4 slices of random widths side by side,
    T across the 512-token switch, runs of random ids (some -1), both
    dtypes, ranks 8-64."""
    rng = np.random.default_rng(9000 + seed)
    T = int(rng.choice([1, 5, 64, 128, 200, 256, 300, 512, 600]))
    L = int(rng.integers(1, 70))
    rank = int(rng.choice([8, 16, 32, 64]))
    d = int(rng.choice([128, 1032, 2048, 4096]))
    ns = int(rng.integers(2, 5))
    widths = [int(rng.integers(1, 1100)) * 4 for _ in range(ns)]
    dtype = torch.bfloat16 if seed % 2 else torch.float16
    idx = torch.from_numpy(np.repeat(rng.integers(-1, L, size=T), rng.integers(1, 6, size=T))[:T])
    announce(f"nslice random seed {seed}: T={T} L={L} r={rank} d={d} widths={widths} {dtype}")
    idx, x, was, wbs, y0 = inputs(T, L, rank, d, widths, dtype, 9100 + seed, idx)
    offs = [sum(widths[:i]) for i in range(ns)]
    engine = WarpPipeEngine()
    y = run(engine, idx, x, was, wbs, y0, 0.5, offs)
    segs = so.seg_bounds(idx.tolist()).tolist()
    assert_close(y, bgmv.add_lora_nslice(y0, x, was, wbs, 0.5, segs, offs), f"seed {seed}")
    assert engine.device_errors() == 0


@pytest.mark.parametrize("rank", [8, 16, 32, 64])
def test_nslice_ranks_ragged_windows(rank):
    """Four slices of ragged widths at non-adjacent offsets of a wider y; the
    columns between them stay untouched."""
    T, L, d = 77, 7, 1032
    widths = [260, 4, 516, 132]
    offs = [4, 272, 280, 804]
    announce(f"nslice ragged r={rank}")
    idx, x, was, wbs, _ = inputs(T, L, rank, d, widths, torch.bfloat16, 30 + rank)
    y0 = randn((T, 940), 3, torch.bfloat16)
    engine = WarpPipeEngine()
    y = run(engine, idx, x, was, wbs, y0, 0.75, offs)
    segs = so.seg_bounds(idx.tolist()).tolist()
    assert_close(y, bgmv.add_lora_nslice(y0, x, was, wbs, 0.75, segs, offs), f"r={rank}")
    assert engine.device_errors() == 0


def test_nslice_four_rank64_slices_wide_d():
    """Four 64-column A slices over d = 4096: the d-range count is capped so
    that the partial rows (d-ranges x 256 columns) fit the partial buffer."""
    T, L, d, widths = 256, 16, 4096, [1024, 1024, 512, 512]
    announce("nslice four rank-64 slices d=4096")
    idx = wl.zipf_indices(T, L, 1.1, 2)
    idx, x, was, wbs, y0 = inputs(T, L, 64, d, widths, torch.bfloat16, 60, idx)
    offs = [sum(widths[:i]) for i in range(len(widths))]
    engine = WarpPipeEngine()
    y = run(engine, idx, x, was, wbs, y0, 0.5, offs)
    segs = so.seg_bounds(idx.tolist()).tolist()
    assert_close(y, bgmv.add_lora_nslice(y0, x, was, wbs, 0.5, segs, offs), "4 x r64")
    assert engine.device_errors() == 0


def test_nslice_large_plan():
    """More than 512 tokens (64-token blocks): one shrink launch per A slice
    into its columns of the engine's H, then one expand."""
    T, L, d, widths = 1500, 12, 2048, [2048, 512, 512]
    announce("nslice large plan T=1500")
    lens = wl.lognormal_segments(T, L, 5.0, 1.0, seed=9)
    idx = torch.repeat_interleave(torch.arange(L), torch.tensor(lens))
    idx, x, was, wbs, y0 = inputs(T, L, 64, d, widths, torch.float16, 40, idx)
    offs = [0, 2048, 2560]
    engine = WarpPipeEngine()
    y = run(engine, idx, x, was, wbs, y0, 0.25, offs)
    segs = so.seg_bounds(idx.tolist()).tolist()
    assert_close(y, bgmv.add_lora_nslice(y0, x, was, wbs, 0.25, segs, offs), "large plan")
    assert engine.device_errors() == 0


def test_nslice_shared_a_equals_add_lora_slices():
    """The same A passed for every slice gives the shared-A call's result (one
    shrink) within the tolerance (the two may split d differently, so the
    fp32 partial sums can differ in order)."""
    T, L, d, widths = 200, 9, 2048, [1024, 1024, 512]
    idx, x, was, wbs, y0 = inputs(T, L, 32, d, widths, torch.bfloat16, 50)
    offs = [0, 1024, 2048]
    engine = WarpPipeEngine()
    assert engine.build_seg_bounds(idx.cuda())
    wa = was[0].cuda()
    wbd = [w.cuda() for w in wbs]
    y1, y2 = y0.cuda(), y0.cuda()
    announce("nslice with one A repeated vs the shared-A call")
    assert engine.add_lora_slices(y1, x.cuda(), [wa, wa, wa], wbd, 0.5, offs)
    assert engine.add_lora_slices(y2, x.cuda(), wa, wbd, 0.5, offs)
    torch.cuda.synchronize()
    segs = so.seg_bounds(idx.tolist()).tolist()
    assert_close(y1, bgmv.add_lora(y0, x, was[0], wbs, 0.5, segs, offs), "repeated A")
    assert_close(y2, y1.cpu(), "shared A vs repeated A")


def test_nslice_graph_replays_new_routing():
    """cfg5-shaped qkv call captured with build_seg_bounds; replays with new
    routings each match the oracle."""
    T, L, d, widths = 128, 32, 2048, [2048, 2048, 2048]
    idx, x, was, wbs, y0 = inputs(T, L, 32, d, widths, torch.bfloat16, 60)
    offs = [0, 2048, 4096]
    engine = WarpPipeEngine()
    xd, wad, wbd = x.cuda(), [w.cuda() for w in was], [w.cuda() for w in wbs]
    idx_buf = idx.cuda()
    y = y0.cuda()

    def step():
        engine.build_seg_bounds(idx_buf)
        engine.add_lora_slices(y, xd, wad, wbd, 2.0, offs)

    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    g = torch.Generator().manual_seed(61)
    for rep in range(3):
        announce(f"nslice replay {rep}")
        new_idx = torch.randint(-1, L, (T,), generator=g)
        idx_buf.copy_(new_idx)
        y.copy_(y0.cuda())
        graph.replay()
        torch.cuda.synchronize()
        segs = so.seg_bounds(new_idx.tolist()).tolist()
        assert_close(y, bgmv.add_lora_nslice(y0, x, was, wbs, 2.0, segs, offs), f"replay {rep}")
    assert engine.device_errors() == 0


class FakePunica:
    """vLLM 0.6.3 PunicaWrapper stand-in: its add_lora_packed_nslice is the
    loop of add_lora calls over the slices; both record their calls."""

    def __init__(self, indices):
        self.token_lora_indices = indices
        self.is_prefill = False
        self.calls = []

    def update_metadata(self, mapping, lora_index_to_id, max_loras, vocab_size, extra_vocab_size,
                        long_lora_context=None):
        self.calls.append("update_metadata")

    def add_lora(self, y, x, wa_t_all, wb_t_all, scale, y_offset=None, y_slice_size=None, *, buffer=None):
        self.calls.append("stock add_lora")
        idx = self.token_lora_indices
        y2 = y.view(-1, y.shape[-1])
        off = int(y_offset or 0)
        o = int(wb_t_all.size(-2))
        for t in range(x.shape[0]):
            i = int(idx[t])
            if i >= 0:
                h = (x[t].float() @ wa_t_all[i, 0].float().T) * scale
                y2[t, off:off + o] = (y2[t, off:off + o].float() + h @ wb_t_all[i, 0].float().T).to(y.dtype)

    def add_lora_packed_nslice(self, y, x, lora_a_stacked, lora_b_stacked, scale, output_slices):
        self.calls.append("stock nslice")
        off = 0
        for a, b, o in zip(lora_a_stacked, lora_b_stacked, output_slices):
            self.add_lora(y, x, a, b, scale, off, o)
            off += o


class FakeManager:
    def __init__(self, wrapper):
        class AdapterManager:
            pass

        self._adapter_manager = AdapterManager()
        self._adapter_manager.punica_wrapper = wrapper


def test_hook_nslice_on_kernels_and_fallback(monkeypatch):
    monkeypatch.setenv("AS_WARP_PIPE", "1")
    monkeypatch.setattr(pw, "_engine", WarpPipeEngine())
    T, L, d = 64, 5, 1024
    idx, x, was, wbs, y0 = inputs(T, L, 16, d, [1024, 256, 256], torch.bfloat16, 70)
    w = FakePunica(idx.cuda())
    assert pw.install_warp_pipe_add_lora(FakeManager(w))
    w.update_metadata(None, None, L, 0, 0)
    announce("hook add_lora_packed_nslice on the kernels")
    y = y0.cuda()
    w.add_lora_packed_nslice(y, x.cuda(), tuple(a.cuda() for a in was), tuple(b.cuda() for b in wbs), 0.5,
                             (1024, 256, 256))
    torch.cuda.synchronize()
    assert w.calls == ["update_metadata"], w.calls
    segs = so.seg_bounds(idx.tolist()).tolist()
    assert_close(y, bgmv.add_lora_nslice(y0, x, was, wbs, 0.5, segs, [0, 1024, 1280]), "hook nslice")
    announce("hook add_lora_packed_nslice with two ranks -> stock")
    wbs2 = [wbs[0], randn((L, 1, 256, 32), 77, torch.bfloat16, 0.02)]
    was2 = [was[0], randn((L, 1, 32, d), 78, torch.bfloat16, 0.02)]
    y = y0[:, :1280].contiguous().cuda()
    w.add_lora_packed_nslice(y, x.cuda(), tuple(a.cuda() for a in was2), tuple(b.cuda() for b in wbs2), 0.5,
                             (1024, 256))
    torch.cuda.synchronize()
    # The parent's loop calls self.add_lora per slice: the switched class runs
    # each of them on the kernels (one launch per slice).
    assert w.calls == ["update_metadata", "stock nslice"], w.calls
    assert_close(y, bgmv.add_lora_nslice(y0[:, :1280], x, was2, wbs2, 0.5, segs, [0, 1024]), "two ranks")


def test_packed_linear_matches_separate_projections():
    """WarpPipeLoRAPackedLinear (one base GEMM over q/k/v, one launch for the
    three deltas) against the three projections computed in torch with the
    engine's rounding points, in a captured step replayed with new routing."""
    HID, K, r, T = 1024, 8, 32, 64
    dt = torch.bfloat16
    torch.manual_seed(3)
    bases = [nn.Linear(HID, o, bias=(i == 1)).to(device="cuda", dtype=dt) for i, o in enumerate([1024, 256, 256])]
    for b in bases:
        with torch.no_grad():
            b.weight.copy_(torch.randn_like(b.weight) * 0.03)
            if b.bias is not None:
                b.bias.copy_(torch.randn_like(b.bias) * 0.1)
    As = [randn((K, r, HID), 80 + i, dt, 0.05).cuda() for i in range(3)]
    Bs = [randn((K, b.out_features, r), 90 + i, dt, 0.05).cuda() for i, b in enumerate(bases)]
    engine = WarpPipeEngine()
    ctx = DraftLoRAContext(engine, T, scale=2.0)
    mod = WarpPipeLoRAPackedLinear(bases, As, Bs, ctx)
    x = randn((T, HID), 95, dt).cuda()
    g = torch.Generator().manual_seed(96)
    routes = [torch.randint(-1, K, (T,), generator=g) for _ in range(3)]
    ctx.set_routing(routes[0].cuda())
    out = {}

    def step():
        ctx.begin_step()
        out["qkv"] = mod(x)

    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for rep, idx in enumerate(routes):
        announce(f"packed linear replay {rep}")
        ctx.set_routing(idx.cuda())
        graph.replay()
        torch.cuda.synchronize()
        for i, (b, A, B) in enumerate(zip(bases, As, Bs)):
            base = F.linear(x, b.weight, b.bias)
            ok = (idx >= 0).cuda()
            ii = idx.clamp(min=0).cuda()
            h = torch.bmm(x.float().unsqueeze(1), A.float()[ii].transpose(1, 2).contiguous())[:, 0]
            h = (h * 2.0).to(dt)
            delta = torch.bmm(h.float().unsqueeze(1), B.float()[ii].transpose(1, 2).contiguous())[:, 0]
            ref = torch.where(ok[:, None], (base.float() + delta).to(dt), base)
            assert_close(out["qkv"][i], ref, f"replay {rep} projection {i}")
    assert engine.device_errors() == 0
