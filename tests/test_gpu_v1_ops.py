"""GPU: vLLM V1's LoRA op surface (adapterslotsplusplus_amd.punica_v1) on the
HIP kernels, against the CPU oracle of V1's ops (oracle/v1_ops.py).

A duck-typed PunicaWrapperGPU stands in for vLLM's (not importable here): its
update_metadata keeps token_lora_indices, and its add_shrink / add_expand /
add_lora_embedding / add_lora_linear -- the parent methods the mixin falls
back to -- compute V1's formulas with the oracle and record that they ran,
so a test can tell which path produced a result.  The live wrapper is
switched with install_warp_pipe_v1 and AS_WARP_PIPE=1."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from adapterslotsplusplus_amd import WarpPipeConfig, WarpPipeEngine
from adapterslotsplusplus_amd import punica_v1 as v1
from adapterslotsplusplus_amd import punica_wrapper as pw
from adapterslotsplusplus_amd import workloads as wl
from oracle import v1_ops
from tests.helpers import announce, assert_close, h_tie_flips, randn, seeds

pytestmark = pytest.mark.gpu


class FakeV1Punica:
    """PunicaWrapperGPU stand-in: the parent's bookkeeping and V1's formulas."""

    def __init__(self):
        self.calls = []
        self.is_prefill = False
        self._idx = None

    @property
    def token_lora_indices(self):
        return self._idx

    def update_metadata(self, mapping, lora_index_to_id, max_loras, vocab_size, extra_vocab_size, **kwargs):
        self.calls.append("update_metadata")
        self.is_prefill = mapping.is_prefill
        self._idx = torch.tensor(mapping.index_mapping, dtype=torch.int64, device="cuda")

    def add_shrink(self, y, x, lora_a_stacked, scale, **kwargs):
        self.calls.append("parent add_shrink")
        ids = self._idx.cpu()
        y.copy_(v1_ops.lora_shrink(y.cpu(), x.cpu(), [a.cpu() for a in lora_a_stacked], scale, ids).to(y.device))

    def add_expand(self, y, x, lora_b_stacked, lora_bias_stacked, output_slices, offset_start=0, add_inputs=True,
                   **kwargs):
        self.calls.append("parent add_expand")
        ids = self._idx.cpu()
        bs = None if lora_bias_stacked is None else [None if b is None else b.cpu() for b in lora_bias_stacked]
        yc = v1_ops.apply_bias(y.cpu(), bs, output_slices, ids, offset_start)
        yc = v1_ops.lora_expand(yc, x.cpu(), [b.cpu() for b in lora_b_stacked], output_slices, ids, offset_start, True)
        y.copy_(yc.view_as(y).to(y.device))

    def add_lora_embedding(self, y, x, lora_b_stacked, add_inputs=True, **kwargs):
        self.calls.append("parent add_lora_embedding")
        ids = self._idx.cpu()
        yc = v1_ops.lora_expand(y.cpu(), x.cpu().unsqueeze(0), [lora_b_stacked.cpu()], [int(lora_b_stacked.size(-2))],
                                ids, 0, add_inputs)
        y.copy_(yc.view_as(y).to(y.device))

    def add_lora_linear(self, y, x, lora_a_stacked, lora_b_stacked, lora_bias_stacked, scale, output_slices, *,
                        buffer=None, **kwargs):
        self.calls.append("parent add_lora_linear")
        ids = self._idx.cpu()
        bs = None if lora_bias_stacked is None else [None if b is None else b.cpu() for b in lora_bias_stacked]
        yc = v1_ops.add_lora_linear(y.cpu(), x.cpu(), [a.cpu() for a in lora_a_stacked],
                                    [b.cpu() for b in lora_b_stacked], bs, scale, output_slices, ids)
        y.copy_(yc.view_as(y).to(y.device))


class FakeManager:
    def __init__(self, wrapper):
        self._adapter_manager = SimpleNamespace(punica_wrapper=wrapper)


def mapping(ids, is_prefill=False):
    return SimpleNamespace(index_mapping=tuple(int(v) for v in ids), is_prefill=is_prefill)


@pytest.fixture
def wrapper(monkeypatch):
    monkeypatch.setenv("AS_WARP_PIPE", "1")
    monkeypatch.setattr(pw, "_engine", WarpPipeEngine(WarpPipeConfig(max_tokens=4096)))
    w = FakeV1Punica()
    assert v1.install_warp_pipe_v1(FakeManager(w))
    assert isinstance(w, v1.WarpPipeV1Mixin)
    assert not v1.install_warp_pipe_v1(FakeManager(w))
    return w


def routing(T, L, seed, none_every=7):
    ids = wl.zipf_indices(T, L, 1.1, seed)
    ids[::none_every] = -1
    return ids


def weights(L, r, d, outs, dtype, seed, bias_slices=()):
    was = tuple(randn((L, 1, r, d), seed + i, dtype, 0.02).cuda() for i in range(len(outs)))
    wbs = tuple(randn((L, 1, o, r), seed + 10 + i, dtype, 0.02).cuda() for i, o in enumerate(outs))
    bias = None
    if bias_slices:
        bias = tuple(randn((L, 1, o), seed + 20 + i, dtype, 0.5).cuda() if i in bias_slices else None
                     for i, o in enumerate(outs))
    return was, wbs, bias


def cpu(ts):
    return None if ts is None else [None if t is None else t.cpu() for t in ts]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bias_slices", [(), (0, 2)])
def test_add_lora_linear_packed_qkv(wrapper, dtype, bias_slices):
    T, L, r, d, outs = 64, 16, 16, 1024, (1024, 256, 256)
    announce(f"v1 add_lora_linear qkv {dtype} bias {bias_slices}")
    ids = routing(T, L, 3)
    wrapper.update_metadata(mapping(ids), None, L, 0, 0)
    was, wbs, bias = weights(L, r, d, outs, dtype, 40, bias_slices)
    x = randn((T, d), 50, dtype)
    y0 = randn((T, sum(outs)), 51, dtype)
    y = y0.cuda()
    wrapper.add_lora_linear(y, x.cuda(), was, wbs, bias, 1.0, outs)
    torch.cuda.synchronize()
    assert wrapper.calls == ["update_metadata"], wrapper.calls
    ref = v1_ops.add_lora_linear(y0, x, cpu(was), cpu(wbs), cpu(bias), 1.0, outs, ids)
    assert_close(y, ref, "add_lora_linear")
    assert pw._engine.device_errors() == 0


@pytest.mark.parametrize("T,prefill", [(48, False), (1000, True)])
def test_shrink_buffer_then_expand_with_bias_and_offset(wrapper, T, prefill):
    """V1's two-op form: add_shrink into an fp32 [n, T, r] buffer, then
    add_expand of that buffer with biases into windows that start at
    offset_start; decode- and prefill-sized tables."""
    L, r, d, outs, off0 = 8, 32, 512, (384, 128), 64
    dtype = torch.bfloat16
    announce(f"v1 add_shrink + add_expand T={T}")
    if prefill:
        lens = wl.lognormal_segments(T, L, 4.0, 1.0, seed=6)
        ids = torch.repeat_interleave(torch.arange(L), torch.tensor(lens))
        ids[ids == 3] = -1
    else:
        ids = routing(T, L, 5)
    wrapper.update_metadata(mapping(ids, prefill), None, L, 0, 0)
    was, wbs, bias = weights(L, r, d, outs, dtype, 60, (1,))
    x = randn((T, d), 70, dtype)
    buf0 = torch.randn(2, T, r, generator=torch.Generator().manual_seed(71))
    buf = buf0.cuda()
    wrapper.add_shrink(buf, x.cuda(), was, 0.5)
    torch.cuda.synchronize()
    buf_ref = v1_ops.lora_shrink(buf0, x, cpu(was), 0.5, ids)
    assert_close(buf, buf_ref, "add_shrink buffer", rtol=1e-4, atol=1e-4)
    y0 = randn((T, off0 + sum(outs) + 32), 72, dtype)
    y = y0.cuda()
    wrapper.add_expand(y, buf, wbs, bias, outs, offset_start=off0)
    torch.cuda.synchronize()
    assert wrapper.calls == ["update_metadata"], wrapper.calls
    ref = v1_ops.lora_expand(v1_ops.apply_bias(y0, cpu(bias), outs, ids, off0), buf.cpu(), cpu(wbs), outs, ids, off0)
    assert_close(y, ref, "add_expand")
    assert pw._engine.device_errors() == 0


@pytest.mark.parametrize("add_inputs", [True, False])
def test_add_lora_embedding(wrapper, add_inputs):
    T, L, r, o = 40, 6, 8, 768
    dtype = torch.float16
    announce(f"v1 add_lora_embedding add_inputs={add_inputs}")
    ids = routing(T, L, 8, none_every=5)
    wrapper.update_metadata(mapping(ids), None, L, 0, 0)
    h = randn((T, r), 80, dtype)
    wb = randn((L, 1, o, r), 81, dtype, 0.1).cuda()
    y0 = randn((T, o), 82, dtype)
    y = y0.cuda()
    wrapper.add_lora_embedding(y, h.cuda(), wb, add_inputs=add_inputs)
    torch.cuda.synchronize()
    assert wrapper.calls == ["update_metadata"], wrapper.calls
    ref = v1_ops.lora_expand(y0, h.unsqueeze(0), [wb.cpu()], [o], ids, 0, add_inputs)
    assert_close(y, ref, "add_lora_embedding")


def test_fallbacks(wrapper):
    """A rank without kernels, slices of different ranks, and a table the
    engine could not build each run the parent's method."""
    dtype = torch.bfloat16
    T, L, d = 32, 4, 256
    ids = routing(T, L, 9)
    wrapper.update_metadata(mapping(ids), None, L, 0, 0)
    x = randn((T, d), 90, dtype)
    cases = []
    was, wbs, _ = weights(L, 24, d, (256,), dtype, 91)
    cases.append(("rank 24", was, wbs))
    wa16, wb16, _ = weights(L, 16, d, (256,), dtype, 92)
    wa32, wb32, _ = weights(L, 32, d, (256,), dtype, 93)
    cases.append(("mixed ranks", wa16 + wa32, wb16 + wb32))
    for what, was, wbs in cases:
        announce(f"v1 fallback: {what}")
        outs = tuple(int(b.size(-2)) for b in wbs)
        y0 = randn((T, sum(outs)), 94, dtype)
        y = y0.cuda()
        wrapper.calls.clear()
        wrapper.add_lora_linear(y, x.cuda(), was, wbs, None, 1.0, outs)
        assert wrapper.calls == ["parent add_lora_linear"], (what, wrapper.calls)
        torch.cuda.synchronize()
        ref = v1_ops.add_lora_linear(y0, x, cpu(was), cpu(wbs), None, 1.0, outs, ids)
        assert_close(y, ref, f"fallback {what}")
    # More tokens than the engine's max_tokens: the whole step falls back.
    big = torch.zeros(5000, dtype=torch.int64)
    wrapper.update_metadata(mapping(big, True), None, L, 0, 0)
    was, wbs, _ = weights(L, 16, d, (256,), dtype, 95)
    xb = randn((5000, d), 96, dtype).cuda()
    yb = torch.zeros(5000, 256, dtype=dtype, device="cuda")
    wrapper.calls.clear()
    wrapper.add_lora_linear(yb, xb, was, wbs, None, 1.0, (256,))
    assert wrapper.calls == ["parent add_lora_linear"], wrapper.calls


def test_captured_replays_follow_update_metadata(wrapper):
    """add_lora_linear (with a bias) captured once; update_metadata runs outside
    the graph with a new routing before each replay, and every replay matches
    the oracle for that routing (and not for the previous one)."""
    T, L, r, d, outs = 64, 12, 32, 1024, (1024, 512)
    dtype = torch.bfloat16
    announce("v1 captured add_lora_linear")
    was, wbs, bias = weights(L, r, d, outs, dtype, 110, (0,))
    x = randn((T, d), 111, dtype)
    y0 = randn((T, sum(outs)), 112, dtype)
    xd, y = x.cuda(), y0.cuda()
    routings = [routing(T, L, 120 + k) for k in range(3)]
    wrapper.update_metadata(mapping(routings[0]), None, L, 0, 0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        wrapper.add_lora_linear(y, xd, was, wbs, bias, 1.0, outs)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        wrapper.add_lora_linear(y, xd, was, wbs, bias, 1.0, outs)
    prev = None
    for k, ids in enumerate(routings):
        wrapper.update_metadata(mapping(ids), None, L, 0, 0)
        y.copy_(y0.cuda())
        g.replay()
        torch.cuda.synchronize()
        ref = v1_ops.add_lora_linear(y0, x, cpu(was), cpu(wbs), cpu(bias), 1.0, outs, ids)
        assert_close(y, ref, f"replay {k}")
        if prev is not None:
            assert not torch.equal(y.cpu(), prev), "a replay reproduced the previous routing's result"
        prev = ref
    assert "parent add_lora_linear" not in wrapper.calls
    assert pw._engine.device_errors() == 0


def test_update_metadata_reports_skipped_tokens(wrapper, monkeypatch):
    """An id outside the stacked weights makes the kernels skip its tokens
    (device error 1); the next steps' update_metadata report it without a
    host wait, and AS_WARP_PIPE_STRICT=1 turns the report into an error."""
    T, L, r, d, outs = 32, 4, 16, 256, (256,)
    dtype = torch.bfloat16
    announce("v1 skipped tokens reported")
    ids = routing(T, L, 130)
    ids[5] = L + 3  # beyond the stacked weights
    wrapper.update_metadata(mapping(ids), None, L, 0, 0)
    was, wbs, _ = weights(L, r, d, outs, dtype, 131)
    y = torch.zeros(T, 256, dtype=dtype, device="cuda")
    wrapper.add_lora_linear(y, randn((T, d), 132, dtype).cuda(), was, wbs, None, 1.0, outs)
    before = pw.device_errors_seen
    pw.device_errors_seen = 0
    try:
        ok = routing(T, L, 133)
        seen = 0
        # The first poll after the call enqueues the move of the word; a later
        # one returns it once that move has completed.
        for _ in range(3):
            wrapper.update_metadata(mapping(ok), None, L, 0, 0)
            torch.cuda.synchronize()
            seen |= pw.device_errors_seen
        assert seen & 1, f"device error 1 not reported (seen 0x{seen:x})"
        assert pw._engine.device_errors() == 0
        # Strict mode raises on the report.
        wrapper.update_metadata(mapping(ids), None, L, 0, 0)
        wrapper.add_lora_linear(y, randn((T, d), 132, dtype).cuda(), was, wbs, None, 1.0, outs)
        monkeypatch.setenv("AS_WARP_PIPE_STRICT", "1")
        with pytest.raises(RuntimeError, match="skipped tokens"):
            for _ in range(3):
                wrapper.update_metadata(mapping(ok), None, L, 0, 0)
                torch.cuda.synchronize()
    finally:
        pw.device_errors_seen |= before


@pytest.mark.parametrize("seed", seeds(8))
def test_random_v1_calls(wrapper, seed):
    """Seeded V1 calls on the kernels: T across the 512-token switch (decode
    and prefill tables), 1-3 slices of one rank (8-64) with ragged widths,
    biases on some slices, both dtypes; add_lora_linear, then add_shrink +
    add_expand (with an offset_start) on the same step.  No call may fall
    back.  H is rounded to the I/O type before the expand; where an exact H
    element sits within fp32 summation error of a rounding midpoint either
    neighbour is correct, and the output may move by that step times |B|."""
    rng = np.random.default_rng(5000 + seed)
    dtype = (torch.bfloat16, torch.float16)[seed % 2]
    T = int(rng.choice([1, 33, 200, 512, 513, 900]))
    d = int(rng.choice([64, 520, 2048]))
    r = int(rng.choice([8, 16, 32, 64]))
    L = int(rng.integers(1, 20))
    n = int(rng.integers(1, 4))
    # Slice widths of 8-element multiples keep y's rows 16-byte aligned.
    outs = tuple(int(rng.integers(1, 100)) * 8 for _ in range(n))
    bias_slices = tuple(i for i in range(n) if rng.integers(2))
    scale = float(rng.uniform(0.25, 2.0))
    off0 = int(rng.integers(0, 8)) * 8
    ids = torch.from_numpy(np.repeat(rng.integers(-1, L, size=T), rng.integers(1, 6, size=T))[:T].astype(np.int64))
    prefill = T > 512
    announce(f"v1 random seed {seed}: T={T} d={d} r={r} L={L} outs={outs} bias={bias_slices} off0={off0} {dtype}")
    wrapper.calls.clear()
    wrapper.update_metadata(mapping(ids, prefill), None, L, 0, 0)
    was, wbs, bias = weights(L, r, d, outs, dtype, 6000 + 10 * seed, bias_slices)
    x = randn((T, d), 6001 + 10 * seed, dtype)
    y0 = randn((T, sum(outs)), 6002 + 10 * seed, dtype)
    y = y0.cuda()
    wrapper.add_lora_linear(y, x.cuda(), was, wbs, bias, scale, outs)
    torch.cuda.synchronize()
    slack = torch.zeros(y0.shape, dtype=torch.float32)
    for a in torch.unique(ids[ids >= 0]).tolist():
        rows = torch.nonzero(ids == a).flatten()
        off = 0
        for i, o in enumerate(outs):
            flips = h_tie_flips(x[rows], was[i][a, 0].cpu(), scale, dtype)
            slack[rows, off:off + o] += (flips @ wbs[i][a, 0].cpu().double().abs().T).float()
            off += o
    ref = v1_ops.add_lora_linear(y0, x, cpu(was), cpu(wbs), cpu(bias), scale, outs, ids)
    assert_close(y, ref, f"add_lora_linear seed {seed}", slack=slack)
    # V1's two-op form on the same step: the fp32 buffer, then the expand into
    # windows from offset_start.
    buf = torch.zeros(n, T, r, device="cuda")
    wrapper.add_shrink(buf, x.cuda(), was, scale)
    torch.cuda.synchronize()
    buf_ref = v1_ops.lora_shrink(torch.zeros(n, T, r), x, cpu(was), scale, ids)
    assert_close(buf, buf_ref, f"add_shrink seed {seed}", rtol=1e-4, atol=1e-4)
    z0 = randn((T, off0 + sum(outs) + 8), 6003 + 10 * seed, dtype)
    z = z0.cuda()
    wrapper.add_expand(z, buf, wbs, bias, outs, offset_start=off0)
    torch.cuda.synchronize()
    zref = v1_ops.lora_expand(v1_ops.apply_bias(z0, cpu(bias), outs, ids, off0), buf.cpu(), cpu(wbs), outs, ids, off0)
    assert_close(z, zref, f"add_expand seed {seed}")
    assert wrapper.calls == ["update_metadata"], wrapper.calls
    assert pw._engine.device_errors() == 0
