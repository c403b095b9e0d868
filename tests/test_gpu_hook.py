"""GPU: the punica add_lora hook (reference lora_warp_pipe/punica_wrapper.py:119-159,
:219-238) driven end to end on the HIP kernels.

A duck-typed PunicaWrapper stands in for vLLM / AdapterSlots' wrapper (absent
in the reference checkout and here).  Its own add_lora is the stock path
(shrink into an fp32 buffer, then expand, as vLLM 0.6.3's PunicaWrapper does)
and records every call, so a test can tell which path ran.  The live wrapper
is switched with install_warp_pipe_add_lora and AS_WARP_PIPE=1; kernel-path
outputs are checked against the CPU oracle, fallback outputs against the
stock formula.  The capture case mirrors
tests/correctness/test_warp_pipe_graph_capture.py:39-129: update_metadata runs
outside the graph, the captured add_lora calls read the table built for the
replay-time indices."""
import pytest
import torch

from adapterslotsplusplus_amd import WarpPipeConfig, WarpPipeEngine
from adapterslotsplusplus_amd import punica_wrapper as pw
from oracle import bgmv
from oracle import segments as so
from tests.helpers import announce, assert_close, randn

pytestmark = pytest.mark.gpu


class FakePunica:
    """PunicaWrapper stand-in: token_lora_indices, is_prefill, update_metadata
    and the stock add_lora (fp32 buffer between shrink and expand)."""

    def __init__(self, indices: torch.Tensor):
        self.token_lora_indices = indices
        self.is_prefill = False
        self.calls = []

    def update_metadata(self, mapping, lora_index_to_id, max_loras, vocab_size, extra_vocab_size,
                        long_lora_context=None):
        self.calls.append("update_metadata")

    def add_lora(self, y, x, wa_t_all, wb_t_all, scale, y_offset=None, y_slice_size=None, *, buffer=None):
        self.calls.append(("stock", y_offset, y_slice_size))
        stock_add_lora(y, x, wa_t_all, wb_t_all, scale, self.token_lora_indices, y_offset, y_slice_size)


def stock_add_lora(y, x, wa, wb, scale, idx, y_offset=None, y_slice_size=None):
    """The stock path's formula: fp32 H (no rounding), one rounding of y."""
    y2 = y.view(-1, y.shape[-1])
    x2 = x.view(-1, x.shape[-1]).float()
    off = int(y_offset or 0)
    o = int(wb.size(-2)) if y_slice_size is None else int(y_slice_size)
    for t in range(x2.shape[0]):
        i = int(idx[t])
        if i < 0:
            continue
        h = (x2[t] @ wa[i, 0].float().T) * scale
        y2[t, off:off + o] = (y2[t, off:off + o].float() + h @ wb[i, 0].float().T).to(y.dtype)


class FakeManager:
    def __init__(self, wrapper):
        class AdapterManager:
            pass

        self._adapter_manager = AdapterManager()
        self._adapter_manager.punica_wrapper = wrapper


@pytest.fixture
def hook(monkeypatch):
    """A switched wrapper over a fresh process engine, AS_WARP_PIPE=1."""
    monkeypatch.setenv("AS_WARP_PIPE", "1")
    monkeypatch.setattr(pw, "_engine", WarpPipeEngine())

    def make(indices):
        w = FakePunica(indices)
        assert pw.install_warp_pipe_add_lora(FakeManager(w))
        assert isinstance(w, pw.WarpPipeAddLoraMixin)
        return w

    return make


def weights(L, rank, d, o, seed, dtype=torch.bfloat16):
    return randn((L, 1, rank, d), seed, dtype, 0.02), randn((L, 1, o, rank), seed + 1, dtype, 0.02)


def test_hook_step_on_kernels(hook):
    """update_metadata builds the table; four add_lora calls with their own
    weights (one into a column window of a wider y) run on the kernels; a
    rank-24 call reaches the stock path."""
    T, L, d = 96, 6, 1024
    g = torch.Generator().manual_seed(3)
    idx = torch.randint(-1, L, (T,), generator=g)
    w = hook(idx.cuda())
    w.update_metadata(None, None, L, 0, 0)
    assert w._wp_step_ok
    segs = so.seg_bounds(idx.tolist()).tolist()
    x = randn((T, d), 10, torch.bfloat16)
    xd = x.cuda()
    for k, (rank, o, off, width) in enumerate([(32, 1024, None, None), (16, 512, None, None),
                                               (64, 768, None, None), (32, 256, 512, 1280)]):
        announce(f"hook add_lora call {k}: r={rank} o={o} y_offset={off} width={width}")
        wa, wb = weights(L, rank, d, o, 20 + k)
        y0 = randn((T, width or o), 30 + k, torch.bfloat16)
        y = y0.cuda()
        n_before = len(w.calls)
        w.add_lora(y, xd, wa.cuda(), wb.cuda(), 0.5, off, o if off is not None else None)
        torch.cuda.synchronize()
        assert len(w.calls) == n_before, f"call {k} fell back to the stock path"
        assert_close(y, bgmv.add_lora(y0, x, wa, wb, 0.5, segs, off or 0), f"hook call {k}")
    announce("hook add_lora rank 24 -> stock path")
    wa, wb = weights(L, 24, d, 256, 40)
    y0 = randn((T, 256), 41, torch.bfloat16)
    y = y0.cuda()
    w.add_lora(y, xd, wa.cuda(), wb.cuda(), 0.5)
    torch.cuda.synchronize()
    assert w.calls[-1] == ("stock", None, None)
    ref = y0.clone()
    stock_add_lora(ref, x, wa, wb, 0.5, idx)
    assert_close(y, ref, "rank-24 stock call")
    assert pw._get_engine().device_errors() == 0


def test_hook_over_capacity_step_falls_back(hook, monkeypatch):
    """A step with more tokens than the engine takes: build_seg_bounds returns
    False in update_metadata, and every add_lora of that step takes the stock
    path (the reference would reuse the previous step's table, Appendix B 3);
    the next step that fits runs on the kernels again."""
    monkeypatch.setattr(pw, "_engine", WarpPipeEngine(WarpPipeConfig(max_tokens=64)))
    L, d, o, rank = 4, 512, 256, 32
    wa, wb = weights(L, rank, d, o, 50)
    wad, wbd = wa.cuda(), wb.cuda()
    g = torch.Generator().manual_seed(4)
    for T, on_kernels in [(48, True), (80, False), (64, True)]:
        announce(f"hook step T={T} (max_tokens 64)")
        idx = torch.randint(-1, L, (T,), generator=g)
        w = hook(idx.cuda())
        w.update_metadata(None, None, L, 0, 0)
        assert w._wp_step_ok == on_kernels
        x = randn((T, d), 60 + T, torch.bfloat16)
        y0 = randn((T, o), 61 + T, torch.bfloat16)
        y = y0.cuda()
        w.add_lora(y, x.cuda(), wad, wbd, 0.25)
        torch.cuda.synchronize()
        if on_kernels:
            assert w.calls[-1] == "update_metadata"
            assert_close(y, bgmv.add_lora(y0, x, wa, wb, 0.25, so.seg_bounds(idx.tolist()).tolist()), f"T={T}")
        else:
            assert w.calls[-1] == ("stock", None, None)
            ref = y0.clone()
            stock_add_lora(ref, x, wa, wb, 0.25, idx)
            assert_close(y, ref, f"T={T} stock step")


def test_hook_captured_add_lora_replays_new_indices(hook):
    """test_warp_pipe_graph_capture.py:39-129 through the hook: add_lora calls
    captured once; update_metadata (outside the graph) with other indices
    before each replay; every replay matches the oracle for the replay-time
    indices, and differs from the capture-time result."""
    T, L, d, o, rank = 16, 8, 4096, 4096, 32
    capture_idx = [0, 0, 0, 0, 1, 1, 1, 1, -1, -1, 2, 2, 2, 2, 2, 2]
    replay_idx = [3, 3, 5, 5, 5, 5, 5, 5, 5, 5, 5, 5, 5, 5, -1, 6]
    idx_buf = torch.tensor(capture_idx, dtype=torch.int64, device="cuda")
    w = hook(idx_buf)
    wa1, wb1 = weights(L, rank, d, o, 70, torch.float16)
    wa2, wb2 = weights(L, rank, d, o, 72, torch.float16)
    x = randn((T, d), 74, torch.float16, 0.1)
    y0 = randn((T, o), 75, torch.float16, 0.1)
    xd, y1, y2 = x.cuda(), y0.cuda(), y0.cuda()
    dev_w = [(wa1.cuda(), wb1.cuda()), (wa2.cuda(), wb2.cuda())]
    w.update_metadata(None, None, L, 0, 0)

    def step():
        w.add_lora(y1, xd, dev_w[0][0], dev_w[0][1], 0.5)
        w.add_lora(y2, xd, dev_w[1][0], dev_w[1][1], 0.5)

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    assert all(c == "update_metadata" for c in w.calls), "a captured call fell back"
    results = {}
    for name, ids in [("capture", capture_idx), ("replay", replay_idx), ("capture-again", capture_idx)]:
        announce(f"hook graph replay with {name} indices")
        idx_buf.copy_(torch.tensor(ids, dtype=torch.int64))
        w.update_metadata(None, None, L, 0, 0)
        y1.copy_(y0.cuda())
        y2.copy_(y0.cuda())
        graph.replay()
        torch.cuda.synchronize()
        segs = so.seg_bounds(ids).tolist()
        assert_close(y1, bgmv.add_lora(y0, x, wa1, wb1, 0.5, segs), f"{name} call 1")
        assert_close(y2, bgmv.add_lora(y0, x, wa2, wb2, 0.5, segs), f"{name} call 2")
        results[name] = y1.cpu().clone()
    assert not torch.equal(results["capture"], results["replay"]), "replay reproduced the capture-time routing"
    assert torch.equal(results["capture"], results["capture-again"])
    assert pw._get_engine().device_errors() == 0
