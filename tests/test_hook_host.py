"""Host logic of the punica add_lora hook (reference lora_warp_pipe/punica_wrapper.py),
exercised with a duck-typed wrapper on CPU tensors: every case here must take
the stock fallback path without touching the engine."""
import pytest
import torch

from adapterslotsplusplus_amd import punica_wrapper as pw


class FakePunica:
    """Stands in for vLLM / AdapterSlots' PunicaWrapper (absent here)."""

    def __init__(self, indices, is_prefill=False):
        self.token_lora_indices = indices
        self.is_prefill = is_prefill
        self.calls = []

    def update_metadata(self, mapping, lora_index_to_id, max_loras, vocab_size, extra_vocab_size,
                        long_lora_context=None):
        self.calls.append("update_metadata")

    def add_lora(self, y, x, wa_t_all, wb_t_all, scale, y_offset=None, y_slice_size=None, *, buffer=None):
        self.calls.append(("add_lora", y_offset, y_slice_size))
        y += (x @ wa_t_all[0, 0].T * scale) @ wb_t_all[0, 0].T


class FakeManager:
    def __init__(self, wrapper):
        class AM:
            pass
        self._adapter_manager = AM()
        self._adapter_manager.punica_wrapper = wrapper


def test_install_switches_class_once():
    w = FakePunica(torch.zeros(4, dtype=torch.int64))
    mgr = FakeManager(w)
    assert pw.install_warp_pipe_add_lora(mgr) is True
    assert isinstance(w, pw.WarpPipeAddLoraMixin) and isinstance(w, FakePunica)
    assert pw.install_warp_pipe_add_lora(mgr) is False  # already switched
    assert pw.install_warp_pipe_add_lora(None) is False


def test_install_without_wrapper_is_noop():
    class Empty:
        _adapter_manager = None
    assert pw.install_warp_pipe_add_lora(Empty()) is False


def test_disabled_env_falls_back(monkeypatch):
    monkeypatch.setenv("AS_WARP_PIPE", "0")
    w = FakePunica(torch.zeros(4, dtype=torch.int64))
    w.__class__ = pw.warp_pipe_class_for(FakePunica)
    w.update_metadata(None, None, 1, 0, 0)
    x = torch.randn(4, 8)
    y = torch.zeros(4, 6)
    wa = torch.randn(1, 1, 32, 8)
    wb = torch.randn(1, 1, 6, 32)
    w.add_lora(y, x, wa, wb, 0.5)
    assert w.calls == ["update_metadata", ("add_lora", None, None)]
    assert torch.allclose(y, (x @ wa[0, 0].T * 0.5) @ wb[0, 0].T)


def test_cpu_tensors_fall_back_even_when_enabled(monkeypatch):
    monkeypatch.setenv("AS_WARP_PIPE", "1")
    w = FakePunica(torch.zeros(4, dtype=torch.int64), is_prefill=True)
    w.__class__ = pw.warp_pipe_class_for(FakePunica)
    w.update_metadata(None, None, 1, 0, 0)  # prefill: no build_seg_bounds
    x = torch.randn(4, 8)
    y = torch.zeros(4, 6)
    w.add_lora(y, x, torch.randn(1, 1, 32, 8), torch.randn(1, 1, 6, 32), 1.0, 0, 6)
    assert w.calls[-1] == ("add_lora", 0, 6)


class _StubEngine:
    """Engine stand-in whose polls return queued error words."""

    def __init__(self, words):
        self.words = list(words)
        self.polls = 0
        self.built = []

    def poll_device_errors(self):
        self.polls += 1
        return self.words.pop(0) if self.words else 0

    def build_seg_bounds(self, idx):
        self.built.append(int(idx.numel()))
        return True


def test_update_metadata_reports_polled_errors(monkeypatch, caplog):
    """Decode steps poll the engine's error word before building the table;
    nonzero words are logged and ORed into device_errors_seen, and raise with
    AS_WARP_PIPE_STRICT=1."""
    monkeypatch.setenv("AS_WARP_PIPE", "1")
    monkeypatch.setattr(pw, "_WARP_PIPE_IMPORT_OK", True)
    stub = _StubEngine([0, 2, 0, 9])
    monkeypatch.setattr(pw, "_engine", stub)
    monkeypatch.setattr(pw, "device_errors_seen", 0)
    w = FakePunica(torch.zeros(4, dtype=torch.int64))
    w.__class__ = pw.warp_pipe_class_for(FakePunica)
    with caplog.at_level("WARNING"):
        for _ in range(3):
            w.update_metadata(None, None, 1, 0, 0)
    assert stub.polls == 3 and stub.built == [4, 4, 4]
    assert pw.device_errors_seen == 2
    assert "not registered" in caplog.text
    monkeypatch.setenv("AS_WARP_PIPE_STRICT", "1")
    with pytest.raises(RuntimeError, match="0x9"):
        w.update_metadata(None, None, 1, 0, 0)
    assert pw.device_errors_seen == 11
    # Prefill steps neither poll nor build.
    w.is_prefill = True
    w.update_metadata(None, None, 1, 0, 0)
    assert stub.polls == 4


def test_describe_device_errors():
    assert pw.describe_device_errors(0) == "none"
    assert pw.describe_device_errors(1 | 16) == ("adapter id outside the stacked weights, "
                                                 "more adapter blocks than the call's grid")


def test_draft_context_polls_outside_capture(monkeypatch):
    from adapterslotsplusplus_amd import lora_linear as ll

    stub = _StubEngine([4, 0])
    ctx = ll.DraftLoRAContext.__new__(ll.DraftLoRAContext)
    ctx.engine, ctx.tokens, ctx.mode, ctx.device_errors = stub, 4, "lora", 0
    ctx.idx = torch.zeros(4, dtype=torch.int64)
    monkeypatch.setattr(pw, "device_errors_seen", 0)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    ctx.begin_step()
    ctx.begin_step()
    assert stub.polls == 2 and stub.built == [4, 4] and ctx.device_errors == 4
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    ctx.begin_step()  # inside capture: builds, does not poll
    assert stub.polls == 2 and stub.built == [4, 4, 4]


class FakeV1:
    """V1 PunicaWrapperGPU stand-in on the CPU: records which parent methods ran."""

    def __init__(self, idx):
        self._idx = idx
        self.is_prefill = False
        self.calls = []

    @property
    def token_lora_indices(self):
        return self._idx

    def update_metadata(self, mapping, lora_index_to_id, max_loras, vocab_size, extra_vocab_size, **kwargs):
        self.calls.append("update_metadata")

    def add_shrink(self, y, x, lora_a_stacked, scale, **kwargs):
        self.calls.append("add_shrink")

    def add_expand(self, y, x, lora_b_stacked, lora_bias_stacked, output_slices, offset_start=0, add_inputs=True,
                   **kwargs):
        self.calls.append("add_expand")

    def add_lora_embedding(self, y, x, lora_b_stacked, add_inputs=True, **kwargs):
        self.calls.append("add_lora_embedding")

    def add_lora_linear(self, y, x, lora_a_stacked, lora_b_stacked, lora_bias_stacked, scale, output_slices, *,
                        buffer=None, **kwargs):
        self.calls.append("add_lora_linear")


def _v1_calls(w):
    x = torch.randn(4, 8)
    wa = (torch.randn(2, 1, 16, 8),)
    wb = (torch.randn(2, 1, 6, 16),)
    w.add_shrink(torch.zeros(1, 4, 16), x, wa, 1.0)
    w.add_expand(torch.zeros(4, 6), torch.zeros(1, 4, 16), wb, None, (6,))
    w.add_lora_embedding(torch.zeros(4, 6), torch.zeros(4, 16), wb[0])
    w.add_lora_linear(torch.zeros(4, 6), x, wa, wb, None, 1.0, (6,))


@pytest.mark.parametrize("enabled", ["0", "1"])
def test_v1_mixin_falls_back_without_the_engine(monkeypatch, enabled):
    """AS_WARP_PIPE unset, or CPU tensors: every V1 op runs the parent's."""
    from adapterslotsplusplus_amd import punica_v1 as v1

    monkeypatch.setenv("AS_WARP_PIPE", enabled)
    monkeypatch.setattr(pw, "_engine", _StubEngine([]))
    monkeypatch.setattr(pw, "_WARP_PIPE_IMPORT_OK", True)
    monkeypatch.setattr(v1, "_WARP_PIPE_IMPORT_OK", True)
    w = FakeV1(torch.zeros(4, dtype=torch.int64))
    assert v1.install_warp_pipe_v1(FakeManager(w))
    assert isinstance(w, v1.WarpPipeV1Mixin) and not v1.install_warp_pipe_v1(FakeManager(w))
    w.update_metadata(None, None, 2, 0, 0)
    _v1_calls(w)
    assert w.calls == ["update_metadata", "add_shrink", "add_expand", "add_lora_embedding", "add_lora_linear"]
    assert v1.install_warp_pipe_v1(None) is False
