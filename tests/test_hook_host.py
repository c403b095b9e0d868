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
