"""Host-side checks of the draft-model wrapper (no GPU): shape validation
and module replacement."""
import pytest
import torch
import torch.nn as nn

from adapterslotsplusplus_amd.lora_linear import WarpPipeLoRALinear, wrap_linears


class _Ctx:
    mode = "none"
    tokens = 4


def test_shapes_are_checked():
    base = nn.Linear(64, 32)
    ctx = _Ctx()
    WarpPipeLoRALinear(base, torch.zeros(3, 8, 64), torch.zeros(3, 32, 8), ctx)
    with pytest.raises(RuntimeError, match=r"\[K, rank, in\]"):
        WarpPipeLoRALinear(base, torch.zeros(3, 8, 64), torch.zeros(2, 32, 8), ctx)
    with pytest.raises(RuntimeError, match="do not match"):
        WarpPipeLoRALinear(base, torch.zeros(3, 8, 48), torch.zeros(3, 32, 8), ctx)


def test_wrap_replaces_named_linears_and_mode_none_is_base():
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(64, 64), nn.ReLU(), nn.Linear(64, 32))
    x = torch.randn(4, 64)
    ref = model(x)
    ctx = _Ctx()
    done = wrap_linears(model, {"0": (torch.zeros(2, 8, 64), torch.zeros(2, 64, 8))}, ctx)
    assert list(done) == ["0"]
    assert isinstance(model[0], WarpPipeLoRALinear) and isinstance(model[2], nn.Linear)
    assert torch.equal(model(x), ref)
    with pytest.raises(RuntimeError, match="not an nn.Linear"):
        wrap_linears(model, {"1": (torch.zeros(2, 8, 64), torch.zeros(2, 64, 8))}, ctx)
