"""Draft-model integration (adapterslotsplusplus_amd.lora_linear) on the GPU.

Mirrors the reference's BGMVLoRALinear use (benchmarks/e2e/
serve_multitenant.py:56-87) inside a graph-captured fixed-shape step
(benchmarks/e2e/batched_spec_loop.py:69-131): a small two-layer model whose
q/v projections carry K per-tenant adapters, one adapter id per token.

Reference: the same model in torch with the engine's rounding points -- the
base linear as F.linear computes it, H = rn(scale * x . A^T) (fp32
accumulate), y = rn(base + H . B^T) -- so the comparison holds at the
north-star tolerance layer after layer."""
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from adapterslotsplusplus_amd import WarpPipeEngine
from adapterslotsplusplus_amd.lora_linear import CapturedStep, DraftLoRAContext, wrap_linears
from tests.helpers import announce, assert_close, randn

pytestmark = pytest.mark.gpu

HID, RANK, K, B_, S_ = 512, 16, 6, 8, 4
T = B_ * S_
DT = torch.bfloat16


class Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.q_proj = nn.Linear(HID, HID, bias=False)
        self.v_proj = nn.Linear(HID, HID, bias=True)
        self.o_proj = nn.Linear(HID, HID, bias=False)

    def forward(self, x):
        return x + self.o_proj(F.silu(self.q_proj(x)) * self.v_proj(x))


class Tiny(nn.Module):
    def __init__(self):
        super().__init__()
        self.layers = nn.ModuleList([Block(), Block()])

    def forward(self, x):
        for blk in self.layers:
            x = blk(x)
        return x


def make_model(seed):
    torch.manual_seed(seed)
    m = Tiny()
    for p in m.parameters():
        with torch.no_grad():
            p.copy_(torch.randn(p.shape) * 0.04)
    return m.to(device="cuda", dtype=DT).eval()


def lora_weights(seed):
    w = {}
    for li in range(2):
        for name in ("q_proj", "v_proj"):
            A = randn((K, RANK, HID), seed + 10 * li + (0 if name == "q_proj" else 5), DT, 0.05).cuda()
            B = randn((K, HID, RANK), seed + 10 * li + (1 if name == "q_proj" else 6), DT, 0.05).cuda()
            w[f"layers.{li}.{name}"] = (A, B)
    return w


def ref_forward(model, weights, x, idx, scale):
    """The model with each wrapped linear computed in torch (fp32 math,
    the engine's two rounding points)."""
    def lin(name, mod, h):
        y = F.linear(h, mod.weight, mod.bias)
        if name not in weights:
            return y
        A, B = weights[name]
        h2 = h.reshape(-1, HID).float()
        ok = (idx >= 0)
        ii = idx.clamp(min=0)
        Hr = torch.einsum("ti,tri->tr", h2, A.float()[ii]) * scale
        Hr = Hr.to(DT).float()
        delta = torch.einsum("tr,tor->to", Hr, B.float()[ii])
        out = (y.reshape(-1, HID).float() + delta).to(DT)
        out = torch.where(ok[:, None], out, y.reshape(-1, HID))
        return out.reshape(y.shape)

    for li, blk in enumerate(model.layers):
        q = lin(f"layers.{li}.q_proj", blk.q_proj, x)
        v = lin(f"layers.{li}.v_proj", blk.v_proj, x)
        x = x + F.linear(F.silu(q) * v, blk.o_proj.weight, blk.o_proj.bias)
    return x


def routing(seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-1, K, (T,), generator=g).cuda()


def test_wrapped_linears_eager_and_captured():
    announce("lora_linear eager + graph")
    engine = WarpPipeEngine()
    model = make_model(1)
    ref_model = make_model(1)
    weights = lora_weights(200)
    ctx = DraftLoRAContext(engine, T, scale=2.0)
    names = wrap_linears(model, weights, ctx)
    assert sorted(names) == sorted(weights)

    x = randn((B_, S_, HID), 3, DT, 1.0).cuda()
    with torch.inference_mode():
        r1 = routing(7)
        ctx.set_routing(r1)
        ctx.begin_step()
        out = model(x)
        torch.cuda.synchronize()
        assert_close(out, ref_forward(ref_model, weights, x, r1, 2.0), "eager")

        x_static = x.clone()
        step = CapturedStep(lambda: model(x_static), ctx)
        for n, seed in enumerate((11, 12, 7)):
            r = routing(seed)
            x_new = randn((B_, S_, HID), 20 + n, DT, 1.0).cuda()
            x_static.copy_(x_new)
            got = step.replay(r).clone()
            torch.cuda.synchronize()
            assert_close(got, ref_forward(ref_model, weights, x_new, r, 2.0), f"replay {n}")
    assert engine.device_errors() == 0


def test_mode_none_is_base_only():
    announce("lora_linear mode none")
    engine = WarpPipeEngine()
    model = make_model(2)
    base = make_model(2)
    ctx = DraftLoRAContext(engine, T, scale=2.0)
    wrap_linears(model, lora_weights(300), ctx)
    ctx.mode = "none"
    x = randn((B_, S_, HID), 4, DT, 1.0).cuda()
    with torch.inference_mode():
        ctx.begin_step()
        out = model(x)
        torch.cuda.synchronize()
        assert torch.equal(out, base(x))


def test_row_count_must_match_routing():
    engine = WarpPipeEngine()
    model = make_model(3)
    ctx = DraftLoRAContext(engine, T, scale=2.0)
    wrap_linears(model, lora_weights(400), ctx)
    ctx.set_routing(routing(1))
    ctx.begin_step()
    with torch.inference_mode(), pytest.raises(RuntimeError, match="routing covers"):
        model(randn((B_, S_ + 1, HID), 5, DT, 1.0).cuda())
