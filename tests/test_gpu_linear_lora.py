"""GPU: linear_lora -- a base linear and its per-token LoRA delta in one launch
(wp_linear_lora).  Reference: the base linear in torch fp32 on the CPU,
rounded to the I/O type as the base linear's output is, then the oracle's
add_lora on it (oracle.bgmv.add_lora: rn(y + rn(scale . x . A^T) . B^T) per
segment of the build_seg_bounds table), on the same seeded inputs."""
import numpy as np
import pytest
import torch

from adapterslotsplusplus_amd import WarpPipeEngine
from oracle import bgmv
from oracle import segments as so
from tests.helpers import announce, randn, seeds

pytestmark = pytest.mark.gpu


def make(T, d_in, d_out, L, rank, dtype, seed, bias=True, idx=None):
    if idx is None:
        idx = torch.from_numpy(np.random.default_rng(seed).integers(-1, L, size=T))
    x = randn((T, d_in), seed + 1, dtype)
    W = randn((d_out, d_in), seed + 2, dtype, 0.02)
    b = randn((d_out,), seed + 3, dtype, 0.1) if bias else None
    wa = randn((L, 1, rank, d_in), seed + 4, dtype, 0.02)
    wb = randn((L, 1, d_out, rank), seed + 5, dtype, 0.02)
    return idx, x, W, b, wa, wb


def reference(idx, x, W, b, wa, wb, scale):
    """(y_ref, base_ref): the oracle's add_lora on the base output rounded to
    the I/O type."""
    base = x.float() @ W.float().T
    if b is not None:
        base = base + b.float()
    segs = so.seg_bounds(idx.tolist()).tolist()
    base = base.to(x.dtype)
    return bgmv.add_lora(base, x, wa, wb, scale, segs), base


def check(y, refs, what):
    """The tolerance of the LoRA path (rtol 1e-2, atol 1e-3), plus one unit in
    the last place of the base output: the base is rounded to the I/O type
    before the delta is added (as the base linear's output is), and an fp32
    sum over K in another order (ours vs the CPU's) can land on the other
    side of that rounding when the base sits on a boundary."""
    ref, base = refs
    d = y.float().cpu()
    r = ref.float()
    bb = base.float().abs()
    mant = 7 if base.dtype == torch.bfloat16 else 10
    ulp = torch.where(bb > 0, torch.exp2(torch.floor(torch.log2(bb.clamp_min(1e-30))) - mant), torch.zeros_like(bb))
    err = (d - r).abs()
    bad = err > 1e-3 + 1e-2 * r.abs() + ulp
    assert torch.isfinite(d).all(), f"{what}: non-finite values"
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.numel()} elements out of tolerance; max abs err "
                           f"{float(err.max()):.4g}")


def run(engine, idx, x, W, b, wa, wb, scale):
    assert engine.build_seg_bounds(idx.cuda())
    y = engine.linear_lora(x.cuda(), W.cuda(), b.cuda() if b is not None else None, wa.cuda(), wb.cuda(), scale)
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bias", [True, False])
def test_draft_shape(dtype, bias):
    """The draft step's projection: T=128 (32 tenants x 4), h=2048, r=32."""
    announce(f"linear_lora draft shape {dtype} bias={bias}")
    T, h, L, r = 128, 2048, 32, 32
    idx = torch.repeat_interleave(torch.randperm(L, generator=torch.Generator().manual_seed(3)), 4)
    idx, x, W, b, wa, wb = make(T, h, h, L, r, dtype, 10, bias, idx)
    engine = WarpPipeEngine()
    y = run(engine, idx, x, W, b, wa, wb, 2.0)
    assert y is not None
    check(y, reference(idx, x, W, b, wa, wb, 2.0), "draft shape")
    assert engine.device_errors() == 0


@pytest.mark.parametrize("case", seeds(10))
def test_random_shapes_one_engine(case):
    """Seeded shapes across token groups (T up to 512), K-splits, ranks and
    dtypes, ids -1 among them; one engine for all calls of a case (the
    counters and flags are back to zero between calls)."""
    rng = np.random.default_rng(100 + case)
    engine = WarpPipeEngine()
    for call in range(3):
        T = int(rng.choice([1, 17, 100, 128, 129, 256, 300, 512]))
        d_in = int(rng.choice([128, 384, 1024, 2048, 4096]))
        d_out = int(rng.choice([16, 48, 528, 2048, 4096]))
        rank = int(rng.choice([8, 16, 32, 64]))
        L = int(rng.integers(1, 40))
        dtype = torch.bfloat16 if rng.integers(2) else torch.float16
        bias = bool(rng.integers(2))
        announce(f"linear_lora case {case}.{call}: T={T} d_in={d_in} d_out={d_out} r={rank} L={L} {dtype} bias={bias}")
        idx, x, W, b, wa, wb = make(T, d_in, d_out, L, rank, dtype, 1000 * case + 10 * call, bias)
        y = run(engine, idx, x, W, b, wa, wb, 0.5)
        assert y is not None
        check(y, reference(idx, x, W, b, wa, wb, 0.5), f"case {case}.{call}")
    assert engine.device_errors() == 0


def test_captured_replays_follow_routing():
    """build_seg_bounds + three linear_lora calls captured once; replays with
    other routings (eager work between them) each match the reference."""
    T, h, L, r = 96, 1024, 12, 16
    dtype = torch.bfloat16
    engine = WarpPipeEngine()
    idx0, x, W, b, wa, wb = make(T, h, h, L, r, dtype, 77)
    routings = [torch.from_numpy(np.random.default_rng(s).integers(-1, L, size=T)) for s in range(3)]
    xd, Wd, bd, wad, wbd = x.cuda(), W.cuda(), b.cuda(), wa.cuda(), wb.cuda()
    idx_buf = routings[0].cuda()
    outs = [torch.empty(T, h, dtype=dtype, device="cuda") for _ in range(3)]

    def step():
        engine.build_seg_bounds(idx_buf)
        for o in outs:
            engine.linear_lora(xd, Wd, bd, wad, wbd, 1.5, out=o)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    announce("linear_lora graph capture")
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    for it, k in enumerate([1, 2, 0, 1]):
        announce(f"linear_lora graph replay {it}")
        idx_buf.copy_(routings[k])
        for o in outs:
            o.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        ref = reference(routings[k], x, W, b, wa, wb, 1.5)
        for o in outs:
            check(o, ref, f"replay {it}")
        _ = (xd.float() * 2).sum().item()
    assert engine.device_errors() == 0


def test_not_handled_shapes_and_checks():
    engine = WarpPipeEngine()
    announce("linear_lora shapes without kernels")
    idx, x, W, b, wa, wb = make(64, 200, 256, 4, 16, torch.bfloat16, 5)
    assert engine.build_seg_bounds(idx.cuda())
    # d_in not a multiple of 128: the caller runs the linear and add_lora.
    assert engine.linear_lora(x.cuda(), W.cuda(), b.cuda(), wa.cuda(), wb.cuda(), 1.0) is None
    # A rank without kernels.
    idx, x, W, b, wa, wb = make(64, 256, 256, 4, 24, torch.bfloat16, 6)
    assert engine.build_seg_bounds(idx.cuda())
    assert engine.linear_lora(x.cuda(), W.cuda(), b.cuda(), wa.cuda(), wb.cuda(), 1.0) is None
    idx, x, W, b, wa, wb = make(64, 256, 256, 4, 16, torch.bfloat16, 7)
    with pytest.raises(RuntimeError, match="weight"):
        engine.linear_lora(x.cuda(), W[:, :128].cuda(), b.cuda(), wa.cuda(), wb.cuda(), 1.0)
    assert engine.device_errors() == 0
