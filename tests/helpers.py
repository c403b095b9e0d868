"""Shared helpers of the GPU parity tests."""
import os
import sys

import torch

# Tolerance of the north star: bf16/fp16 I/O with fp32 accumulation.
RTOL = 1e-2
ATOL = 1e-3


def seeds(default: int) -> range:
    """Seeds of a randomized parity test: `default` of them, or
    WP_TEST_SEEDS (for a wider sweep, e.g. WP_TEST_SEEDS=200 python -m pytest
    tests -m gpu -k random)."""
    return range(int(os.environ.get("WP_TEST_SEEDS", default)))


def announce(msg: str) -> None:
    """Names the case before a GPU step, flushed, so a failure is attributable."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def assert_close(dev: torch.Tensor, ref: torch.Tensor, what: str = "", rtol: float = RTOL, atol: float = ATOL,
                 slack: torch.Tensor = None):
    """|dev - ref| <= atol + rtol |ref| (+ slack, per element, where given)."""
    d = dev.detach().float().cpu()
    r = ref.detach().float().cpu()
    assert d.shape == r.shape, f"{what}: shape {tuple(d.shape)} vs {tuple(r.shape)}"
    assert torch.isfinite(d).all(), f"{what}: non-finite values"
    err = (d - r).abs()
    bound = atol + rtol * r.abs()
    if slack is not None:
        bound = bound + slack
    bad = err > bound
    if bad.any():
        i = int(torch.nonzero(bad.flatten())[0])
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.numel()} elements out of tolerance; first at flat index {i}: "
            f"dev={d.flatten()[i].item():.6g} ref={r.flatten()[i].item():.6g}; max abs err {err.max().item():.3g}")


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(int(seed))


def randn(shape, seed, dtype, std=1.0):
    return (torch.randn(*shape, generator=gen(seed)) * std).to(dtype)


def h_tie_flips(x: torch.Tensor, a: torch.Tensor, scale: float, dtype) -> torch.Tensor:
    """Per element of H = rn(scale * x @ a^T) (rn: rounding to `dtype`), the
    size of the one-ulp step its rounding may take either way: nonzero only
    where the exact value lies within fp32 summation error of a rounding
    midpoint.  Any fp32 summation order is a valid H, so the device and the
    oracle may round such an element to different neighbours.  The window is
    eight standard deviations of a length-d fp32 sum's rounding error taken as
    a random walk, 8 * 2^-24 * sqrt(d) * ||terms||_2 (the worst-case bound,
    d * 2^-24 * sum |terms|, is as wide as a bf16 step of H at d ~ 2000 and
    would excuse almost every element)."""
    x64, a64 = x.double(), a.double()
    h = scale * (x64 @ a64.T)
    win = 8.0 * 2.0 ** -24 * x.shape[1] ** 0.5 * abs(scale) * ((x64 * x64) @ (a64 * a64).T).sqrt()
    lo = (h - win).float().to(dtype).double()
    hi = (h + win).float().to(dtype).double()
    return (hi - lo).abs()
