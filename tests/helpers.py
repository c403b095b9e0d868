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


def assert_close(dev: torch.Tensor, ref: torch.Tensor, what: str = "", rtol: float = RTOL, atol: float = ATOL):
    d = dev.detach().float().cpu()
    r = ref.detach().float().cpu()
    assert d.shape == r.shape, f"{what}: shape {tuple(d.shape)} vs {tuple(r.shape)}"
    assert torch.isfinite(d).all(), f"{what}: non-finite values"
    err = (d - r).abs()
    bound = atol + rtol * r.abs()
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
