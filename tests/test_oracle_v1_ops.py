"""Pins the vLLM V1 LoRA-op oracle (oracle/v1_ops.py) on the CPU.

vLLM is not importable here, so the oracle is pinned by what fixes it
independently of its own formulas:
  * without biases, add_lora_linear must equal oracle.bgmv.add_lora_nslice
    (pinned against a float64 brute force in test_oracle_bgmv.py) on the
    segment table of the same routing;
  * lora_shrink against a float64 brute-force loop (fp32 accuracy);
  * biases on one-hot data: only the rows of adapters with a bias change,
    by exactly that adapter's row; rows with id -1 never change;
  * add_inputs=False overwrites exactly the routed rows' windows;
  * a planted mistake -- the bias added after the expand's rounding instead
    of before it -- is detected.
"""
import pytest
import torch

from oracle import bgmv
from oracle import segments as so
from oracle import v1_ops

DTYPES = [torch.float16, torch.bfloat16]


def case(seed, T, d, outs, r, L, dtype):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(-1, L, (T,), generator=g)
    x = torch.randn(T, d, generator=g).to(dtype)
    was = [(torch.randn(L, 1, r, d, generator=g) * 0.3).to(dtype) for _ in outs]
    wbs = [(torch.randn(L, 1, o, r, generator=g) * 0.3).to(dtype) for o in outs]
    y = torch.randn(T, sum(outs), generator=g).to(dtype)
    return ids, x, was, wbs, y


@pytest.mark.parametrize("dtype", DTYPES)
def test_add_lora_linear_without_bias_is_nslice(dtype):
    for seed in range(10):
        outs = [8, 4, 4]
        ids, x, was, wbs, y = case(seed, 9, 16, outs, 4, 3, dtype)
        got = v1_ops.add_lora_linear(y, x, was, wbs, None, 0.75, outs, ids)
        segs = so.seg_bounds(ids.tolist()).tolist()
        ref = bgmv.add_lora_nslice(y, x, was, wbs, 0.75, segs, [0, 8, 12])
        assert torch.equal(got, ref), f"seed {seed}"


def test_shrink_matches_float64_brute_force():
    for seed in range(6):
        ids, x, was, _, _ = case(seed, 7, 24, [8, 8], 4, 3, torch.bfloat16)
        out0 = torch.randn(2, 7, 8, generator=torch.Generator().manual_seed(99 + seed))
        got = v1_ops.lora_shrink(out0, x, was, 0.5, ids)
        ref = out0.double().clone()
        for s, A in enumerate(was):
            for t in range(7):
                a = int(ids[t])
                if a < 0:
                    continue
                for k in range(4):
                    ref[s, t, k] += 0.5 * sum(float(x[t, j]) * float(A[a, 0, k, j]) for j in range(24))
        assert torch.allclose(got.double(), ref, rtol=1e-6, atol=1e-6)
        # Columns past the rank and rows without an adapter keep their values.
        assert torch.equal(got[:, :, 4:], out0[:, :, 4:])
        assert torch.equal(got[:, ids < 0], out0[:, ids < 0])


@pytest.mark.parametrize("dtype", DTYPES)
def test_bias_one_hot(dtype):
    T, L = 6, 3
    ids = torch.tensor([0, 2, -1, 1, 2, 0])
    y = torch.zeros(T, 8, dtype=dtype)
    biases = [torch.arange(L * 4, dtype=torch.float32).reshape(L, 1, 4).to(dtype), None]
    got = v1_ops.apply_bias(y, biases, [4, 4], ids)
    for t in range(T):
        a = int(ids[t])
        want = biases[0][a, 0] if a >= 0 else torch.zeros(4, dtype=dtype)
        assert torch.equal(got[t, :4], want)
        assert torch.equal(got[t, 4:], torch.zeros(4, dtype=dtype))
    # offset_start shifts every window.
    got2 = v1_ops.apply_bias(torch.zeros(T, 10, dtype=dtype), biases, [4, 4], ids, offset_start=2)
    assert torch.equal(got2[:, 2:6], got[:, :4]) and torch.equal(got2[:, :2], torch.zeros(T, 2, dtype=dtype))


@pytest.mark.parametrize("dtype", DTYPES)
def test_expand_overwrite_touches_only_routed_rows(dtype):
    ids, x, _, wbs, y = case(3, 8, 16, [8], 4, 3, dtype)
    h = torch.randn(1, 8, 4, generator=torch.Generator().manual_seed(1))
    got = v1_ops.lora_expand(y, h, wbs, [8], ids, add_inputs=False)
    assert torch.equal(got[ids < 0], y[ids < 0])
    for t in range(8):
        a = int(ids[t])
        if a >= 0:
            want = (h[0, t].to(dtype).float() @ wbs[0][a, 0].float().T).to(dtype)
            assert torch.equal(got[t], want)


@pytest.mark.parametrize("dtype", DTYPES)
def test_bias_after_rounding_is_detected(dtype):
    """Planted mistake: bias added to the expand's rounded result rather than
    to y before the expand.  Some seed must tell the two apart."""
    diffs = 0
    for seed in range(20):
        outs = [8]
        ids, x, was, wbs, y = case(seed, 9, 16, outs, 4, 3, dtype)
        g = torch.Generator().manual_seed(500 + seed)
        biases = [(torch.randn(3, 1, 8, generator=g) * 3).to(dtype)]
        good = v1_ops.add_lora_linear(y, x, was, wbs, biases, 0.5, outs, ids)
        nb = v1_ops.add_lora_linear(y, x, was, wbs, None, 0.5, outs, ids)
        bad = v1_ops.apply_bias(nb, biases, outs, ids)
        diffs += int(not torch.equal(good, bad))
    assert diffs > 0
