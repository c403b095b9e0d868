"""torch fp32 CPU restatement of vLLM V1's LoRA ops -- TEST INFRASTRUCTURE ONLY
(the checker of the engine's V1 op surface, never the thing measured or
shipped).

vLLM is an absent dependency here (the reference pins vllm==0.6.3.post1,
requirements.txt:13, and benchmarks against V1, benchmarks/sota/versions.txt:18-19;
its hook scopes the V1 ops out, lora_warp_pipe/punica_wrapper.py:8-16).  The
restated behaviour is that of V1's PunicaWrapperGPU and its grouped Triton ops
as published in vLLM's source:

  _apply_bias     y[t, window s] += bias[s][id_t] in y's dtype (rows with id -1
                  get 0, i.e. stay as they are);
  lora_shrink     y[s][t, :r] += scale * (x[t] . A_s[id_t]^T), fp32 accumulate,
                  fp32 output buffer (add_shrink);
  lora_expand     y[t, off_s + o] = rn((add_inputs ? y : 0) + rn_w(x[s][t]) . B_s[id_t][o]^T):
                  an fp32 input is cast to the weights' dtype before the
                  product, accumulation is fp32, the output rounded once;
                  windows are consecutive from offset_start; rows with id -1
                  are not written (add_expand, add_lora_embedding);
  add_lora_linear _apply_bias, then lora_shrink into a zero fp32 buffer, then
                  lora_expand with add_inputs=True.

Parity pinning (tests/test_oracle_v1_ops.py): without biases add_lora_linear
equals oracle.bgmv.add_lora_nslice, itself pinned against a float64 brute
force; lora_shrink matches a float64 brute force to fp32 accuracy; bias-only
cases against a hand-computed sum on one-hot data; a planted mistake (the bias
added after the expand's rounding) is detected.
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch


def _groups(ids: torch.Tensor):
    """(adapter id, row indices) for every id >= 0 that occurs."""
    ids = ids.reshape(-1).to(torch.int64)
    for a in sorted(set(int(v) for v in ids.tolist() if v >= 0)):
        yield a, torch.nonzero(ids == a).flatten()


def apply_bias(y: torch.Tensor, biases: Optional[Sequence[Optional[torch.Tensor]]], output_slices: Sequence[int],
               ids: torch.Tensor, offset_start: int = 0) -> torch.Tensor:
    y = y.reshape(-1, y.shape[-1]).clone()
    if biases is None:
        return y
    off = int(offset_start)
    for b, o in zip(biases, output_slices):
        if b is not None:
            b2 = b.reshape(b.shape[0], -1)
            for a, rows in _groups(ids):
                y[rows, off:off + o] = (y[rows, off:off + o].float() + b2[a, :o].float()).to(y.dtype)
        off += int(o)
    return y


def lora_shrink(out: torch.Tensor, x: torch.Tensor, lora_a_stacked: Sequence[torch.Tensor], scale: float,
                ids: torch.Tensor) -> torch.Tensor:
    """out: fp32 [n, T, >= r]; returns the updated copy."""
    out = out.clone()
    x2 = x.reshape(-1, x.shape[-1])
    for s, A in enumerate(lora_a_stacked):
        for a, rows in _groups(ids):
            m = A[a].reshape(-1, A.shape[-1]).float()
            r = m.shape[0]
            out[s, rows, :r] += (x2[rows].float() @ m.T) * scale
    return out


def lora_expand(y: torch.Tensor, h: torch.Tensor, lora_b_stacked: Sequence[torch.Tensor], output_slices: Sequence[int],
                ids: torch.Tensor, offset_start: int = 0, add_inputs: bool = True) -> torch.Tensor:
    """h: [n, T, >= r] fp32 or y's dtype; returns the updated copy of y (2-D)."""
    y = y.reshape(-1, y.shape[-1]).clone()
    off = int(offset_start)
    for s, (B, o) in enumerate(zip(lora_b_stacked, output_slices)):
        hs = h[s].to(B.dtype)
        for a, rows in _groups(ids):
            m = B[a].reshape(-1, B.shape[-1]).float()
            r = m.shape[1]
            acc = hs[rows, :r].float() @ m.T
            if add_inputs:
                acc = acc + y[rows, off:off + o].float()
            y[rows, off:off + o] = acc.to(y.dtype)
        off += int(o)
    return y


def add_lora_linear(y: torch.Tensor, x: torch.Tensor, lora_a_stacked, lora_b_stacked, biases, scale: float,
                    output_slices: Sequence[int], ids: torch.Tensor) -> torch.Tensor:
    y = apply_bias(y, biases, output_slices, ids)
    r = max(int(b.shape[-1]) for b in lora_b_stacked)
    buf = torch.zeros(len(output_slices), y.shape[0], r, dtype=torch.float32)
    buf = lora_shrink(buf, x, lora_a_stacked, scale, ids)
    return lora_expand(y, buf, lora_b_stacked, output_slices, ids, 0, True)
