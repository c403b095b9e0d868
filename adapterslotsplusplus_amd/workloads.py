"""Seeded synthetic workloads of the five benchmark configurations, and the
algorithmic-bytes model used for roofline figures.

Every tensor is drawn on the CPU with a seeded torch.Generator, so the GPU run
and the CPU oracle see identical bytes (the reference seeds the CUDA generator,
which is not reproducible across vendors).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import torch


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(int(seed))
    return g


def zipf_indices(T: int, n_adapters: int, s: float, seed: int) -> torch.Tensor:
    """T iid draws of adapter ids 0..n-1 with P(id = k-1) proportional to k^-s."""
    k = torch.arange(1, n_adapters + 1, dtype=torch.float64)
    p = k.pow(-s)
    p = p / p.sum()
    return torch.multinomial(p, T, replacement=True, generator=_gen(seed)).to(torch.int64)


def uniform_indices(T: int, n_adapters: int, seed: int) -> torch.Tensor:
    return torch.randint(0, n_adapters, (T,), generator=_gen(seed), dtype=torch.int64)


def lognormal_segments(T: int, n_adapters: int, mu: float, sigma: float, seed: int) -> List[int]:
    """Segment lengths ~ lognormal(mu, sigma), normalised to sum T by
    largest-remainder rounding; every segment gets at least one token."""
    g = _gen(seed)
    raw = torch.exp(mu + sigma * torch.randn(n_adapters, generator=g, dtype=torch.float64))
    share = raw / raw.sum() * (T - n_adapters)
    base = torch.floor(share)
    rem = int(T - n_adapters - int(base.sum().item()))
    order = torch.argsort(share - base, descending=True)
    lens = base.to(torch.int64) + 1
    lens[order[:rem]] += 1
    assert int(lens.sum()) == T
    return [int(v) for v in lens]


def normal(shape, std: float, dtype: torch.dtype, seed: int) -> torch.Tensor:
    return (torch.randn(*shape, generator=_gen(seed), dtype=torch.float32) * std).to(dtype)


def algorithmic_bytes(T: int, d_in: int, d_out: int, touched_ranks, elem_bytes: int = 2) -> int:
    """Minimum HBM bytes of one grouped shrink+expand call: X read once, Y read
    and written once, each touched adapter's A [r, d_in] and B [d_out, r] read
    once; the intermediate H is excluded."""
    s = elem_bytes
    return s * T * d_in + 2 * s * T * d_out + sum(s * int(r) * (d_in + d_out) for r in touched_ranks)


def algorithmic_bytes_nslice(T: int, d_in: int, d_outs, touched_ranks, elem_bytes: int = 2) -> int:
    """algorithmic_bytes of one call with one A per output slice: X read once,
    every slice's Y window read and written once, each touched adapter's A_i
    [r, d_in] and B_i [o_i, r] read once per slice."""
    s = elem_bytes
    return (s * T * d_in + 2 * s * T * sum(d_outs)
            + sum(s * int(r) * (d_in + int(o)) for r in touched_ranks for o in d_outs))


def algorithmic_flops(T: int, d_in: int, d_out: int, token_ranks) -> int:
    """2*T*r*(d_in + d_out) summed over tokens (token_ranks: rank per routed token)."""
    return sum(2 * int(r) * (d_in + d_out) for r in token_ranks)


@dataclass
class DecodeLayer:
    """One LoRA-enabled linear of a decode step, in vLLM's stacked layout."""
    wa: torch.Tensor                 # [L, 1, r, d_in]
    wbs: List[torch.Tensor]          # per slice [L, 1, o_i, r]
    y_offsets: List[int]
    d_in: int
    d_out: int                       # columns of y
    name: str = ""


@dataclass
class DecodeStep:
    """Routing and per-layer weights of one decode step."""
    T: int
    rank: int
    n_adapters: int
    dtype: torch.dtype
    indices: torch.Tensor            # [T] int64
    layers: List[DecodeLayer] = field(default_factory=list)

    def touched(self) -> List[int]:
        return sorted(set(int(v) for v in self.indices.tolist() if v >= 0))

    def bytes_per_step(self) -> int:
        k = len(self.touched())
        return sum(algorithmic_bytes(self.T, L.d_in, L.d_out, [self.rank] * k) for L in self.layers)


def llama7b_decode_layer_pair(T: int, n_adapters: int, rank: int, dtype: torch.dtype, seed: int,
                              hidden: int = 4096, device: Optional[str] = None):
    """(qkv, o_proj) LoRA layers of a Llama-7B-shaped decoder layer:
    qkv = shrink hidden->r, expand r->3 slices of hidden at offsets 0/h/2h;
    o_proj = shrink hidden->r, expand r->hidden.  Weights ~ N(0, 0.02^2)."""
    wa_q = normal((n_adapters, 1, rank, hidden), 0.02, dtype, seed)
    wbs_q = [normal((n_adapters, 1, hidden, rank), 0.02, dtype, seed + 1 + i) for i in range(3)]
    wa_o = normal((n_adapters, 1, rank, hidden), 0.02, dtype, seed + 4)
    wb_o = normal((n_adapters, 1, hidden, rank), 0.02, dtype, seed + 5)
    if device is not None:
        wa_q, wa_o, wb_o = wa_q.to(device), wa_o.to(device), wb_o.to(device)
        wbs_q = [w.to(device) for w in wbs_q]
    qkv = DecodeLayer(wa_q, wbs_q, [0, hidden, 2 * hidden], hidden, 3 * hidden, "qkv")
    o = DecodeLayer(wa_o, [wb_o], [0], hidden, hidden, "o_proj")
    return qkv, o


# Configuration 2 of the benchmark: Llama-7B decode, 256 tokens, 64 resident
# adapters, rank 32, bf16, Zipf(1.1) routing (seed 1), 40 layers x {qkv, o_proj}.
CFG2 = dict(T=256, n_adapters=64, rank=32, hidden=4096, layers=40, zipf_s=1.1, routing_seed=1,
            dtype=torch.bfloat16)
