"""Draft-model integration: nn.Linear + per-token LoRA delta through the engine.

The reference's speculative-decoding benchmarks wrap the draft model's
projections in `BGMVLoRALinear` (benchmarks/e2e/serve_multitenant.py:56-87):
the base linear plus a per-row delta from vLLM's bgmv_shrink/bgmv_expand,
routed by a module-global `STATE["idx"]`, inside a CUDA-graph-captured
fixed-shape step (benchmarks/e2e/batched_spec_loop.py:69-131).  This module
is the engine-backed counterpart:

  * `DraftLoRAContext` owns the routing tensor (one adapter id per TOKEN of
    the flattened [B*S, in] activations, as batched_spec_loop.py:88-92 notes)
    and the engine.  `begin_step()` builds the step's segment table once
    (build_seg_bounds); every wrapped linear of the step then reuses it.
    Both are capture-safe, so a whole draft step -- routing table included --
    records into one graph, and a replay reads whatever ids were copied into
    `ctx.idx` before it.
  * `WarpPipeLoRALinear.forward` computes the base linear and adds
    scale * (x . A_idx^T) . B_idx^T to it in place with one add_lora_packed
    call (shrink + expand in one launch, fp32 accumulation, one rounding of
    base + delta).  mode "none" returns the base only (the reference's
    shared-draft mode).
  * `WarpPipeLoRAPackedLinear` groups linears that read the same input
    (q/k/v): one base GEMM over their stacked weights and one launch for all
    their deltas, each projection with its own adapters.

There is no fallback: a call the engine cannot take (a rank without kernels,
more tokens than the engine was sized for) raises.
"""
from __future__ import annotations

from typing import Dict, Iterable, Optional, Sequence, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from .engine import WarpPipeEngine
from .punica_wrapper import report_device_errors


class DraftLoRAContext:
    """Routing and engine shared by every WarpPipeLoRALinear of one model.

    tokens: the fixed number of flattened rows a step's linears see (B * S);
    idx holds one adapter id per row (-1: no LoRA for that row)."""

    def __init__(self, engine: WarpPipeEngine, tokens: int, scale: float = 2.0, device=None,
                 fused_linear: bool = False):
        self.engine = engine
        self.tokens = int(tokens)
        self.scale = float(scale)
        self.mode = "lora"
        # True: each wrapped linear runs its base GEMM and LoRA delta as one
        # engine launch (engine.linear_lora), falling back to F.linear +
        # add_lora_packed for shapes without that kernel.
        self.fused_linear = bool(fused_linear)
        dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        self.idx = torch.zeros(self.tokens, dtype=torch.int64, device=dev)
        # OR of every device error bit poll_errors has seen.
        self.device_errors = 0

    def poll_errors(self) -> int:
        """Device error bits of earlier steps (tokens the kernels skipped, whose
        rows lack their LoRA delta), without a host wait: the bits an earlier
        poll moved to host memory once that move has landed.  ORs them into
        `device_errors` and reports them (a logged warning, or RuntimeError
        with AS_WARP_PIPE_STRICT=1).  Call outside graph capture; replay
        loops call it between replays."""
        bits = self.engine.poll_device_errors()
        self.device_errors |= bits
        return report_device_errors(bits, "DraftLoRAContext")

    def set_routing(self, ids: torch.Tensor) -> None:
        """Copies per-token adapter ids into the routing buffer (stream-ordered,
        so it may sit between graph replays)."""
        ids = ids.reshape(-1)
        if ids.numel() != self.tokens:
            raise RuntimeError(f"DraftLoRAContext: routing has {ids.numel()} ids, the step has {self.tokens} tokens")
        self.idx.copy_(ids)

    def begin_step(self) -> None:
        """Builds the step's segment table from `idx` (once per step, before the
        model's forward; inside a captured step it is one graph node).
        Outside capture it first reports tokens an earlier step's kernels had
        to skip (poll_errors)."""
        if self.mode == "none":
            return
        if not torch.cuda.is_current_stream_capturing():
            self.poll_errors()
        if not self.engine.build_seg_bounds(self.idx):
            raise RuntimeError(f"DraftLoRAContext: {self.tokens} tokens exceed the engine's max_tokens")


class WarpPipeLoRALinear(nn.Module):
    """Base nn.Linear + per-token draft-LoRA delta, K adapter slots.

    A: [K, rank, in], B: [K, out, rank] (the layouts of serve_multitenant.py:
    74-75), same dtype and device as the base weight."""

    def __init__(self, base: nn.Linear, A: torch.Tensor, B: torch.Tensor, ctx: DraftLoRAContext):
        super().__init__()
        if A.dim() != 3 or B.dim() != 3 or A.size(0) != B.size(0) or A.size(1) != B.size(2):
            raise RuntimeError("WarpPipeLoRALinear: A must be [K, rank, in] and B [K, out, rank]")
        if A.size(2) != base.in_features or B.size(1) != base.out_features:
            raise RuntimeError("WarpPipeLoRALinear: A/B do not match the base linear's shape")
        self.in_features = base.in_features
        self.out_features = base.out_features
        self.weight = base.weight
        self.bias = base.bias
        self.rank = int(A.size(1))
        self.ctx = ctx
        # The engine's stacked layout: wa_t_all [K, 1, r, in], wb_t_all [K, 1, out, r].
        self.register_buffer("wa_t_all", A.detach().unsqueeze(1).contiguous(), persistent=False)
        self.register_buffer("wb_t_all", B.detach().unsqueeze(1).contiguous(), persistent=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.ctx.mode != "none" and self.ctx.fused_linear:
            x2d = x.reshape(-1, self.in_features)
            if not x2d.is_contiguous():
                x2d = x2d.contiguous()
            if x2d.size(0) != self.ctx.tokens:
                raise RuntimeError(
                    f"WarpPipeLoRALinear: {x2d.size(0)} rows, but the step's routing covers {self.ctx.tokens} tokens")
            y = self.ctx.engine.linear_lora(x2d, self.weight, self.bias, self.wa_t_all, self.wb_t_all, self.ctx.scale)
            if y is not None:
                return y.view(*x.shape[:-1], self.out_features)
        y = F.linear(x, self.weight, self.bias)
        if self.ctx.mode == "none":
            return y
        x2d = x.reshape(-1, self.in_features)
        if not x2d.is_contiguous():
            x2d = x2d.contiguous()
        y = y.contiguous()
        if x2d.size(0) != self.ctx.tokens:
            raise RuntimeError(
                f"WarpPipeLoRALinear: {x2d.size(0)} rows, but the step's routing covers {self.ctx.tokens} tokens")
        if not self.ctx.engine.add_lora_packed(y.view(-1, self.out_features), x2d, self.wa_t_all, self.wb_t_all,
                                               self.ctx.scale):
            raise RuntimeError(f"WarpPipeLoRALinear: rank {self.rank} has no kernels")
        return y


class WarpPipeLoRAPackedLinear(nn.Module):
    """Several linears that read the same input (q/k/v, gate/up) as one module:
    one base GEMM over their stacked weights, then every projection's
    per-token LoRA delta in ONE engine launch with one adapter pair per
    projection (add_lora_slices with per-slice A: x is read once).
    forward(x) returns one output per projection (views into one packed y).

    bases: the nn.Linear modules (same in_features, dtype, device); As[i]
    [K, rank, in] and Bs[i] [K, out_i, rank] are projection i's adapters."""

    def __init__(self, bases: Sequence[nn.Linear], As: Sequence[torch.Tensor], Bs: Sequence[torch.Tensor],
                 ctx: DraftLoRAContext):
        super().__init__()
        if not 1 <= len(bases) <= 4 or len(As) != len(bases) or len(Bs) != len(bases):
            raise RuntimeError("WarpPipeLoRAPackedLinear: 1..4 linears, one (A, B) pair each")
        self.in_features = bases[0].in_features
        self.out_sizes = [b.out_features for b in bases]
        if any(b.in_features != self.in_features for b in bases):
            raise RuntimeError("WarpPipeLoRAPackedLinear: the linears must share in_features")
        ranks = {int(A.size(1)) for A in As}
        if len(ranks) != 1:
            raise RuntimeError("WarpPipeLoRAPackedLinear: one rank for every projection")
        self.rank = ranks.pop()
        for base, A, B in zip(bases, As, Bs):
            if (A.dim() != 3 or B.dim() != 3 or A.size(0) != B.size(0) or A.size(1) != B.size(2)
                    or A.size(2) != self.in_features or B.size(1) != base.out_features):
                raise RuntimeError("WarpPipeLoRAPackedLinear: A must be [K, rank, in] and B [K, out, rank]")
        with torch.no_grad():
            self.weight = nn.Parameter(torch.cat([b.weight.detach() for b in bases], 0), requires_grad=False)
            if any(b.bias is not None for b in bases):
                bias = [b.bias.detach() if b.bias is not None else torch.zeros(b.out_features, dtype=b.weight.dtype,
                                                                               device=b.weight.device) for b in bases]
                self.bias = nn.Parameter(torch.cat(bias), requires_grad=False)
            else:
                self.bias = None
        self.ctx = ctx
        self._offsets = [sum(self.out_sizes[:i]) for i in range(len(bases))]
        self._was = [A.detach().unsqueeze(1).contiguous() for A in As]
        self._wbs = [B.detach().unsqueeze(1).contiguous() for B in Bs]
        for i, (wa, wb) in enumerate(zip(self._was, self._wbs)):
            self.register_buffer(f"wa_t_all_{i}", wa, persistent=False)
            self.register_buffer(f"wb_t_all_{i}", wb, persistent=False)

    def forward(self, x: torch.Tensor):
        y = F.linear(x, self.weight, self.bias)
        if self.ctx.mode != "none":
            x2d = x.reshape(-1, self.in_features)
            if not x2d.is_contiguous():
                x2d = x2d.contiguous()
            if x2d.size(0) != self.ctx.tokens:
                raise RuntimeError(f"WarpPipeLoRAPackedLinear: {x2d.size(0)} rows, but the step's routing covers "
                                   f"{self.ctx.tokens} tokens")
            if not self.ctx.engine.add_lora_slices(y.view(-1, y.size(-1)), x2d, self._was, self._wbs, self.ctx.scale,
                                                   self._offsets):
                raise RuntimeError(f"WarpPipeLoRAPackedLinear: rank {self.rank} has no kernels")
        return tuple(y.split(self.out_sizes, dim=-1))


def wrap_linears(model: nn.Module, weights: Dict[str, Tuple[torch.Tensor, torch.Tensor]],
                 ctx: DraftLoRAContext) -> Iterable[str]:
    """Replaces every nn.Linear of `model` whose qualified name is a key of
    `weights` ({name: (A [K, r, in], B [K, out, r])}) by a WarpPipeLoRALinear;
    returns the names replaced (the counterpart of extract_draft_lora's
    module selection, serve_multitenant.py:90-110)."""
    done = []
    for name, (A, B) in weights.items():
        parent_name, _, child = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        base = getattr(parent, child)
        if not isinstance(base, nn.Linear):
            raise RuntimeError(f"wrap_linears: {name} is not an nn.Linear")
        setattr(parent, child, WarpPipeLoRALinear(base, A, B, ctx))
        done.append(name)
    return done


class CapturedStep:
    """One fixed-shape step (routing table + model forward) recorded into a
    HIP graph; replay() reads the inputs and routing copied in before it
    (batched_spec_loop.py:69-131's Step, reduced to what the LoRA path needs)."""

    def __init__(self, fn, ctx: DraftLoRAContext, warmup: int = 2):
        self.fn = fn
        self.ctx = ctx
        self.out: Optional[torch.Tensor] = None
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                ctx.begin_step()
                fn()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            ctx.begin_step()
            self.out = fn()

    def replay(self, routing: Optional[torch.Tensor] = None) -> torch.Tensor:
        if routing is not None:
            self.ctx.set_routing(routing)
        if self.ctx.mode != "none":
            self.ctx.poll_errors()
        self.graph.replay()
        return self.out
