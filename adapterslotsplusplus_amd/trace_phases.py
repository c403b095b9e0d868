"""Phase breakdown of the fused decode kernels, from a traced build.

    python -m adapterslotsplusplus_amd.build --trace
    python -m adapterslotsplusplus_amd.trace_phases [--call o_proj|qkv|cfg5_o|cfg5_qkv|cfg4_shrink|linear|plan|cfg3_shrink] [--out FILE]

The traced library (-DWP_TRACE) records, per workgroup, the 100 MHz
real-time counter at the phase boundaries of one fused launch (thread 0,
after waiting for wave 0's memory operations, which perturbs the timing a
little): entry, plan loaded; shrink workgroups: first token tile's MFMAs done,
partials stored and acknowledged; expand workgroups: B and Y loaded, gate
open, partials collected, Y stored.  This script runs the cfg2 decode step's
calls over 40 layers of distinct weights (so the traced call's weights are
not in the caches), traces one call of the last layer, and prints a markdown
table of each phase's duration (median, p10, p90 over workgroups) and of the
times, from the first workgroup's entry, at which each role reaches each
stamp; the same call's duration from HIP events on the normal library is
measured separately by bench.py.

--call cfg4_shrink traces the large-plan shrink launch of the cfg4 prefill
chunk instead (shrink() over T=8192 tokens of 16 adapters, r=64, fp16, d=4096,
8 layers of distinct weights): per workgroup the entry, block resolution,
slice loop, partial store and count, and for each block's last workgroup
the d-range sum into H; with each workgroup's compute unit (from its
hardware ids), the workgroups per compute unit and when each unit finished.
"""
from __future__ import annotations

import argparse
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))


def _pct(v, q):
    v = sorted(v)
    if not v:
        return float("nan")
    i = min(len(v) - 1, max(0, int(round(q * (len(v) - 1)))))
    return v[i]


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--call", default="o_proj",
                    choices=["o_proj", "qkv", "cfg5_o", "cfg5_qkv", "cfg4_shrink", "linear", "plan", "cfg3_shrink"])
    ap.add_argument("--out", default=None)
    args = ap.parse_args(argv)
    if args.call == "cfg4_shrink":
        return trace_cfg4_shrink(args)
    if args.call == "linear":
        return trace_linear(args)
    if args.call == "plan":
        return trace_plan(args)
    if args.call == "cfg3_shrink":
        return trace_cfg3_shrink(args)
    from . import build as wp_build

    if not os.path.exists(wp_build.TRACE_LIB_PATH):
        raise SystemExit("build the traced library first: python -m adapterslotsplusplus_amd.build --trace")
    import torch

    from . import _lib, workloads as wl
    from .engine import WarpPipeEngine

    # The library is loaded when the first engine is created: point it at the
    # traced build before that.
    if _lib._lib is not None and _lib.LIB_PATH != wp_build.TRACE_LIB_PATH:
        raise SystemExit("the normal library is already loaded in this process")
    _lib.LIB_PATH = wp_build.TRACE_LIB_PATH

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.call in ("cfg5_o", "cfg5_qkv"):
        T, L, r, h, n_layers = 128, 32, 32, 2048, 40
        idx = torch.repeat_interleave(torch.arange(L), 4).to(dev)
    else:
        c = wl.CFG2
        T, L, r, h, n_layers = c["T"], c["n_adapters"], c["rank"], c["hidden"], 40
        idx = wl.zipf_indices(T, L, c["zipf_s"], c["routing_seed"]).to(dev)
    dt = torch.bfloat16
    gen = torch.Generator(device=dev)
    gen.manual_seed(77)

    def rn(shape, std):
        return (torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32) * std).to(dt)

    n_slices = 3 if args.call in ("qkv", "cfg5_qkv") else 1
    # cfg5_qkv: one A per slice (add_lora_packed_nslice's form), the others one shared A.
    per_slice_a = args.call == "cfg5_qkv"
    layers = [dict(wa=[rn((L, 1, r, h), .02) for _ in range(n_slices)] if per_slice_a else rn((L, 1, r, h), .02),
                   wb=[rn((L, 1, h, r), .02) for _ in range(n_slices)],
                   x=rn((T, h), 1.), y=rn((T, n_slices * h), 1.)) for _ in range(n_layers)]
    engine = WarpPipeEngine()
    lib = _lib.load()
    words = 1 << 20
    buf = torch.zeros(words, dtype=torch.int64, device=dev)
    assert engine.build_seg_bounds(idx)
    offs = [k * h for k in range(n_slices)]

    def call(ly):
        engine.add_lora_slices(ly["y"], ly["x"], ly["wa"], ly["wb"], 0.5, offs)

    for ly in layers:
        call(ly)
    torch.cuda.synchronize()
    for ly in layers[:-1]:
        call(ly)
    torch.cuda.synchronize()
    _lib.check(lib.wp_set_trace(engine._handle, buf.data_ptr(), words), "set_trace")
    call(layers[-1])
    torch.cuda.synchronize()
    _lib.check(lib.wp_set_trace(engine._handle, None, 0), "set_trace")
    assert engine.device_errors() == 0
    tr = buf.view(-1, 8).cpu()
    tags = tr[:, 7]
    live = tags != 0
    tr = tr[live]
    tags = tags[live]
    role = (tags & 0xFF).tolist()
    t0 = int(tr[:, 0].min())
    ticks_us = 0.01  # 100 MHz
    rows = tr.tolist()
    shrink = [x for x, ro in zip(rows, role) if ro == 1]
    expand = [x for x, ro in zip(rows, role) if ro == 2]

    def rel(lst, i):
        return [(x[i] - t0) * ticks_us for x in lst if x[i] > 0]

    def dur(lst, i, j):
        return [(x[j] - x[i]) * ticks_us for x in lst if x[i] > 0 and x[j] > 0]

    end = max(max(x[3] for x in shrink) if shrink else 0, max(x[5] for x in expand) if expand else 0)
    lines = [f"### Phases of one `{args.call}` call (T={T}, {L} resident adapters, r={r}, h={h}, bf16, "
             f"{n_layers} layers of distinct weights; traced build)", "",
             f"Workgroups with work: {len(shrink)} shrink, {len(expand)} expand; first entry to last stamp "
             f"{(end - t0) * ticks_us:.2f} us.", "",
             "| role | phase | median us | p10 | p90 |", "|---|---|---|---|---|"]

    def row(name, phase, v):
        lines.append(f"| {name} | {phase} | {_pct(v, .5):.2f} | {_pct(v, .1):.2f} | {_pct(v, .9):.2f} |")

    row("shrink", "entry, from the first entry (dispatch)", rel(shrink, 0))
    row("shrink", "plan loads (entry -> plan loaded)", dur(shrink, 0, 1))
    row("shrink", "A and X stream + MFMA (-> first tile done)", dur(shrink, 1, 2))
    row("shrink", "reduce + partial store acknowledged", dur(shrink, 2, 3))
    row("shrink", "partials stored, from the first entry", rel(shrink, 3))
    row("expand", "entry, from the first entry (dispatch)", rel(expand, 0))
    row("expand", "plan loads (entry -> plan loaded)", dur(expand, 0, 1))
    row("expand", "B and Y loads (-> landed)", dur(expand, 1, 2))
    row("expand", "gate (-> every shrink workgroup's probe word written)", dur(expand, 2, 3))
    row("expand", "partials collected (-> H in LDS)", dur(expand, 3, 4))
    row("expand", "MFMA + Y store acknowledged", dur(expand, 4, 5))
    row("expand", "gate open, from the first entry", rel(expand, 3))
    row("expand", "Y stored, from the first entry", rel(expand, 5))
    text = "\n".join(lines)
    print(text)
    if args.out:
        with open(args.out, "w") as f:
            f.write(text + "\n")


def trace_linear(args):
    """One linear_lora launch at the draft shape (T=128 = 32 tenants x 4
    tokens, 2048 x 2048 bf16 with bias, r=32), 40 layers of distinct weights:
    shrink workgroups (entry, block resolved, first tile, partials stored),
    block reducers (entry, partials there, H stored before the flag) and GEMM
    workgroups (entry, K-range done, partial stored, counted; each tile's last
    one: K-split partials, B rows and H flags loaded and the base summed, then
    H rows loaded, delta added and y stored)."""
    _lib = _load_traced()
    import torch

    from .engine import WarpPipeEngine

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    T, L, r, h, n_layers = 128, 32, 32, 2048, 40
    dt = torch.bfloat16
    idx = torch.repeat_interleave(torch.arange(L), 4).to(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(78)

    def rn(shape, std):
        return (torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32) * std).to(dt)

    layers = [dict(x=rn((T, h), 1.), w=rn((h, h), .02), b=rn((h,), .1), wa=rn((L, 1, r, h), .02),
                   wb=rn((L, 1, h, r), .02), y=torch.empty(T, h, dtype=dt, device=dev)) for _ in range(n_layers)]
    engine = WarpPipeEngine()
    lib = _lib.load()
    words = 1 << 20
    buf = torch.zeros(words, dtype=torch.int64, device=dev)
    assert engine.build_seg_bounds(idx)

    def call(ly):
        assert engine.linear_lora(ly["x"], ly["w"], ly["b"], ly["wa"], ly["wb"], 0.5, out=ly["y"]) is not None

    for _ in range(2):
        for ly in layers:
            call(ly)
    torch.cuda.synchronize()
    for ly in layers[:-1]:
        call(ly)
    torch.cuda.synchronize()
    _lib.check(lib.wp_set_trace(engine._handle, buf.data_ptr(), words), "set_trace")
    call(layers[-1])
    torch.cuda.synchronize()
    _lib.check(lib.wp_set_trace(engine._handle, None, 0), "set_trace")
    assert engine.device_errors() == 0
    tr = buf.view(-1, 8).cpu()
    tags = tr[:, 7]
    live = tags != 0
    tr = tr[live]
    role = (tags[live] & 0xFF).tolist()
    t0 = int(tr[:, 0].min())
    ticks_us = 0.01
    rows = tr.tolist()
    shrink = [x for x, ro in zip(rows, role) if ro == 1]
    red = [x for x, ro in zip(rows, role) if ro == 4]
    gemm = [x for x, ro in zip(rows, role) if ro == 5]
    last = [x for x in gemm if x[6] > 0]

    def rel(lst, i):
        return [(x[i] - t0) * ticks_us for x in lst if x[i] > 0]

    def dur(lst, i, j):
        return [(x[j] - x[i]) * ticks_us for x in lst if x[i] > 0 and x[j] > 0]

    end = max(x[6] for x in last) if last else t0
    lines = [f"### Phases of one `linear_lora` launch (T={T} = 32 tenants x 4 tokens, {h} x {h} bf16 with bias, "
             f"r={r}, {n_layers} layers of distinct weights; traced build)", "",
             f"Workgroups with work: {len(shrink)} shrink, {len(red)} block reducers, {len(gemm)} GEMM "
             f"({len(last)} tile epilogues); first entry to last stamp {(end - t0) * ticks_us:.2f} us.", "",
             "| role | phase | median us | p10 | p90 |", "|---|---|---|---|---|"]

    def row(name, phase, v):
        lines.append(f"| {name} | {phase} | {_pct(v, .5):.2f} | {_pct(v, .1):.2f} | {_pct(v, .9):.2f} |")

    row("shrink", "entry, from the first entry (dispatch)", rel(shrink, 0))
    row("shrink", "block resolved (entry ->)", dur(shrink, 0, 1))
    row("shrink", "A and X stream + MFMA (-> first tile done)", dur(shrink, 1, 2))
    row("shrink", "reduce + partial store acknowledged", dur(shrink, 2, 3))
    row("shrink", "partials stored, from the first entry", rel(shrink, 3))
    row("reducer", "entry, from the first entry (dispatch)", rel(red, 0))
    row("reducer", "block resolved (entry ->)", dur(red, 0, 1))
    row("reducer", "partials there (-> gate)", dur(red, 1, 2))
    row("reducer", "H rows stored and acknowledged", dur(red, 2, 3))
    row("reducer", "H flag set, from the first entry", rel(red, 3))
    row("GEMM", "entry, from the first entry (dispatch)", rel(gemm, 0))
    row("GEMM", "K-range loads + MFMA (entry ->)", dur(gemm, 0, 1))
    row("GEMM", "partial stored and acknowledged", dur(gemm, 1, 2))
    row("GEMM", "tile counter returned", dur(gemm, 2, 3))
    row("GEMM", "counted, from the first entry", rel(gemm, 3))
    row("epilogue", "K-split partials, B rows and H flags (-> base summed, rounded)", dur(last, 3, 4))
    row("epilogue", "workgroup barrier", dur(last, 4, 5))
    row("epilogue", "H rows, delta MFMA, y stored", dur(last, 5, 6))
    row("epilogue", "base summed, from the first entry", rel(last, 4))
    row("epilogue", "y stored, from the first entry", rel(last, 6))
    text = "\n".join(lines)
    print(text)
    if args.out:
        with open(args.out, "w") as f:
            f.write(text + "\n")


def trace_plan(args):
    """build_seg_bounds (the one-workgroup plan kernel) on the cfg2 routing
    (T=256, Zipf(1.1) over 64 adapters), the cfg5 routing (T=128, 32 tenants x
    4) and a T=2048 Zipf routing: the phase boundaries of one build each,
    median over 20 traced builds."""
    _lib = _load_traced()
    import torch

    from . import workloads as wl
    from .engine import WarpPipeEngine

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    engine = WarpPipeEngine()
    lib = _lib.load()
    buf = torch.zeros(8, dtype=torch.int64, device=dev)
    cases = [("cfg2 routing, T=256", wl.zipf_indices(256, 64, 1.1, 1)),
             ("cfg5 routing, T=128", torch.repeat_interleave(torch.arange(32), 4)),
             ("Zipf(1.1) over 64, T=2048", wl.zipf_indices(2048, 64, 1.1, 1))]
    names = ["ids in LDS, maintenance done", "run starts", "segment table stored", "runs sorted",
             "perm stored", "block table stored", "block token lists and header stored"]
    lines = ["### Phases of one `build_seg_bounds` plan build (traced build; median of 20 builds, us)", "",
             "| phase | " + " | ".join(c[0] for c in cases) + " |", "|---|" + "---|" * len(cases)]
    cols = []
    for _, idx in cases:
        idx = idx.to(dev)
        for _ in range(3):
            assert engine.build_seg_bounds(idx)
        torch.cuda.synchronize()
        runs = []
        _lib.check(lib.wp_set_trace(engine._handle, buf.data_ptr(), 8), "set_trace")
        for _ in range(20):
            buf.zero_()
            assert engine.build_seg_bounds(idx)
            torch.cuda.synchronize()
            runs.append(buf.cpu().tolist())
        _lib.check(lib.wp_set_trace(engine._handle, None, 0), "set_trace")
        cols.append([_pct([(r[i + 1] - r[i]) * 0.01 for r in runs], .5) for i in range(7)] +
                    [_pct([(r[7] - r[0]) * 0.01 for r in runs], .5)])
    for i, nm in enumerate(names):
        lines.append(f"| {nm} | " + " | ".join(f"{c[i]:.2f}" for c in cols) + " |")
    lines.append("| entry to end | " + " | ".join(f"{c[7]:.2f}" for c in cols) + " |")
    assert engine.device_errors() == 0
    text = "\n".join(lines)
    print(text)
    if args.out:
        with open(args.out, "w") as f:
            f.write(text + "\n")


def trace_cfg3_shrink(args):
    """shrink() at the cfg3 shapes (T=512 Zipf(1.1) over 128 adapters, ranks
    uniform in {8,16,32,64}, bf16, registered adapters; gate 5120 -> r and
    down 13824 -> r), 8 engines of distinct weights per shape: the
    decode-sized split's shrink workgroups (entry, block resolved, first
    tile's MFMAs, partials stored) and its block reducers (entry, H stored)."""
    _lib = _load_traced()
    import torch

    from . import workloads as wl
    from .engine import WarpPipeEngine

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    T, dt, n_eng = 512, torch.bfloat16, 8
    g = torch.Generator().manual_seed(2)
    ranks = [int(v) for v in torch.tensor([8, 16, 32, 64])[torch.randint(0, 4, (128,), generator=g)]]
    idx = wl.zipf_indices(T, 128, 1.1, seed=3).to(dev)
    touched = sorted(set(idx.tolist()))
    gen = torch.Generator(device=dev)
    gen.manual_seed(79)

    def rn(shape, std):
        return (torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32) * std).to(dt)

    lib = _lib.load()
    words = 1 << 20
    buf = torch.zeros(words, dtype=torch.int64, device=dev)
    lines = []
    for name, d_in in (("gate", 5120), ("down", 13824)):
        engs = []
        for _ in range(n_eng):
            e = WarpPipeEngine()
            for i in touched:
                e.register_adapter(i, rn((ranks[i], d_in), .02), rn((64, ranks[i]), .02), 1.0, rank=ranks[i])
            assert e.build_seg_bounds(idx)
            engs.append((e, rn((T, d_in), 1.), torch.zeros(T, 64, dtype=dt, device=dev)))
        for _ in range(2):
            for e, X, H in engs:
                e.shrink(X, d_in, 0, T, out=H)
        torch.cuda.synchronize()
        for e, X, H in engs[:-1]:
            e.shrink(X, d_in, 0, T, out=H)
        e, X, H = engs[-1]
        buf.zero_()
        torch.cuda.synchronize()
        _lib.check(lib.wp_set_trace(e._handle, buf.data_ptr(), words), "set_trace")
        e.shrink(X, d_in, 0, T, out=H)
        torch.cuda.synchronize()
        _lib.check(lib.wp_set_trace(e._handle, None, 0), "set_trace")
        assert e.device_errors() == 0
        tr = buf.view(-1, 8).cpu()
        tags = tr[:, 7]
        live = tags != 0
        tr = tr[live]
        role = (tags[live] & 0xFF).tolist()
        t0 = int(tr[:, 0].min())
        rows = tr.tolist()
        shrink = [x for x, ro in zip(rows, role) if ro == 1]
        red = [x for x, ro in zip(rows, role) if ro == 2]

        def rel(lst, i):
            return [(x[i] - t0) * 0.01 for x in lst if x[i] > 0]

        def dur(lst, i, j):
            return [(x[j] - x[i]) * 0.01 for x in lst if x[i] > 0 and x[j] > 0]

        end = max(max(x[3] for x in shrink), max((x[4] for x in red), default=0))
        lines += [f"### `shrink()` at the cfg3 {name} shape (T={T}, d={d_in}, {len(touched)} adapters of ranks "
                  f"8-64, bf16; traced build)", "",
                  f"Workgroups with work: {len(shrink)} shrink, {len(red)} block reducers; first entry to last stamp "
                  f"{(end - t0) * 0.01:.2f} us.", "",
                  "| role | phase | median us | p10 | p90 |", "|---|---|---|---|---|"]

        def row(nm, phase, v):
            lines.append(f"| {nm} | {phase} | {_pct(v, .5):.2f} | {_pct(v, .1):.2f} | {_pct(v, .9):.2f} |")

        row("shrink", "entry, from the first entry (dispatch)", rel(shrink, 0))
        row("shrink", "block resolved (entry ->)", dur(shrink, 0, 1))
        row("shrink", "A and X stream + MFMA (-> first tile done)", dur(shrink, 1, 2))
        row("shrink", "reduce + partial store acknowledged", dur(shrink, 2, 3))
        row("shrink", "partials stored, from the first entry", rel(shrink, 3))
        row("reducer", "entry, from the first entry (dispatch)", rel(red, 0))
        row("reducer", "partials summed, H stored (block resolved ->)", dur(red, 1, 4))
        row("reducer", "H stored, from the first entry", rel(red, 4))
        lines.append("")
        del engs
    text = "\n".join(lines)
    print(text)
    if args.out:
        with open(args.out, "w") as f:
            f.write(text + "\n")


def _load_traced():
    from . import build as wp_build

    if not os.path.exists(wp_build.TRACE_LIB_PATH):
        raise SystemExit("build the traced library first: python -m adapterslotsplusplus_amd.build --trace")
    from . import _lib

    if _lib._lib is not None and _lib.LIB_PATH != wp_build.TRACE_LIB_PATH:
        raise SystemExit("the normal library is already loaded in this process")
    _lib.LIB_PATH = wp_build.TRACE_LIB_PATH
    return _lib


def trace_cfg4_shrink(args):
    _lib = _load_traced()
    import torch

    from . import workloads as wl
    from .config import WarpPipeConfig
    from .engine import WarpPipeEngine

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    T, L, r, h, n_layers, dt = 8192, 16, 64, 4096, 8, torch.float16
    lens = wl.lognormal_segments(T, L, 6.0, 1.0, seed=4)
    idx = torch.repeat_interleave(torch.arange(L), torch.tensor(lens)).to(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)

    def rn(shape, std):
        return (torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32) * std).to(dt)

    # One store layer per model layer: the shrink reads each layer's A.
    engine = WarpPipeEngine(WarpPipeConfig(layer_stride=L))
    lib = _lib.load()
    xs = [rn((T, h), 1.) for _ in range(n_layers)]
    zb = torch.zeros(8, r, dtype=dt, device=dev)
    for lay in range(n_layers):
        for i in range(L):
            engine.register_adapter(i, rn((r, h), .02), zb, 0.25, rank=r, layer=lay)
    Hs = [torch.empty(T, r, dtype=dt, device=dev) for _ in range(n_layers)]
    assert engine.build_seg_bounds(idx)
    words = 1 << 20
    buf = torch.zeros(words, dtype=torch.int64, device=dev)

    def call(lay):
        engine.shrink(xs[lay], h, r, T, out=Hs[lay], layer=lay)

    for lay in range(n_layers):
        call(lay)
    torch.cuda.synchronize()
    for lay in range(n_layers - 1):
        call(lay)
    torch.cuda.synchronize()
    _lib.check(lib.wp_set_trace(engine._handle, buf.data_ptr(), words), "set_trace")
    call(n_layers - 1)
    torch.cuda.synchronize()
    _lib.check(lib.wp_set_trace(engine._handle, None, 0), "set_trace")
    assert engine.device_errors() == 0
    tr = buf.view(-1, 8).cpu()
    live = (tr[:, 7] & 0xFF) == 3
    rows = tr[live].tolist()
    t0 = min(x[0] for x in rows)
    us = 0.01

    def cu_key(hw):
        xcc = (hw >> 32) & 0xF
        h32 = hw & 0xFFFFFFFF
        return (xcc, (h32 >> 13) & 0x7, (h32 >> 12) & 1, (h32 >> 8) & 0xF)

    def rel(i, sel=None):
        return [(x[i] - t0) * us for x in (sel or rows) if x[i] > 0]

    def dur(i, j, sel=None):
        return [(x[j] - x[i]) * us for x in (sel or rows) if x[i] > 0 and x[j] > 0]

    last = [x for x in rows if x[4] > 0]
    end = max(max(x[3] for x in rows), max((x[4] for x in last), default=0))
    per_cu = {}
    for x in rows:
        per_cu.setdefault(cu_key(x[6]), []).append(x)
    counts = {}
    for k, v in per_cu.items():
        counts.setdefault(len(v), []).append(max(max(y[3], y[4]) for y in v))
    lines = [f"### Phases of one cfg4 `shrink` launch (T={T}, {L} adapters lognormal(6,1) seed 4, r={r}, d={h}, fp16, "
             f"{n_layers} layers of distinct weights; traced build)", "",
             f"Workgroups with work: {len(rows)} on {len(per_cu)} compute units ({len(last)} last arrivers); "
             f"first entry to last stamp {(end - t0) * us:.2f} us.", "",
             "| phase | median us | p10 | p90 | max |", "|---|---|---|---|---|"]

    def row(phase, v):
        lines.append(f"| {phase} | {_pct(v, .5):.2f} | {_pct(v, .1):.2f} | {_pct(v, .9):.2f} | {max(v) if v else 0:.2f} |")

    row("entry, from the first entry (dispatch)", rel(0))
    row("block resolved (entry -> plan and adapter loaded)", dur(0, 1))
    row("slice loop (-> last MFMA)", dur(1, 2))
    row("partial store acknowledged + counter", dur(2, 3))
    row("last arriver: d-range sum + H store", dur(3, 4, last))
    row("slice loop done, from the first entry", rel(2))
    row("counted, from the first entry", rel(3))
    row("H stored (last arrivers), from the first entry", rel(4, last))
    lines += ["", "| workgroups per compute unit | compute units | finish from first entry: median us | max |",
              "|---|---|---|---|"]
    for n in sorted(counts):
        f = [(v - t0) * us for v in counts[n]]
        lines.append(f"| {n} | {len(f)} | {_pct(f, .5):.2f} | {max(f):.2f} |")
    text = "\n".join(lines)
    print(text)
    if args.out:
        with open(args.out, "w") as f:
            f.write(text + "\n")


if __name__ == "__main__":
    sys.exit(main())
