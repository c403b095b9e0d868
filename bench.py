#!/usr/bin/env python3
"""bench.py -- grouped multi-LoRA apply on one MI355X.

Workload (the metric's configuration): one
Llama-7B-shaped decode step of 40 layers x {packed-qkv, o_proj} LoRA calls =
80 grouped shrink+expand calls, T=256 tokens (one per request) routed
Zipf(1.1) over 64 resident adapters, rank 32, bf16, weights ~ N(0, 0.02^2),
x ~ N(0, 1).  Every layer has its own weights, inputs and outputs (3.9 GB of
weights per step, far above the 256 MB Infinity Cache).  A step is
build_seg_bounds + the 80 calls, captured in one HIP graph; the timed region
replays it K times.

value = algorithmic HBM bytes of the 80 calls / step time (GB/s); the bytes
count X read once, Y read and written once and each touched adapter's A and B
read once per call (H excluded).

roofline: the dominant kernel is the fused apply kernel of the packed-qkv
call (one launch per call, about 60% of the step).  Its average launch
duration is measured with HIP events on the launch stream around replays of a
graph holding only the 40 qkv launches (back to back, as in the step);
achieved = the call's algorithmic bytes / that duration.  traffic (HBM bytes per launch) comes from the rocprofv3 --pmc
FETCH_SIZE / WRITE_SIZE runs summarised in profiles/apply_qkv_cfg2_pmc.json,
scaled by the same counters' reading for the plain copy this script launches
once (COPY_BYTES read + written); null when that summary is absent.
traffic_measured_on names the commit whose kernels those counters were read
on (the summary's `measured_on`).

cpu_baseline: the oracle's per-segment torch fp32 path on this host's cores,
on one cfg2 o_proj call (the metric's unit), with BASELINE.json configs[0]
(cfg1, the reference's CPU-runnable case) beside it under `cfg1`.

Prints one JSON line.  `--gpus N` with N > 1 exits: this build runs on one GPU.

The same line also carries the north star's secondary targets, measured in
the same run (skip with --no-secondary): `flatness_max_over_min` (cfg2 latency
over 1..128 resident adapters, target <= 1.15), `cfg5_us_per_step` (the draft
step, q/k/v of a layer in one call with one A per slice) and
`cfg1_us_per_call`, with their details under `secondary`.

`--workload` selects one measurement alone (each prints its own JSON line;
none is the metric line): `flatness`, `cfg1` (with its CPU baseline), `cfg3`
(13B mixed-rank decode through registered adapters: shrink + expand), `cfg4`
(prefill chunk, MFMA), `cfg5` (the draft step as 88 calls, as 44 launches,
and through the adapter store with 4 cold adapters staged per step), `draft`
(the cfg5 step as a model forward through WarpPipeLoRALinear, with and
without the adapters).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
COPY_BYTES = 256 << 20  # calibration copy: bytes read (and written) once
PMC_SUMMARY = os.path.join(ROOT, "profiles", "apply_qkv_cfg2_pmc.json")
# Bytes one replay of the flatness and cfg1 graphs reads at least: twice the
# 256 MB last-level cache, so those rows are not served from it.
FLAT_WORKING_SET = 512 << 20
METRIC = "shrink+expand achieved HBM GB/s (% of peak); us per 80-call decode step"


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the flatness, cfg5 and cfg1 keys of the default line")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline sample length")
    ap.add_argument("--workload", default="cfg2", choices=["cfg2", "flatness", "cfg1", "cfg3", "cfg4", "cfg5", "draft"])
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(seconds):
    """The oracle's per-segment torch fp32 path (the reference's CPU algorithm)
    on one o_proj call of the same workload, on this host's cores."""
    import torch

    from adapterslotsplusplus_amd import workloads as wl
    from oracle import bgmv
    from oracle import segments as so

    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    c = wl.CFG2
    T, L, r, h = c["T"], c["n_adapters"], c["rank"], c["hidden"]
    idx = wl.zipf_indices(T, L, c["zipf_s"], c["routing_seed"])
    wa = wl.normal((L, 1, r, h), 0.02, c["dtype"], 900)
    wb = wl.normal((L, 1, h, r), 0.02, c["dtype"], 901)
    x = wl.normal((T, h), 1.0, c["dtype"], 902)
    y = wl.normal((T, h), 1.0, c["dtype"], 903)
    segs = so.seg_bounds(idx.numpy()).tolist()
    touched = len(set(idx.tolist()))
    nbytes = wl.algorithmic_bytes(T, h, h, [r] * touched)
    for _ in range(3):
        bgmv.add_lora(y, x, wa, wb, 0.5, segs)
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 20:
        t0 = time.perf_counter()
        bgmv.add_lora(y, x, wa, wb, 0.5, segs)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": round(nbytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"{len(times)} o_proj calls of the same workload (T=256, 64 adapters, r=32, bf16, Zipf(1.1); "
                   f"{len(segs)} run-length segments), median {med * 1e6:.0f} us/call, torch fp32 per segment"),
        "us_per_call": round(med * 1e6, 1),
    }


def launch_duration_us(calls, reps):
    """Average duration (us) of the single kernel launch each call makes: the
    calls are captured into one HIP graph (their launches then run back to
    back), and HIP events on the launch stream time `reps` replays."""
    import torch

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for fn in calls:
            fn()
    g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * len(calls))


def pmc_traffic():
    """(HBM bytes per launch of the qkv apply kernel, the build they were
    counted on) from the committed PMC summary, or (None, None)."""
    try:
        with open(PMC_SUMMARY) as f:
            p = json.load(f)
        return int(p["hbm_bytes_per_launch"]), p.get("measured_on")
    except (OSError, ValueError, KeyError):
        return None, None


def graph_us(fn, reps, warmup=3):
    """Captures fn() into one HIP graph and returns us per replay (HIP events
    on the launch stream around `reps` back-to-back replays)."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps, g


def measure_floor(engine, dev, n_calls, sizes, reps):
    """Per-launch time of the library's read probe (wp_read_probe: 16-byte
    non-temporal loads over two workgroups per compute unit) reading each of
    `sizes` bytes, over n_calls distinct buffers in one graph (no call finds
    its bytes in cache), and of an empty launch.  Reading a call's bytes once
    in one launch is a floor under that call's kernel: the call also writes Y
    and has the shrink -> expand dependency to hide."""
    import ctypes

    import torch

    from adapterslotsplusplus_amd import _lib

    lib = _lib.load()
    stride = (max(sizes) + 255) // 256 * 256
    buf = torch.empty(n_calls * stride, dtype=torch.uint8, device=dev).fill_(1)
    sink = torch.zeros(8192, dtype=torch.uint8, device=dev)
    base = buf.data_ptr()

    def probe(off, nbytes):
        return lambda: _lib.check(lib.wp_read_probe(engine._handle, ctypes.c_void_p(base + off), nbytes,
                                                    ctypes.c_void_p(sink.data_ptr()),
                                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
                                  "read_probe")

    out = {}
    for nbytes in sizes:
        nb = nbytes // 16 * 16
        out[nbytes] = launch_duration_us([probe(i * stride, nb) for i in range(n_calls)], reps)
    out[0] = launch_duration_us([probe(0, 0) for _ in range(n_calls)], reps)
    del buf, sink
    torch.cuda.empty_cache()
    return out


def measure_handoff(dev, n_calls, volumes, reps):
    """Per-launch time of the library's handoff probe (wp_handoff_probe) at a
    call's volumes: `a` = the call's A and X bytes (the shrink side), `b` = B
    and the Y read (the expand side), `y` = the Y write, over n_calls distinct
    buffers in one graph.  Forms: no dependency (mode 0), one chip-wide
    dependency between the two halves on every compute unit (mode 1, the
    expand side's first batch issued before the wait), and the halves on
    separate compute units (mode 3: `group` compute units stream `a` and
    count, the rest stream all of `b` before waiting, then write `y`).  What
    one handoff costs a launch with no MFMA, no partial data and perfect
    balance."""
    import ctypes

    import torch

    from adapterslotsplusplus_amd import _lib

    lib = _lib.load()
    wgs = torch.cuda.get_device_properties(dev).multi_processor_count
    out = {}
    for name, (a_bytes, b_bytes, y_bytes) in volumes.items():
        a16, b16, y16 = (v // 16 * 16 for v in (a_bytes, b_bytes, y_bytes))
        stride = (a16 + b16 + y16 + 255) // 256 * 256
        buf = torch.empty(n_calls * stride, dtype=torch.uint8, device=dev).fill_(1)
        counters = torch.zeros(wgs * 2 * 64, dtype=torch.int32, device=dev)
        err = torch.zeros(1, dtype=torch.int32, device=dev)
        base = buf.data_ptr()

        def probe(i, group, mode):
            o = base + i * stride
            return lambda: _lib.check(lib.wp_handoff_probe(
                ctypes.c_void_p(o), a16, ctypes.c_void_p(o + a16), b16, ctypes.c_void_p(o + a16 + b16), y16,
                ctypes.c_void_p(counters.data_ptr()), ctypes.c_void_p(err.data_ptr()), group, mode, wgs,
                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "handoff_probe")

        res = {"no_wait_us": launch_duration_us([probe(i, 1, 0) for i in range(n_calls)], reps),
               "one_chip_wide_wait_us": launch_duration_us([probe(i, wgs, 1) for i in range(n_calls)], reps)}
        for S in (wgs // 4, 3 * wgs // 8, wgs // 2):
            res[f"split_{S}_of_{wgs}_cus_us"] = launch_duration_us([probe(i, S, 3) for i in range(n_calls)], reps)
        torch.cuda.synchronize()
        if int(err.item()) != 0:
            raise RuntimeError("handoff probe: a wait gave up")
        out[name] = {k: round(v, 3) for k, v in res.items()}
        out[name]["bytes"] = {"a": a16, "b": b16, "y": y16}
        del buf, counters, err
        torch.cuda.empty_cache()
    return out


def calibration_copy(dev):
    """One device copy of COPY_BYTES (read and written once): the reference
    point that scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes.
    Returns its rate in GB/s (bytes read + written over the copy's time; the
    first copy, the one the counters see, then two more timed)."""
    import torch

    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(2):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    gbs = 2 * 2 * COPY_BYTES / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del src, dst
    return gbs


def emit(out):
    print(json.dumps(out), flush=True)


def measure_flatness(reps, sort=False):
    """cfg2 shapes with N resident adapters, N = 1..128 (Zipf(1.1), seed 1;
    sort: the same tokens sorted by adapter): layers x {qkv, o_proj} with
    distinct weights per layer, one graph per N, with as many layers as make
    one replay read FLAT_WORKING_SET bytes.  Returns the rows and max/min of
    the latency per (qkv, o_proj) pair."""
    import torch

    from adapterslotsplusplus_amd import WarpPipeEngine
    from adapterslotsplusplus_amd import workloads as wl

    dev = torch.device("cuda", 0)
    T, r, h, dt = 256, 32, 4096, torch.bfloat16
    gen = torch.Generator(device=dev)
    gen.manual_seed(99)

    def rn(shape, std):
        return (torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32) * std).to(dt)

    engine = WarpPipeEngine()
    offs = [0, h, 2 * h]
    rows = []
    for N in (1, 2, 4, 8, 16, 32, 64, 128):
        idx = wl.zipf_indices(T, N, 1.1, 1).to(dev)
        if sort:
            idx = torch.sort(idx).values
        touched = len(set(idx.tolist()))
        # Enough layers that one replay reads at least FLAT_WORKING_SET bytes
        # (X, both Y and the touched adapters' weights of every layer), past
        # the 256 MB last-level cache, and at least 8.
        per_layer = 2 * T * h * 5 + touched * 2 * r * h * 6
        n_layers = max(8, -(-FLAT_WORKING_SET // per_layer))
        layers = [dict(wa_q=rn((N, 1, r, h), .02), wb_q=[rn((N, 1, h, r), .02) for _ in range(3)],
                       wa_o=rn((N, 1, r, h), .02), wb_o=rn((N, 1, h, r), .02), x=rn((T, h), 1.),
                       y_q=rn((T, 3 * h), 1.), y_o=rn((T, h), 1.)) for _ in range(n_layers)]

        def step():
            engine.build_seg_bounds(idx)
            for ly in layers:
                engine.add_lora_slices(ly["y_q"], ly["x"], ly["wa_q"], ly["wb_q"], 0.5, offs)
                engine.add_lora_packed(ly["y_o"], ly["x"], ly["wa_o"], ly["wb_o"], 0.5)

        us, _ = graph_us(step, reps)
        nbytes = n_layers * (wl.algorithmic_bytes(T, h, 3 * h, [r] * touched) + wl.algorithmic_bytes(T, h, h, [r] * touched))
        pair = us / n_layers
        rows.append({"resident": N, "touched": touched, "layers": n_layers,
                     "working_set_MiB": round(n_layers * per_layer / 2 ** 20, 1), "us_per_graph": round(us, 2),
                     "us_per_qkv_o_pair": round(pair, 3), "us_per_80_call_step": round(pair * 40, 1),
                     "GB_s": round(nbytes / (us * 1e-6) / 1e9, 1)})
        log(f"flatness{' (sorted)' if sort else ''} N={N}: {rows[-1]}")
        del layers
        torch.cuda.empty_cache()
    assert engine.device_errors() == 0
    lat = [x["us_per_qkv_o_pair"] for x in rows]
    return {"rows": rows, "max_over_min_latency": round(max(lat) / min(lat), 3), "target_max_over_min": 1.15}


def run_flatness(args):
    res = measure_flatness(max(5, args.steps))
    res_s = measure_flatness(max(5, args.steps), sort=True)
    emit({"workload": "cfg2 flatness: resident adapters 1..128, layers x (qkv, o_proj) + build_seg_bounds per graph, "
                      "at least 8 layers and 512 MiB read per replay",
          **res, "sorted_routing": res_s})


def measure_cfg1_gpu(reps, sort=False):
    """BASELINE configs[0] on the GPU: h=4096, r=16, 4 adapters, 64 uniformly
    routed tokens (sort: the same tokens sorted by adapter), fp16, scale 1;
    us per add_lora call (a graph of calls over distinct copies of the
    inputs, FLAT_WORKING_SET bytes of them, so that no call finds its
    operands in the last-level cache)."""
    import torch

    from adapterslotsplusplus_amd import WarpPipeEngine
    from adapterslotsplusplus_amd import workloads as wl

    dt = torch.float16
    idx, x, wa, wb = cfg1_inputs()
    if sort:
        idx = torch.sort(idx).values
    nbytes = wl.algorithmic_bytes(64, 4096, 4096, [16] * len(set(idx.tolist())))
    engine = WarpPipeEngine()
    assert engine.build_seg_bounds(idx.cuda())
    per_copy = 4 * 64 * 4096 * 2  # x, A, B, y: 512 KiB each
    copies = [(x.cuda(), wa.cuda(), wb.cuda(), torch.zeros(64, 4096, dtype=dt, device="cuda"))
              for _ in range(-(-FLAT_WORKING_SET // per_copy))]

    def calls():
        for xc, ac, bc, yc in copies:
            engine.add_lora_packed(yc, xc, ac, bc, 1.0)

    us, _ = graph_us(calls, reps)
    us /= len(copies)
    return {"us_per_call": round(us, 3), "bytes_per_call": nbytes, "GB_s": round(nbytes / (us * 1e-6) / 1e9, 1),
            "calls_per_graph": len(copies), "working_set_MiB": round(len(copies) * per_copy / 2 ** 20, 1)}


def cfg1_inputs():
    """BASELINE configs[0]'s inputs on the host: 64 tokens uniform over 4
    adapters (seed 0), h=4096, r=16, fp16."""
    import torch

    from adapterslotsplusplus_amd import workloads as wl

    dt = torch.float16
    idx = wl.uniform_indices(64, 4, seed=0)
    x = wl.normal((64, 4096), 1.0, dt, 10)
    wa = wl.normal((4, 1, 16, 4096), 0.02, dt, 11)
    wb = wl.normal((4, 1, 4096, 16), 0.02, dt, 12)
    return idx, x, wa, wb


def cpu_baseline_cfg1(seconds):
    """BASELINE configs[0] (the reference's CPU-runnable case) through the
    oracle's per-segment torch fp32 path on this host's cores: us per
    add_lora call (median)."""
    import torch

    from adapterslotsplusplus_amd import workloads as wl
    from oracle import bgmv
    from oracle import segments as so

    idx, x, wa, wb = cfg1_inputs()
    nbytes = wl.algorithmic_bytes(64, 4096, 4096, [16] * len(set(idx.tolist())))
    segs = so.seg_bounds(idx.numpy()).tolist()
    y = torch.zeros(64, 4096, dtype=torch.float16)
    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    for _ in range(3):
        bgmv.add_lora(y, x, wa, wb, 1.0, segs)
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 20:
        t0 = time.perf_counter()
        bgmv.add_lora(y, x, wa, wb, 1.0, segs)
        times.append(time.perf_counter() - t0)
    times.sort()
    cpu_us = times[len(times) // 2] * 1e6
    return {"us_per_call": round(cpu_us, 1), "GB_s": round(nbytes / (cpu_us * 1e-6) / 1e9, 3), "cores": cores,
            "kind": "port", "runs": len(times),
            "sample": (f"{len(times)} add_lora calls of cfg1 (T=64, h=4096, r=16, 4 adapters uniform, seed 0, fp16; "
                       f"{len(segs)} run-length segments), torch fp32 per segment")}


def run_cfg1(args):
    """one call on the GPU and the oracle on the host."""
    gpu = measure_cfg1_gpu(max(5, args.steps))
    gpu_s = measure_cfg1_gpu(max(5, args.steps), sort=True)
    cpu = cpu_baseline_cfg1(min(args.cpu_seconds, 10.0))
    emit({"workload": "cfg1: T=64, h=4096, r=16, 4 adapters uniform (seed 0), fp16, one add_lora call",
          "bytes_per_call": gpu["bytes_per_call"], "gpu_us_per_call": gpu["us_per_call"], "gpu_GB_s": gpu["GB_s"],
          "gpu_calls_per_graph": gpu["calls_per_graph"], "gpu_working_set_MiB": gpu["working_set_MiB"],
          "gpu_sorted_routing": {"us_per_call": gpu_s["us_per_call"], "GB_s": gpu_s["GB_s"]},
          "cpu_baseline": cpu})


def run_cfg3(args):
    """13B mixed-rank decode.  T=512 Zipf(1.1) (seed 3) over
    128 adapters with ranks uniform in {8,16,32,64} (seed 2), bf16, registered
    in the adapter store (one engine per layer-target: the store keeps one
    (A, B) per id, like the reference's); per layer gate and up
    (5120 -> r -> 13824) and down (13824 -> r -> 5120), each shrink + expand."""
    import torch

    from adapterslotsplusplus_amd import WarpPipeEngine
    from adapterslotsplusplus_amd import workloads as wl

    dev = torch.device("cuda", 0)
    dt, T, n_layers = torch.bfloat16, 512, 4
    g = torch.Generator().manual_seed(2)
    ranks = [int(v) for v in torch.tensor([8, 16, 32, 64])[torch.randint(0, 4, (128,), generator=g)]]
    idx = wl.zipf_indices(T, 128, 1.1, seed=3)
    touched = sorted(set(idx.tolist()))
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)

    def rn(shape, std):
        return (torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32) * std).to(dt)

    shapes = {"gate": (5120, 13824), "up": (5120, 13824), "down": (13824, 5120)}
    targets = []
    for _ in range(n_layers):
        for name, (d_in, d_out) in shapes.items():
            eng = WarpPipeEngine()
            for i in touched:
                rr = ranks[i]
                eng.register_adapter(i, rn((rr, d_in), .02), rn((d_out, rr), .02), 16.0 / rr, rank=rr)
            assert eng.build_seg_bounds(idx.to(dev))
            targets.append(dict(eng=eng, name=name, d_in=d_in, d_out=d_out, X=rn((T, d_in), 1.),
                                Y=rn((T, d_out), 1.), H=torch.zeros(T, 64, dtype=dt, device=dev)))
    torch.cuda.synchronize()

    def calls():
        for t in targets:
            H = t["eng"].shrink(t["X"], t["d_in"], 0, T, out=t["H"])
            t["eng"].expand(H, t["Y"], t["d_out"], 0)

    us, _ = graph_us(calls, max(5, args.steps))
    tr = [ranks[i] for i in touched]
    nbytes = n_layers * sum(wl.algorithmic_bytes(T, d_in, d_out, tr) for d_in, d_out in shapes.values())
    per = {}
    for name, (d_in, d_out) in shapes.items():
        sel = [t for t in targets if t["name"] == name]

        def one(sel=sel):
            for t in sel:
                H = t["eng"].shrink(t["X"], t["d_in"], 0, T, out=t["H"])
                t["eng"].expand(H, t["Y"], t["d_out"], 0)

        u, _ = graph_us(one, max(5, args.steps))
        b = wl.algorithmic_bytes(T, d_in, d_out, tr)
        per[name] = {"us_per_call": round(u / len(sel), 2), "bytes_per_call": b,
                     "GB_s": round(b / (u / len(sel) * 1e-6) / 1e9, 1)}

    # The same calls with the tokens sorted by adapter (every engine's plan
    # rebuilt outside the graph; the graph reads the plan from HBM).
    idx_sorted = torch.sort(idx).values.to(dev)
    for t in targets:
        assert t["eng"].build_seg_bounds(idx_sorted)
    torch.cuda.synchronize()
    us_sorted, _ = graph_us(calls, max(5, args.steps))
    for t in targets:
        assert t["eng"].build_seg_bounds(idx.to(dev))
    torch.cuda.synchronize()

    # The same targets through shrink_expand(): both halves in one launch.
    def fused_calls():
        for t in targets:
            t["eng"].shrink_expand(t["X"], t["Y"], t["d_out"], 0)

    uf, _ = graph_us(fused_calls, max(5, args.steps))

    # One multi-layer store per model layer (gate, up, down as store layers
    # 0, 1, 2): gate and up as one shrink_expand_slices launch on their shared
    # X, down through shrink_expand.
    from adapterslotsplusplus_amd import WarpPipeConfig
    stores = []
    for li in range(n_layers):
        eng = WarpPipeEngine(WarpPipeConfig(layer_stride=128))
        for k, name in enumerate(["gate", "up", "down"]):
            d_in, d_out = shapes[name]
            for i in touched:
                rr = ranks[i]
                eng.register_adapter(i, rn((rr, d_in), .02), rn((d_out, rr), .02), 16.0 / rr, rank=rr, layer=k)
        assert eng.build_seg_bounds(idx.to(dev))
        stores.append(dict(eng=eng, X=rn((T, 5120), 1.), Y=rn((T, 2 * 13824), 1.), Xd=rn((T, 13824), 1.),
                           Yd=rn((T, 5120), 1.)))
    torch.cuda.synchronize()

    def store_calls():
        for st in stores:
            st["eng"].shrink_expand_slices(st["X"], st["Y"], [0, 1], [13824, 13824], [0, 13824])
            st["eng"].shrink_expand(st["Xd"], st["Yd"], 5120, 0, layer=2)

    us_s, _ = graph_us(store_calls, max(5, args.steps))
    nbytes_s = n_layers * (wl.algorithmic_bytes_nslice(T, 5120, [13824, 13824], tr)
                           + wl.algorithmic_bytes(T, 13824, 5120, tr))
    emit({"workload": f"cfg3: 13B mixed-rank decode, T=512, 128 adapters ({len(touched)} touched), ranks {{8,16,32,64}}, "
                      f"bf16, {n_layers} layers x (gate, up, down), shrink + expand per target",
          "us_per_layer": round(us / n_layers, 2), "GB_s": round(nbytes / (us * 1e-6) / 1e9, 1), "per_target": per,
          "sorted_routing": {"us_per_layer": round(us_sorted / n_layers, 2),
                             "GB_s": round(nbytes / (us_sorted * 1e-6) / 1e9, 1)},
          "shrink_expand_one_launch": {"us_per_layer": round(uf / n_layers, 2),
                                       "GB_s": round(nbytes / (uf * 1e-6) / 1e9, 1)},
          "gate_up_one_launch": {"us_per_layer": round(us_s / n_layers, 2),
                                 "GB_s": round(nbytes_s / (us_s * 1e-6) / 1e9, 1),
                                 "note": "gate+up through shrink_expand_slices on their shared X, down through "
                                         "shrink_expand; one multi-layer store per model layer"}})


def run_cfg4(args):
    """prefill chunk, T=8192 over 16 adapters (lognormal(6,1)
    segment lengths, seed 4), r=64, fp16: per layer the packed q/k/v call
    (3 x 4096 outputs sharing X) and the o call; 4 layers with distinct weights."""
    import torch

    from adapterslotsplusplus_amd import WarpPipeEngine
    from adapterslotsplusplus_amd import workloads as wl

    dev = torch.device("cuda", 0)
    dt, T, h, r, n_layers = torch.float16, 8192, 4096, 64, 4
    lens = wl.lognormal_segments(T, 16, 6.0, 1.0, seed=4)
    idx = torch.repeat_interleave(torch.arange(16), torch.tensor(lens)).to(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)

    def rn(shape, std):
        return (torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32) * std).to(dt)

    engine = WarpPipeEngine()
    layers = [dict(wa_q=rn((16, 1, r, h), .02), wb_q=[rn((16, 1, h, r), .02) for _ in range(3)],
                   wa_o=rn((16, 1, r, h), .02), wb_o=rn((16, 1, h, r), .02), x=rn((T, h), 1.),
                   y_q=rn((T, 3 * h), 1.), y_o=rn((T, h), 1.)) for _ in range(n_layers)]
    offs = [0, h, 2 * h]
    assert engine.build_seg_bounds(idx)

    def calls():
        for ly in layers:
            engine.add_lora_slices(ly["y_q"], ly["x"], ly["wa_q"], ly["wb_q"], 0.25, offs)
            engine.add_lora_packed(ly["y_o"], ly["x"], ly["wa_o"], ly["wb_o"], 0.25)

    us, _ = graph_us(calls, max(5, args.steps))
    calibration_copy(dev)
    b_q = wl.algorithmic_bytes(T, h, 3 * h, [r] * 16)
    b_o = wl.algorithmic_bytes(T, h, h, [r] * 16)
    f_q = wl.algorithmic_flops(T, h, 3 * h, [r] * T)
    f_o = wl.algorithmic_flops(T, h, h, [r] * T)
    per_layer = us / n_layers
    emit({"workload": "cfg4: prefill chunk T=8192, 16 adapters lognormal(6,1) (seed 4), r=64, fp16, "
                      f"{n_layers} layers x (packed q/k/v call, o call)",
          "us_per_layer": round(per_layer, 2), "bytes_per_layer": b_q + b_o, "flops_per_layer": f_q + f_o,
          "GB_s": round((b_q + b_o) / (per_layer * 1e-6) / 1e9, 1),
          "TFLOP_s": round((f_q + f_o) / (per_layer * 1e-6) / 1e12, 2),
          "hbm_frac": round((b_q + b_o) / (per_layer * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
          "mfma_frac_fp16_dense": round((f_q + f_o) / (per_layer * 1e-6) / 2.5e15, 5)})


CFG5_HOT = list(range(28))                         # device-resident tenants
CFG5_COLD = [list(range(28, 32)), list(range(32, 36))]  # staged from the pinned host store, alternate steps


def cfg5_routing(step):
    """32 tenants x 4 draft tokens, tenant-contiguous: the 28 hot tenants and
    this step's 4 cold ones, in a seeded order."""
    import torch

    tenants = CFG5_HOT + CFG5_COLD[step % 2]
    order = torch.randperm(32, generator=torch.Generator().manual_seed(500 + step))
    return torch.repeat_interleave(torch.tensor(tenants)[order], 4)


def measure_cfg5(reps, warmup):
    """draft step, h=2048, 22 layers x {q,k,v,o}, 32
    tenants x 4 draft tokens (T=128, tenant-contiguous), r=32, bf16, one HIP
    graph per step including build_seg_bounds.

    * 88 calls: every target its own add_lora (vLLM stacked weights);
    * 44 launches: per layer one q/k/v call with one A per slice
      (add_lora_packed_nslice) and one o call;
    * staged: the 88 targets through the multi-layer adapter store
      (shrink_expand per target); each step routes 4 cold tenants whose
      target-0 adapters live in the pinned host store: they are prefetched one
      step ahead on the prefetch stream, the step's stream waits for them on
      the device, the replay consumes them, and they are released after it
      (device errors 0 = every routed adapter was applied).  Compared with the
      same graph routed to resident tenants only."""
    import torch

    from adapterslotsplusplus_amd import WarpPipeConfig, WarpPipeEngine
    from adapterslotsplusplus_amd import workloads as wl

    dev = torch.device("cuda", 0)
    dt, T, L, h, r, n_layers = torch.bfloat16, 128, 32, 2048, 32, 22
    gen = torch.Generator(device=dev)
    gen.manual_seed(13)

    def rn(shape, std):
        return (torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32) * std).to(dt)

    out = {}
    engine = WarpPipeEngine()
    idx = torch.repeat_interleave(torch.arange(L), 4).to(dev)
    layers = [dict(wa=[rn((L, 1, r, h), .02) for _ in range(4)], wb=[rn((L, 1, h, r), .02) for _ in range(4)],
                   x=rn((T, h), 1.), y_qkv=rn((T, 3 * h), 1.), y=[rn((T, h), 1.) for _ in range(4)])
              for _ in range(n_layers)]

    def step88():
        engine.build_seg_bounds(idx)
        for ly in layers:
            for j in range(4):
                engine.add_lora_packed(ly["y"][j], ly["x"], ly["wa"][j], ly["wb"][j], 0.5)

    def step44():
        engine.build_seg_bounds(idx)
        for ly in layers:
            engine.add_lora_slices(ly["y_qkv"], ly["x"], ly["wa"][:3], ly["wb"][:3], 0.5, [0, h, 2 * h])
            engine.add_lora_packed(ly["y"][3], ly["x"], ly["wa"][3], ly["wb"][3], 0.5)

    us88, _ = graph_us(step88, reps)
    us44, _ = graph_us(step44, reps)
    assert engine.device_errors() == 0
    b88 = n_layers * 4 * wl.algorithmic_bytes(T, h, h, [r] * L)
    b44 = n_layers * (wl.algorithmic_bytes_nslice(T, h, [h] * 3, [r] * L) + wl.algorithmic_bytes(T, h, h, [r] * L))
    out["88_calls"] = {"us_per_step": round(us88, 1), "us_per_call": round(us88 / 88, 2), "bytes_per_step": b88,
                       "GB_s": round(b88 / (us88 * 1e-6) / 1e9, 1)}
    out["44_launches_nslice"] = {"us_per_step": round(us44, 1), "bytes_per_step": b44,
                                 "GB_s": round(b44 / (us44 * 1e-6) / 1e9, 1)}
    del layers, engine
    torch.cuda.empty_cache()

    # Adapter store: target t's adapter of tenant i under id t * 64 + i.
    n_t, stride = 4 * n_layers, 64
    store = WarpPipeEngine(WarpPipeConfig(layer_stride=stride, max_adapter_ids=n_t * stride))
    for t in range(n_t):
        for i in CFG5_HOT + CFG5_COLD[0] + CFG5_COLD[1]:
            A, B = rn((r, h), .02), rn((h, r), .02)
            if t == 0 and i >= 28:
                A, B = A.cpu(), B.cpu()
            store.register_adapter(i, A, B, 0.5, rank=r, layer=t)
    xs = [rn((T, h), 1.) for _ in range(n_t)]
    ys = [rn((T, h), 1.) for _ in range(n_t)]
    routes = [cfg5_routing(s).to(dev) for s in range(2)]
    hot_route = torch.repeat_interleave(torch.tensor(CFG5_HOT + CFG5_HOT[:4]), 4).to(dev)
    idx_buf = hot_route.clone()

    def step_store():
        store.build_seg_bounds(idx_buf)
        for t in range(n_t):
            store.shrink_expand(xs[t], ys[t], h, r, layer=t)

    us_hot, g = graph_us(step_store, reps)
    assert min(store.prefetch_adapters(CFG5_COLD[0], layer=0)) >= 0
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    n = warmup + reps
    host_s = 0.0
    for s in range(n):
        if s == warmup:
            e0.record()
            t0 = time.perf_counter()
        if s + 1 < n:
            assert min(store.prefetch_adapters(CFG5_COLD[(s + 1) % 2], layer=0)) >= 0
        assert store.wait_prefetches(CFG5_COLD[s % 2], layer=0)
        idx_buf.copy_(routes[s % 2])
        g.replay()
        store.release_prefetches(CFG5_COLD[s % 2], layer=0)
    host_s = time.perf_counter() - t0
    e1.record()
    torch.cuda.synchronize()
    us_cold = e0.elapsed_time(e1) * 1e3 / reps
    errors = store.device_errors()
    b_store = n_t * wl.algorithmic_bytes(T, h, h, [r] * 32)
    out["adapter_store_88_calls"] = {
        "us_per_step_resident_only": round(us_hot, 1),
        "us_per_step_with_4_cold_staged": round(us_cold, 1),
        "GB_s_with_4_cold_staged": round(b_store / (us_cold * 1e-6) / 1e9, 1),
        "host_us_per_step_with_4_cold_staged": round(host_s * 1e6 / reps, 1),
        "bytes_per_prefetch": 2 * r * h * 2, "device_errors": errors,
        "cold_adapters_consumed": errors == 0}
    del store, xs, ys
    torch.cuda.empty_cache()
    return out


def run_cfg5(args):
    res = measure_cfg5(max(5, args.steps), max(1, args.warmup))
    emit({"workload": "cfg5: draft step, h=2048, 22 layers x (q, k, v, o), T=128 (32 tenants x 4), r=32, bf16, "
                      "build_seg_bounds + the layers' calls in one graph per step", **res})


def run_draft(args):
    """The cfg5 draft step as a model forward: 22 blocks of q/k/v/o linears
    (h=2048, bf16, synthetic weights) on T=128 tokens (32 tenants x 4), every
    projection wrapped by WarpPipeLoRALinear (r=32, one adapter per tenant);
    routing table + forward in one graph.  The same model with LoRA off gives
    the base-linear cost, so the difference is what the adapters add."""
    import torch
    import torch.nn as nn
    import torch.nn.functional as F

    from adapterslotsplusplus_amd import WarpPipeEngine
    from adapterslotsplusplus_amd.lora_linear import DraftLoRAContext, wrap_linears

    dev = torch.device("cuda", 0)
    dt, T, L, h, r, n_layers = torch.bfloat16, 128, 32, 2048, 32, 22
    gen = torch.Generator(device=dev)
    gen.manual_seed(17)

    def rn(shape, std):
        return (torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32) * std).to(dt)

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            for n in ("q_proj", "k_proj", "v_proj", "o_proj"):
                lin = nn.Linear(h, h, bias=False, device=dev, dtype=dt)
                with torch.no_grad():
                    lin.weight.copy_(rn((h, h), 0.02))
                setattr(self, n, lin)

        def forward(self, x):
            a = self.q_proj(x) + self.k_proj(x) + self.v_proj(x)
            return x + self.o_proj(F.silu(a))

    model = nn.Sequential(*[Block() for _ in range(n_layers)]).eval()
    engine = WarpPipeEngine()
    ctx = DraftLoRAContext(engine, T, scale=2.0, device=dev)
    weights = {f"{i}.{n}": (rn((L, r, h), .02), rn((L, h, r), .02))
               for i in range(n_layers) for n in ("q_proj", "k_proj", "v_proj", "o_proj")}
    wrap_linears(model, weights, ctx)
    ctx.set_routing(torch.repeat_interleave(torch.arange(L, device=dev), 4))
    x = rn((T, h), 1.0)

    # The forked alternative, measured beside the product's in-place apply:
    # the delta on a second (default-priority) stream into a buffer of its
    # own, concurrently with the base GEMM, added to the GEMM's output after
    # the join.  The side stream runs every delta, so two applies never run
    # at once (they share the engine's partial buffer).
    side = torch.cuda.Stream()
    deltas = {}

    def forked(mod, xx):
        main = torch.cuda.current_stream()
        d = deltas.get(id(mod))
        if d is None:
            d = deltas[id(mod)] = torch.empty(T, mod.out_features, dtype=dt, device=dev)
        side.wait_stream(main)
        with torch.cuda.stream(side):
            d.zero_()
            assert ctx.engine.add_lora_packed(d, xx.reshape(-1, mod.in_features), mod.wa_t_all, mod.wb_t_all,
                                              ctx.scale)
        y = F.linear(xx, mod.weight, mod.bias)
        main.wait_stream(side)
        return y.add_(d)

    lora_mods = [m for m in model.modules() if hasattr(m, "wa_t_all")]
    res = {}
    with torch.inference_mode():
        for mode in ("none", "lora", "forked", "fused"):
            ctx.mode = "lora" if mode in ("forked", "fused") else mode
            ctx.fused_linear = mode == "fused"
            for m in lora_mods:
                if mode == "forked":
                    m.forward = (lambda mm: (lambda xx: forked(mm, xx)))(m)
                else:
                    m.__dict__.pop("forward", None)

            def step():
                ctx.begin_step()
                return model(x)

            us, _ = graph_us(step, max(5, args.steps))
            res[mode] = us
        for m in lora_mods:
            m.__dict__.pop("forward", None)
        ctx.fused_linear = False

    # The same draft model with q/k/v packed: one base GEMM over their
    # stacked weights and one LoRA launch with one adapter pair per
    # projection (WarpPipeLoRAPackedLinear), o_proj as before.
    from adapterslotsplusplus_amd.lora_linear import WarpPipeLoRAPackedLinear, WarpPipeLoRALinear

    class PackedBlock(nn.Module):
        def __init__(self, i):
            super().__init__()
            bases = []
            for n in ("q_proj", "k_proj", "v_proj"):
                lin = nn.Linear(h, h, bias=False, device=dev, dtype=dt)
                with torch.no_grad():
                    lin.weight.copy_(rn((h, h), 0.02))
                bases.append(lin)
            ws = [weights[f"{i}.{n}"] for n in ("q_proj", "k_proj", "v_proj")]
            self.qkv = WarpPipeLoRAPackedLinear(bases, [w[0] for w in ws], [w[1] for w in ws], ctx)
            o = nn.Linear(h, h, bias=False, device=dev, dtype=dt)
            with torch.no_grad():
                o.weight.copy_(rn((h, h), 0.02))
            self.o_proj = WarpPipeLoRALinear(o, *weights[f"{i}.o_proj"], ctx)

        def forward(self, x):
            q, k, v = self.qkv(x)
            return x + self.o_proj(F.silu(q + k + v))

    packed = nn.Sequential(*[PackedBlock(i) for i in range(n_layers)]).eval()
    res_p = {}
    with torch.inference_mode():
        for mode in ("none", "lora"):
            ctx.mode = mode

            def step_p():
                ctx.begin_step()
                return packed(x)

            us, _ = graph_us(step_p, max(5, args.steps))
            res_p[mode] = us
    emit({"workload": "draft step: 22 x (q, k, v, o) bf16 linears h=2048 on T=128 (32 tenants x 4), "
                      "WarpPipeLoRALinear r=32 on all 88, routing table + forward in one graph",
          "us_per_step_base_only": round(res["none"], 1), "us_per_step_with_lora": round(res["lora"], 1),
          "lora_us_per_step": round(res["lora"] - res["none"], 1),
          "lora_us_per_call": round((res["lora"] - res["none"]) / 88, 2),
          "fused_linear": {"us_per_step": round(res["fused"], 1),
                           "lora_us_per_call": round((res["fused"] - res["none"]) / 88, 2),
                           "note": "each projection's base GEMM and LoRA delta as one launch (engine.linear_lora, "
                                   "DraftLoRAContext(fused_linear=True)); lora_us_per_call is the step's time over the "
                                   "base-only step per projection"},
          "forked_delta": {"us_per_step": round(res["forked"], 1),
                           "lora_us_per_call": round((res["forked"] - res["none"]) / 88, 2),
                           "note": "delta on a forked stream beside the base GEMM, added after the join "
                                   "(not used by WarpPipeLoRALinear)"},
          "packed_qkv": {"us_per_step_base_only": round(res_p["none"], 1),
                         "us_per_step_with_lora": round(res_p["lora"], 1),
                         "lora_us_per_step": round(res_p["lora"] - res_p["none"], 1),
                         "lora_us_per_layer": round((res_p["lora"] - res_p["none"]) / n_layers, 2),
                         "note": "q/k/v as one WarpPipeLoRAPackedLinear (one base GEMM over the stacked weights, "
                                 "one LoRA launch with an adapter pair per projection), o_proj as "
                                 "WarpPipeLoRALinear: 44 LoRA launches per step"}})


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU figures are not part of it",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

    if args.workload != "cfg2":
        torch.cuda.set_device(0)
        {"flatness": run_flatness, "cfg1": run_cfg1, "cfg3": run_cfg3, "cfg4": run_cfg4,
         "cfg5": run_cfg5, "draft": run_draft}[args.workload](args)
        return

    from adapterslotsplusplus_amd import WarpPipeEngine
    from adapterslotsplusplus_amd import workloads as wl

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    c = wl.CFG2
    T, L, r, h, dt = c["T"], c["n_adapters"], c["rank"], c["hidden"], c["dtype"]
    n_layers = args.layers
    idx = wl.zipf_indices(T, L, c["zipf_s"], c["routing_seed"]).to(dev)
    touched = len(set(idx.tolist()))
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)

    def rn(shape, std):
        return (torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32) * std).to(dt)

    log(f"allocating {n_layers} layers of weights")
    layers = []
    for _ in range(n_layers):
        layers.append(dict(
            wa_q=rn((L, 1, r, h), 0.02), wb_q=[rn((L, 1, h, r), 0.02) for _ in range(3)],
            wa_o=rn((L, 1, r, h), 0.02), wb_o=rn((L, 1, h, r), 0.02),
            x_q=rn((T, h), 1.0), y_q=rn((T, 3 * h), 1.0), x_o=rn((T, h), 1.0), y_o=rn((T, h), 1.0)))
    bytes_qkv = wl.algorithmic_bytes(T, h, 3 * h, [r] * touched)
    bytes_o = wl.algorithmic_bytes(T, h, h, [r] * touched)
    bytes_step = n_layers * (bytes_qkv + bytes_o)

    engine = WarpPipeEngine()
    offs = [0, h, 2 * h]

    def calls():
        for ly in layers:
            engine.add_lora_slices(ly["y_q"], ly["x_q"], ly["wa_q"], ly["wb_q"], 0.5, offs)
            engine.add_lora_packed(ly["y_o"], ly["x_o"], ly["wa_o"], ly["wb_o"], 0.5)

    def step():
        engine.build_seg_bounds(idx)
        calls()

    log("eager warmup")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert engine.device_errors() == 0

    log("capturing the step graph")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        g.replay()
    torch.cuda.synchronize()

    log(f"timing {args.steps} graph replays")
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record()
    for _ in range(args.steps):
        g.replay()
    ev1.record()
    torch.cuda.synchronize()
    ms_step = ev0.elapsed_time(ev1) / args.steps
    value = bytes_step / (ms_step * 1e-3) / 1e9
    assert engine.device_errors() == 0

    # Each of 200 further replays timed on its own (an event pair around
    # every replay): the median and the spread beside the mean above.
    n_med = 200
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n_med)]
    for e0_, e1_ in evs:
        e0_.record()
        g.replay()
        e1_.record()
    torch.cuda.synchronize()
    per = sorted(e0_.elapsed_time(e1_) * 1e3 for e0_, e1_ in evs)
    step_median = {"replays": n_med, "median_us": round(per[n_med // 2], 2), "p10_us": round(per[n_med // 10], 2),
                   "p90_us": round(per[(9 * n_med) // 10], 2)}
    del g

    # The same step with the tokens sorted by adapter (the same per-adapter
    # token counts, fewer and longer runs): the plan groups tokens by adapter
    # either way, so the apply kernels see the same blocks.
    sorted_us = None
    if not args.no_secondary:
        log("sorted routing")
        idx_unsorted = idx.clone()
        idx.copy_(torch.sort(idx_unsorted).values)
        gs = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gs):
            step()
        for _ in range(args.warmup):
            gs.replay()
        torch.cuda.synchronize()
        ev0.record()
        for _ in range(args.steps):
            gs.replay()
        ev1.record()
        torch.cuda.synchronize()
        sorted_us = ev0.elapsed_time(ev1) * 1e3 / args.steps
        assert engine.device_errors() == 0
        del gs
        idx.copy_(idx_unsorted)

    # Per-launch durations of the two fused kernels (one launch per call),
    # over the 40 distinct layers so no call hits in cache.
    engine.build_seg_bounds(idx)
    torch.cuda.synchronize()

    def qkv_call(ly):
        return lambda: engine.add_lora_slices(ly["y_q"], ly["x_q"], ly["wa_q"], ly["wb_q"], 0.5, offs)

    def o_call(ly):
        return lambda: engine.add_lora_packed(ly["y_o"], ly["x_o"], ly["wa_o"], ly["wb_o"], 0.5)

    reps = max(1, args.steps // 2)
    qkv_us = launch_duration_us([qkv_call(ly) for ly in layers], reps)
    o_us = launch_duration_us([o_call(ly) for ly in layers], reps)
    achieved = bytes_qkv / (qkv_us * 1e-6) / 1e9

    del layers
    torch.cuda.empty_cache()

    log("floor: read probe")
    fl = measure_floor(engine, dev, n_layers, [bytes_qkv, bytes_o], reps)
    floor_step_us = n_layers * (fl[bytes_qkv] + fl[bytes_o])
    log("floor: handoff probe")
    x_bytes = 2 * T * h
    a_side = 2 * touched * r * h + x_bytes
    ho = measure_handoff(dev, n_layers, {
        "qkv": (a_side, 2 * touched * r * 3 * h + 2 * T * 3 * h, 2 * T * 3 * h),
        "o_proj": (a_side, 2 * touched * r * h + 2 * T * h, 2 * T * h)}, reps)

    copy_gbs = calibration_copy(dev)
    traffic, traffic_on = pmc_traffic()

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "us_per_step": round(ms_step * 1e3, 2),
        "frac_of_hbm_peak": round(value / PEAK_HBM_GBS, 4),
        "us_per_step_individually_timed": step_median,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded Zipf routing, N(0,0.02^2) weights, N(0,1) activations)",
        "config": {
            "workload": "cfg2: Llama-7B decode step, 40 layers x (packed-qkv add_lora, o_proj add_lora), "
                        "build_seg_bounds + 80 calls in one HIP graph",
            "tokens": T, "resident_adapters": L, "touched_adapters": touched, "rank": r, "hidden": h,
            "layers": n_layers, "routing": "zipf(1.1), seed 1",
            "bytes_per_step": bytes_step,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "traffic_measured_on": traffic_on,
            "kernel": "wp::apply_kernel<__bf16, 32, kFusedMulti, 1> (packed-qkv call: shrink + expand, one launch)",
            "bytes_per_launch": bytes_qkv,
            "us_per_launch": round(qkv_us, 3),
            "other_kernels": {
                "wp::apply_kernel<__bf16, 32, kFused, 1> (o_proj call)": {
                    "us_per_launch": round(o_us, 3), "bytes_per_launch": bytes_o,
                    "achieved": round(bytes_o / (o_us * 1e-6) / 1e9, 2)},
            },
        },
        # What one launch needs just to read a call's bytes (wp_read_probe over
        # distinct buffers, graph of 40 launches), and an empty launch: the
        # step's calls cannot take less than floor_step_us.
        "floor": {
            "qkv_read_us": round(fl[bytes_qkv], 3),
            "o_proj_read_us": round(fl[bytes_o], 3),
            "empty_launch_us": round(fl[0], 3),
            "floor_step_us": round(floor_step_us, 1),
            "floor_step_frac_of_hbm_peak": round(bytes_step / (floor_step_us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
            "step_frac_of_floor": round(floor_step_us / (ms_step * 1e3), 4),
            "qkv_frac_of_floor": round(fl[bytes_qkv] / qkv_us, 4),
            "read_GB_s_qkv_bytes": round(bytes_qkv / (fl[bytes_qkv] * 1e-6) / 1e9, 1),
            "copy_GB_s_256MiB": round(copy_gbs, 1),
            "handoff_probe": ho,
        },
    }
    if not args.no_secondary:
        # The north star's other targets, on the same run: latency flatness
        # over 1..128 resident adapters, the cfg5 draft step, cfg1 per call.
        reps = max(10, args.steps)
        log("secondary: flatness")
        flat = measure_flatness(reps)
        log("secondary: cfg5 draft step")
        c5 = measure_cfg5(reps, max(2, args.warmup))
        log("secondary: flatness, sorted routing")
        flat_s = measure_flatness(reps, sort=True)
        log("secondary: cfg1")
        c1 = measure_cfg1_gpu(reps)
        c1_s = measure_cfg1_gpu(reps, sort=True)
        out["flatness_max_over_min"] = flat["max_over_min_latency"]
        out["cfg5_us_per_step"] = c5["44_launches_nslice"]["us_per_step"]
        out["cfg1_us_per_call"] = c1["us_per_call"]
        out["secondary"] = {
            "cfg2_sorted_routing": {"us_per_step": round(sorted_us, 2),
                                    "GB_s": round(bytes_step / (sorted_us * 1e-6) / 1e9, 2),
                                    "workload": "the cfg2 step with the same tokens sorted by adapter"},
            "flatness": {**flat, "workload": "cfg2 shapes, N resident adapters, layers x (qkv, o_proj) per graph "
                                             "(at least 8 layers and 512 MiB read per replay)",
                         "sorted_routing": flat_s},
            "cfg5_draft_step": {**c5, "workload": "h=2048, 22 layers x (q, k, v, o), T=128 (32 tenants x 4), r=32, "
                                                  "bf16, build_seg_bounds + the calls in one graph; cfg5_us_per_step "
                                                  "is the 44-launch form (q/k/v in one call, one A per slice)"},
            "cfg1": {**c1, "workload": "T=64, h=4096, r=16, 4 adapters uniform (seed 0), fp16, one add_lora call",
                     "sorted_routing": c1_s},
        }
    if not args.no_cpu_baseline:
        log("cpu baseline")
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
        log("cpu baseline: cfg1")
        out["cpu_baseline"]["cfg1"] = cpu_baseline_cfg1(min(args.cpu_seconds, 10.0))
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
