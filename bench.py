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

Prints one JSON line.  `--gpus N` with N > 1 exits: this build runs on one GPU.
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
METRIC = "shrink+expand achieved HBM GB/s (% of peak); us per 80-call decode step"


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline sample length")
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
    """HBM bytes per launch of the qkv apply kernel from the committed PMC
    summary, or None."""
    try:
        with open(PMC_SUMMARY) as f:
            p = json.load(f)
        return int(p["hbm_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU figures are not part of it",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

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

    # Calibration copy for the PMC runs: reads and writes COPY_BYTES once.
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst

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
            "traffic": pmc_traffic(),
            "kernel": "wp::apply_kernel<__bf16, 32, kFusedMulti> (packed-qkv call: shrink + expand, one launch)",
            "bytes_per_launch": bytes_qkv,
            "us_per_launch": round(qkv_us, 3),
            "other_kernels": {
                "wp::apply_kernel<__bf16, 32, kFused> (o_proj call)": {
                    "us_per_launch": round(o_us, 3), "bytes_per_launch": bytes_o,
                    "achieved": round(bytes_o / (o_us * 1e-6) / 1e9, 2)},
            },
        },
    }
    if not args.no_cpu_baseline:
        log("cpu baseline")
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
