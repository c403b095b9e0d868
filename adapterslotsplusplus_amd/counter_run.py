"""The program the HBM counter summaries are read over (`rocprofv3 --pmc`):
the cfg2 decode calls launched eagerly, one stream, no HIP graph, then one
device copy of known size for the counters' calibration.

    rocprofv3 --pmc FETCH_SIZE -d <dir> -o run -- python3 -m adapterslotsplusplus_amd.counter_run
    rocprofv3 --pmc WRITE_SIZE -d <dir> -o run -- python3 -m adapterslotsplusplus_amd.counter_run

Workload: BASELINE.json configs[1] -- T=256 tokens routed Zipf(1.1) (seed 1)
over 64 resident adapters, rank 32, h=4096, bf16 -- as `--layers` layers of
distinct weights, each a packed-qkv call (3 x 4096 outputs, one shared A) and
an o_proj call, after one build_seg_bounds; `--passes` passes over the
layers.  The calibration copy reads and writes COPY_BYTES once
(`__amd_rocclr_copyBuffer`), after everything else.

Eager launches (instead of bench.py's graph replays) keep the profiler's
per-dispatch counter collection on the ordinary dispatch path."""
import argparse
import sys

COPY_BYTES = 256 << 20


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--passes", type=int, default=3)
    args = ap.parse_args(argv)

    import torch

    from . import workloads as wl
    from .engine import WarpPipeEngine

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    c = wl.CFG2
    T, L, r, h = c["T"], c["n_adapters"], c["rank"], c["hidden"]
    dt = torch.bfloat16
    idx = wl.zipf_indices(T, L, c["zipf_s"], c["routing_seed"]).to(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)

    def rn(shape, std):
        return (torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32) * std).to(dt)

    print(f"[counter_run] allocating {args.layers} layers", flush=True)
    layers = [dict(wa_q=rn((L, 1, r, h), .02), wb_q=[rn((L, 1, h, r), .02) for _ in range(3)],
                   wa_o=rn((L, 1, r, h), .02), wb_o=rn((L, 1, h, r), .02), x_q=rn((T, h), 1.), x_o=rn((T, h), 1.),
                   y_q=rn((T, 3 * h), 1.), y_o=rn((T, h), 1.)) for _ in range(args.layers)]
    engine = WarpPipeEngine()
    offs = [0, h, 2 * h]
    assert engine.build_seg_bounds(idx)
    for p in range(args.passes):
        for ly in layers:
            engine.add_lora_slices(ly["y_q"], ly["x_q"], ly["wa_q"], ly["wb_q"], 0.5, offs)
            engine.add_lora_packed(ly["y_o"], ly["x_o"], ly["wa_o"], ly["wb_o"], 0.5)
        torch.cuda.synchronize()
        print(f"[counter_run] pass {p + 1} of {args.passes}: {2 * args.layers} calls", flush=True)
    errors = engine.device_errors()
    if errors:
        raise RuntimeError(f"device error word 0x{errors:x}")
    del layers
    torch.cuda.empty_cache()
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(f"[counter_run] calibration copy of {COPY_BYTES} bytes done", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
