"""The program the HBM counter summaries are read over (`rocprofv3 --pmc`):
the cfg2 decode calls launched eagerly, one stream, no HIP graph, then one
device copy of known size for the counters' calibration.

    rocprofv3 --pmc FETCH_SIZE -d <dir> -o run -- python3 -m adapterslotsplusplus_amd.counter_run
    rocprofv3 --pmc WRITE_SIZE -d <dir> -o run -- python3 -m adapterslotsplusplus_amd.counter_run
    (add --workload cfg3 for the 13B mixed-rank decode's shrink() and expand())

Workload: BASELINE.json configs[1] -- T=256 tokens routed Zipf(1.1) (seed 1)
over 64 resident adapters, rank 32, h=4096, bf16 -- as `--layers` layers of
distinct weights, each a packed-qkv call (3 x 4096 outputs, one shared A) and
an o_proj call, after one build_seg_bounds; `--passes` passes over the
layers.  The calibration copy reads and writes COPY_BYTES once
(`__amd_rocclr_copyBuffer`), after everything else.

`--workload cfg3`: BASELINE.json configs[2] as bench.py's cfg3 record builds
it -- T=512 routed Zipf(1.1) (seed 3) over 128 adapters with ranks uniform in
{8, 16, 32, 64} (seed 2), bf16, registered in one engine per layer-target --
as `--layers` layers of gate, up and down, each a shrink() then an expand()
(dispatch order: gate shrink, gate expand, up shrink, up expand, down shrink,
down expand, layer after layer).

Eager launches (instead of bench.py's graph replays) keep the profiler's
per-dispatch counter collection on the ordinary dispatch path."""
import argparse
import sys

COPY_BYTES = 256 << 20


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--workload", default="cfg2", choices=["cfg2", "cfg3"])
    ap.add_argument("--layers", type=int, default=None, help="layers (default 40 for cfg2, 4 for cfg3)")
    ap.add_argument("--passes", type=int, default=3)
    args = ap.parse_args(argv)

    import torch

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.workload == "cfg3":
        run_cfg3(args.layers or 4, args.passes, dev)
    else:
        run_cfg2(args.layers or 40, args.passes, dev)
    calibration_copy(dev)
    return 0


def run_cfg2(n_layers, passes, dev):
    import torch

    from . import workloads as wl
    from .engine import WarpPipeEngine

    c = wl.CFG2
    T, L, r, h = c["T"], c["n_adapters"], c["rank"], c["hidden"]
    dt = torch.bfloat16
    idx = wl.zipf_indices(T, L, c["zipf_s"], c["routing_seed"]).to(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)

    def rn(shape, std):
        return (torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32) * std).to(dt)

    print(f"[counter_run] allocating {n_layers} layers", flush=True)
    layers = [dict(wa_q=rn((L, 1, r, h), .02), wb_q=[rn((L, 1, h, r), .02) for _ in range(3)],
                   wa_o=rn((L, 1, r, h), .02), wb_o=rn((L, 1, h, r), .02), x_q=rn((T, h), 1.), x_o=rn((T, h), 1.),
                   y_q=rn((T, 3 * h), 1.), y_o=rn((T, h), 1.)) for _ in range(n_layers)]
    engine = WarpPipeEngine()
    offs = [0, h, 2 * h]
    assert engine.build_seg_bounds(idx)
    for p in range(passes):
        for ly in layers:
            engine.add_lora_slices(ly["y_q"], ly["x_q"], ly["wa_q"], ly["wb_q"], 0.5, offs)
            engine.add_lora_packed(ly["y_o"], ly["x_o"], ly["wa_o"], ly["wb_o"], 0.5)
        torch.cuda.synchronize()
        print(f"[counter_run] pass {p + 1} of {passes}: {2 * n_layers} calls", flush=True)
    errors = engine.device_errors()
    if errors:
        raise RuntimeError(f"device error word 0x{errors:x}")
    del layers
    torch.cuda.empty_cache()


def run_cfg3(n_layers, passes, dev):
    import torch

    from . import workloads as wl
    from .engine import WarpPipeEngine

    dt, T = torch.bfloat16, 512
    g = torch.Generator().manual_seed(2)
    ranks = [int(v) for v in torch.tensor([8, 16, 32, 64])[torch.randint(0, 4, (128,), generator=g)]]
    idx = wl.zipf_indices(T, 128, 1.1, seed=3).to(dev)
    touched = sorted(set(idx.tolist()))
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)

    def rn(shape, std):
        return (torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32) * std).to(dt)

    shapes = (("gate", 5120, 13824), ("up", 5120, 13824), ("down", 13824, 5120))
    print(f"[counter_run] allocating {n_layers} layers x {len(shapes)} targets", flush=True)
    targets = []
    for _ in range(n_layers):
        for name, d_in, d_out in shapes:
            eng = WarpPipeEngine()
            for i in touched:
                rr = ranks[i]
                eng.register_adapter(i, rn((rr, d_in), .02), rn((d_out, rr), .02), 16.0 / rr, rank=rr)
            assert eng.build_seg_bounds(idx)
            targets.append(dict(eng=eng, d_in=d_in, d_out=d_out, X=rn((T, d_in), 1.), Y=rn((T, d_out), 1.),
                                H=torch.zeros(T, 64, dtype=dt, device=dev)))
    torch.cuda.synchronize()
    for p in range(passes):
        for t in targets:
            t["eng"].shrink(t["X"], t["d_in"], 0, T, out=t["H"])
            t["eng"].expand(t["H"], t["Y"], t["d_out"], 0)
        torch.cuda.synchronize()
        print(f"[counter_run] pass {p + 1} of {passes}: {2 * len(targets)} launches", flush=True)
    for t in targets:
        errors = t["eng"].device_errors()
        if errors:
            raise RuntimeError(f"device error word 0x{errors:x}")
    del targets
    torch.cuda.empty_cache()


def calibration_copy(dev):
    import torch

    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(f"[counter_run] calibration copy of {COPY_BYTES} bytes done", flush=True)


if __name__ == "__main__":
    sys.exit(main())
