"""CPU: bench.py's contract pieces that need no GPU -- more than one GPU is
refused with a message, and the committed counter summary it quotes as
roofline.traffic carries the build it was read on."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


def test_traffic_figure_names_its_build():
    traffic, on = bench.pmc_traffic()
    with open(bench.PMC_SUMMARY) as f:
        p = json.load(f)
    assert traffic == int(p["hbm_bytes_per_launch"]) and traffic > 0
    assert on == p["measured_on"] and on
    # The summary's own figures agree with each other.
    k = p["kernels"][p["kernel"]]
    assert k["hbm_bytes_per_launch"] == traffic
    assert abs(p["traffic_over_algorithmic"] - traffic / p["algorithmic_bytes_per_launch"]) < 1e-3
