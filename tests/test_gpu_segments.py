"""GPU: the device-built segment table is bit-exact with the reference rule.

Mirrors the reference's segment checks (test_add_lora_packed.py index lists,
test_warp_pipe_graph_capture.py capture/replay lists, test_segment_builder.py)
through the known-answer fixtures, and compares the plan kernel with the CPU
oracle on random routings up to the 8192-token capacity, including the
internal by-adapter grouping (perm and blocks)."""
import json
import os

import numpy as np
import pytest
import torch

from adapterslotsplusplus_amd import WarpPipeConfig, WarpPipeEngine, _lib
from oracle import segments as so
from tests.helpers import announce

pytestmark = pytest.mark.gpu

@pytest.fixture(scope="module")
def engine():
    return WarpPipeEngine()


def kat(golden_dir, name):
    with open(os.path.join(golden_dir, name)) as f:
        return json.load(f)


def oracle_blocks(idx):
    """Blocks of at most wp_block_tokens(T) tokens cut from each adapter's group."""
    bt = _lib.load().wp_block_tokens(len(idx))
    perm, gid, goff = so.group_tokens(idx)
    blocks = []
    for g in range(gid.size):
        n = int(goff[g + 1] - goff[g])
        for j in range(0, n, bt):
            blocks.append((int(gid[g]), int(goff[g]) + j, min(bt, n - j), int(gid[g])))
    return perm.tolist(), blocks


@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
def test_known_answers(engine, golden_dir, dtype):
    for case in kat(golden_dir, "seg_bounds_kat.json")["cases"]:
        announce(f"seg_bounds KAT {case['source']} {dtype}")
        idx = torch.tensor(case["indices"], dtype=dtype, device="cuda")
        assert engine.build_seg_bounds(idx)
        assert engine.read_segments() == [tuple(s) for s in case["segments"]], case["source"]


def test_capacity_known_answers(golden_dir):
    for case in kat(golden_dir, "seg_bounds_kat.json")["capacity_cases"]:
        announce(f"seg_bounds capacity {case}")
        eng = WarpPipeEngine(WarpPipeConfig(max_tokens=case["max_tokens"]))
        idx = torch.zeros(case["total_tokens"], dtype=torch.int64, device="cuda")
        assert eng.build_seg_bounds(idx) is case["handled"]


def test_default_capacity_and_empty(engine):
    announce("seg_bounds T=0 and T=8193")
    assert engine.build_seg_bounds(torch.zeros(0, dtype=torch.int64, device="cuda"))
    assert engine.read_segments() == []
    assert engine.build_seg_bounds(torch.zeros(8193, dtype=torch.int64, device="cuda")) is False


@pytest.mark.parametrize("T", [1, 17, 64, 255, 256, 257, 1000, 2048, 2049, 5000, 8192])
def test_random_routings_match_oracle(engine, T):
    rng = np.random.default_rng(T)
    for trial in range(5):
        if trial == 0:
            idx = rng.integers(-1, 64, size=T)
        elif trial == 1:  # long runs
            idx = np.repeat(rng.integers(-1, 16, size=T), rng.integers(1, 90, size=T))[:T]
        elif trial == 2:  # Zipf-like
            p = 1.0 / np.arange(1, 129) ** 1.1
            idx = rng.choice(128, size=T, p=p / p.sum())
        elif trial == 3:  # large ids, sorted prefill-like runs
            idx = np.sort(rng.integers(0, 1 << 20, size=T))
        else:             # a dozen long runs, repeated ids (few runs: the plan's counting sort)
            cuts = np.sort(rng.choice(np.arange(1, max(T, 2)), size=min(11, max(T - 1, 0)), replace=False))
            idx = np.repeat(rng.integers(-1, 8, size=len(cuts) + 1), np.diff(np.concatenate([[0], cuts, [T]])))
        announce(f"seg_bounds random T={T} trial={trial}")
        t = torch.from_numpy(idx.astype(np.int64)).cuda()
        assert engine.build_seg_bounds(t)
        got = engine.read_segments()
        assert got == [tuple(s) for s in so.seg_bounds(idx).tolist()]
        perm, blocks = engine.read_plan()
        operm, oblocks = oracle_blocks(idx)
        assert perm == operm
        assert blocks == oblocks


def test_host_table_known_answers(engine, golden_dir):
    spec = kat(golden_dir, "segment_table_kat.json")
    A = torch.zeros(32, 64, dtype=torch.float16, device="cuda")
    B = torch.zeros(64, 32, dtype=torch.float16, device="cuda")
    for i in range(257):
        engine.register_adapter(i, A, B, 1.0, rank=32)
    for case in spec["cases"]:
        announce(f"build_segments KAT {case['source']}")
        engine.build_segments(case["ids"], case["offsets"])
        assert engine.read_segments() == [tuple(s) for s in case["segments"]]
    k = spec["generated_cases"][0]["k"]
    engine.build_segments(list(range(k)), list(range(k + 1)))
    assert engine.read_segments() == [(i, i, 1) for i in range(k)]
    with pytest.raises(RuntimeError, match="K\\+1"):
        engine.build_segments([0, 1], [0, 4])
    with pytest.raises(RuntimeError, match="WP_MAX_SEGMENTS"):
        engine.build_segments(list(range(257)), list(range(258)))
    with pytest.raises(RuntimeError, match="unknown adapter_id"):
        engine.build_segments([9999], [0, 4])
    for i in range(257):
        engine.evict_adapter(i)


def test_host_table_past_max_tokens_is_rejected():
    """A host table whose token rows reach past max_tokens is refused before
    any launch: large-plan calls index the engine's H scratch by token row."""
    announce("build_segments past max_tokens")
    eng = WarpPipeEngine(WarpPipeConfig(max_tokens=256))
    A = torch.zeros(32, 64, dtype=torch.float16, device="cuda")
    B = torch.zeros(64, 32, dtype=torch.float16, device="cuda")
    eng.register_adapter(0, A, B, 1.0, rank=32)
    with pytest.raises(RuntimeError, match="beyond max_tokens"):
        eng.build_segments([0], [500, 600])
    eng.build_segments([0], [200, 256])
    assert eng.read_segments() == [(0, 200, 56)]
