"""GPU: staging slots, the pinned host store, eviction and stress, mirroring
tests/unit/test_staging_buffer.py and tests/stress/*.py of the reference with
every output checked against the CPU oracle."""
import random
import time

import pytest
import torch

from adapterslotsplusplus_amd import WarpPipeConfig, WarpPipeEngine
from oracle import bgmv
from oracle import segments as so
from tests.helpers import announce, assert_close, randn

pytestmark = pytest.mark.gpu

R, D, O = 32, 4096, 4096
ALPHA = 16.0 / 32
SLOTS = 8  # reference WP_MAX_STAGING


def make_engine(k, dtype=torch.float16, seed=0, host=False):
    engine = WarpPipeEngine()
    A = randn((k, R, D), seed, dtype, 0.02)
    B = randn((k, O, R), seed + 1, dtype, 0.02)
    adapters = {}
    for i in range(k):
        a, b = A[i].contiguous(), B[i].contiguous()
        engine.register_adapter(i, a if host else a.cuda(), b if host else b.cuda(), ALPHA)
        adapters[i] = (A[i], B[i], ALPHA)
    return engine, adapters


def wait_ready(engine, aid, timeout_s=5.0):
    deadline = time.time() + timeout_s
    while time.time() < deadline:
        if engine.is_prefetch_ready(aid):
            return True
        time.sleep(0.001)
    return False


def test_acquire_and_ready():
    """test_staging_buffer.py:39-45."""
    engine, _ = make_engine(1)
    assert not engine.is_prefetch_ready(0)
    slot = engine.prefetch_adapter(0)
    assert slot >= 0
    assert wait_ready(engine, 0)


def test_pool_exhaustion_is_safe():
    """test_staging_buffer.py:48-63: 8 succeed, 2 get -1."""
    engine, _ = make_engine(SLOTS + 2)
    slots = [engine.prefetch_adapter(i) for i in range(SLOTS + 2)]
    assert sum(s >= 0 for s in slots) == SLOTS
    assert sum(s == -1 for s in slots) == 2
    for i in range(SLOTS):
        assert wait_ready(engine, i)
    for i in range(SLOTS, SLOTS + 2):
        assert not engine.is_prefetch_ready(i)


def test_release_and_reacquire():
    """test_staging_buffer.py:66-75."""
    engine, _ = make_engine(2)
    s0 = engine.prefetch_adapter(0)
    assert wait_ready(engine, 0)
    engine.release_prefetch(0)
    assert not engine.is_prefetch_ready(0)
    s1 = engine.prefetch_adapter(1)
    assert s1 == s0
    assert wait_ready(engine, 1)


def test_idempotent_double_prefetch_and_unknown_id():
    """test_staging_buffer.py:78-86; unknown id -> -1 (bindings:47)."""
    engine, _ = make_engine(1)
    assert engine.prefetch_adapter(0) == engine.prefetch_adapter(0)
    assert wait_ready(engine, 0)
    assert engine.prefetch_adapter(12345) == -1
    engine.release_prefetch(12345)  # no-op


def test_slot_count_follows_config():
    engine = WarpPipeEngine(WarpPipeConfig(num_staging_slots=2))
    a = torch.zeros(R, 64, dtype=torch.float16, device="cuda")
    b = torch.zeros(64, R, dtype=torch.float16, device="cuda")
    for i in range(3):
        engine.register_adapter(i, a, b, 1.0)
    assert [engine.prefetch_adapter(i) for i in range(3)] == [0, 1, -1]


def test_host_resident_adapters_need_staging():
    """Cold adapters live in the pinned host store; prefetch stages them (H2D on
    the prefetch stream) and build_segments then reads the staged copy."""
    announce("host-resident staging")
    dtype = torch.bfloat16
    engine, adapters = make_engine(3, dtype=dtype, seed=5, host=True)
    with pytest.raises(RuntimeError, match="not staged"):
        engine.build_segments([0], [0, 4])
    for i in range(3):
        assert engine.prefetch_adapter(i) >= 0
        assert wait_ready(engine, i)
    X = randn((20, D), 6, dtype)
    Y0 = randn((20, O), 7, dtype)
    engine.build_segments([2, 0, 1], [0, 5, 12, 20])
    H = engine.shrink(X.cuda(), D, R, 20)
    Y = Y0.cuda()
    engine.expand(H, Y, O, R)
    torch.cuda.synchronize()
    segs = so.segment_table([2, 0, 1], [0, 5, 12, 20]).tolist()
    H_ref = bgmv.shrink(X, segs, adapters, R, 20)
    assert_close(H, H_ref, "H staged")
    assert_close(Y, bgmv.expand(H_ref, Y0, segs, adapters), "Y staged")


def test_prefetched_device_adapters_give_same_result():
    announce("staged vs direct")
    engine, adapters = make_engine(4, seed=9)
    X = randn((40, D), 10, torch.float16, 0.1)
    Y0 = randn((40, O), 11, torch.float16, 0.1)
    outs = []
    for staged in (False, True):
        if staged:
            for i in range(4):
                engine.prefetch_adapter(i)
                assert wait_ready(engine, i)
        engine.build_segments([0, 1, 2, 3], [0, 10, 20, 30, 40])
        H = engine.shrink(X.cuda(), D, R, 40)
        Y = Y0.cuda()
        engine.expand(H, Y, O, R)
        torch.cuda.synchronize()
        outs.append((H.cpu(), Y.cpu()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


def test_concurrent_adapters_random_subsets():
    """tests/stress/test_concurrent_adapters.py: K=32 pool, 25 iterations of a
    random subset with 1..32 tokens per adapter, random.Random(0)."""
    engine, adapters = make_engine(32, seed=20)
    rng = random.Random(0)
    for it in range(25):
        active = rng.sample(range(32), rng.randint(1, 32))
        tokens_per = {a: rng.randint(1, 32) for a in active}
        offs = [0]
        for a in active:
            offs.append(offs[-1] + tokens_per[a])
        T = offs[-1]
        announce(f"stress iter {it} T={T}")
        X = randn((T, D), 100 + it, torch.float16, 0.1)
        Y0 = randn((T, O), 200 + it, torch.float16, 0.1)
        engine.build_segments(active, offs)
        H = engine.shrink(X.cuda(), D, R, T)
        Y = Y0.cuda()
        engine.expand(H, Y, O, R)
        torch.cuda.synchronize()
        segs = so.segment_table(active, offs).tolist()
        H_ref = bgmv.shrink(X, segs, adapters, R, T)
        assert_close(H, H_ref, f"H iter {it}")
        assert_close(Y, bgmv.expand(H_ref, Y0, segs, adapters), f"Y iter {it}")


def test_burst_epochs_with_prefetch():
    """tests/stress/test_burst_workload.py:62-82: six alternating epochs."""
    engine, adapters = make_engine(16, seed=30)
    epochs = [
        (list(range(16)), {i: 8 for i in range(16)}, True),
        ([0], {0: 1}, False),
        (list(range(12)), {i: 16 for i in range(12)}, True),
        ([3, 7], {3: 2, 7: 1}, False),
        (list(range(16)), {i: 4 for i in range(16)}, False),
        ([0], {0: 1}, False),
    ]
    for e, (active, tokens_per, use_prefetch) in enumerate(epochs):
        announce(f"burst epoch {e}")
        if use_prefetch:
            for a in active[:SLOTS]:
                engine.prefetch_adapter(a)
            torch.cuda.synchronize()
        offs = [0]
        for a in active:
            offs.append(offs[-1] + tokens_per[a])
        T = offs[-1]
        X = randn((T, D), 300 + e, torch.float16, 0.1)
        Y0 = randn((T, O), 400 + e, torch.float16, 0.1)
        engine.build_segments(active, offs)
        H = engine.shrink(X.cuda(), D, R, T)
        Y = Y0.cuda()
        engine.expand(H, Y, O, R)
        torch.cuda.synchronize()
        segs = so.segment_table(active, offs).tolist()
        H_ref = bgmv.shrink(X, segs, adapters, R, T)
        assert_close(H, H_ref, f"H epoch {e}")
        assert_close(Y, bgmv.expand(H_ref, Y0, segs, adapters), f"Y epoch {e}")
        if use_prefetch:
            for a in active[:SLOTS]:
                engine.release_prefetch(a)


def test_eviction_under_load():
    """tests/stress/test_eviction_under_load.py:27-57: 40 register/use/evict
    cycles over ids mod 4, fresh tensors each cycle."""
    engine = WarpPipeEngine()
    for cycle in range(40):
        announce(f"evict cycle {cycle}")
        a = randn((R, D), 500 + cycle, torch.float16, 0.02)
        b = randn((O, R), 600 + cycle, torch.float16, 0.02)
        aid = cycle % 4
        engine.register_adapter(aid, a.cuda(), b.cuda(), ALPHA)
        engine.build_segments([aid], [0, 4])
        X = randn((4, D), 700 + cycle, torch.float16, 0.1)
        Y0 = randn((4, O), 800 + cycle, torch.float16, 0.1)
        H = engine.shrink(X.cuda(), D, R, 4)
        Y = Y0.cuda()
        engine.expand(H, Y, O, R)
        engine.evict_adapter(aid)
        torch.cuda.synchronize()
        H_ref = bgmv.shrink_rows(X, a, ALPHA)
        assert_close(H, H_ref, f"H cycle {cycle}")
        assert_close(Y, bgmv.expand_rows(H_ref, b, Y0), f"Y cycle {cycle}")
    with pytest.raises(RuntimeError, match="no segment table"):
        engine.shrink(torch.zeros(4, D, dtype=torch.float16, device="cuda"), D, R, 4)


def test_evict_releases_slot():
    """Eviction frees the id's staging slot (the reference keeps it, so a
    re-registered id can read stale staged weights)."""
    engine, _ = make_engine(SLOTS)
    for i in range(SLOTS):
        assert engine.prefetch_adapter(i) >= 0
    engine.evict_adapter(3)
    assert not engine.is_prefetch_ready(3)
    a = torch.zeros(R, D, dtype=torch.float16, device="cuda")
    b = torch.zeros(O, R, dtype=torch.float16, device="cuda")
    engine.register_adapter(99, a, b, 1.0)
    assert engine.prefetch_adapter(99) >= 0


def test_score_policy_keeps_top_adapters_staged():
    """ScorePrefetchPolicy over host-resident adapters: after each update the
    top-scored ones are staged and usable, the rest released; a step that
    routes to the staged set matches the oracle."""
    from adapterslotsplusplus_amd.prefetch_policy import ScorePrefetchPolicy

    announce("score-driven staging")
    engine, adapters = make_engine(10, seed=40, host=True)
    policy = ScorePrefetchPolicy(engine, slots=4)
    rng = random.Random(5)
    for it in range(3):
        scores = {a: rng.random() for a in range(10)}
        must = [it]
        policy.update(scores, must=must)
        want = policy.ranking(scores, must)[:4]
        assert sorted(policy.staged) == sorted(want)
        for a in want:
            assert wait_ready(engine, a)
        T = 48
        ids = [want[j % 4] for j in range(T)]
        X = randn((T, D), 41 + it, torch.float16, 0.1)
        Y0 = randn((T, O), 51 + it, torch.float16, 0.1)
        assert engine.build_seg_bounds(torch.tensor(ids, device="cuda"))
        H = engine.shrink(X.cuda(), D, R, T)
        Y = Y0.cuda()
        engine.expand(H, Y, O, R)
        torch.cuda.synchronize()
        segs = so.seg_bounds(ids).tolist()
        H_ref = bgmv.shrink(X, segs, adapters, R, T)
        assert_close(H, H_ref, f"H update {it}")
        assert_close(Y, bgmv.expand(H_ref, Y0, segs, adapters), f"Y update {it}")
        assert engine.device_errors() == 0
    policy.release_all()
    assert policy.staged == {}
