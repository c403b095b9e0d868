"""GPU: adapters registered by reference (register_adapter(..., copy=False),
wp_register_adapter_ref) -- the reference's pointer registry
(csrc/memory/adapter_store.h:21-27): nothing is copied, the kernels read the
caller's tensors, and updates to them are seen by later calls.  Checked
against the CPU oracle (oracle.bgmv.shrink / expand) on the same inputs."""
import gc

import numpy as np
import pytest
import torch

from adapterslotsplusplus_amd import WarpPipeEngine
from oracle import bgmv
from oracle import segments as so
from tests.helpers import announce, assert_close, randn

pytestmark = pytest.mark.gpu

T, D, O, R = 96, 1024, 768, 16
DT = torch.bfloat16


def reference(X, Y0, idx, adapters):
    segs = [sg for sg in so.seg_bounds(idx).tolist() if sg[0] in adapters]
    return bgmv.expand(bgmv.shrink(X, segs, adapters, 64, T), Y0, segs, adapters)


def test_by_reference_sees_updates_and_outlives_the_callers_names():
    announce("adapters registered by reference")
    engine = WarpPipeEngine()
    idx = np.random.default_rng(3).integers(-1, 6, size=T)
    X = randn((T, D), 1, DT)
    Y0 = randn((T, O), 2, DT)
    cpu, dev = {}, {}
    for i in range(6):
        A = randn((R, D), 10 + i, DT, 0.02)
        B = randn((O, R), 20 + i, DT, 0.02)
        cpu[i] = (A, B, 0.5 + 0.1 * i)
        dev[i] = (A.cuda(), B.cuda())
        # Ids 0..2 by reference, 3..5 copied: one plan serves both kinds.
        engine.register_adapter(i, dev[i][0], dev[i][1], 0.5 + 0.1 * i, rank=R, copy=i >= 3)
    Xd = X.cuda()
    assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())

    def run():
        Y = Y0.cuda()
        engine.shrink_expand(Xd, Y, O, 0)
        torch.cuda.synchronize()
        return Y

    assert_close(run(), reference(X, Y0, idx, cpu), "first call")
    # In-place updates: seen for the borrowed adapters, not for the copied.
    for i in (1, 4):
        dev[i][0].mul_(2.0)
        dev[i][1].add_(0.01)
    upd = dict(cpu)
    upd[1] = (dev[1][0].cpu(), dev[1][1].cpu(), cpu[1][2])
    assert_close(run(), reference(X, Y0, idx, upd), "after in-place updates")
    # The engine holds the borrowed tensors: dropping every other name keeps them.
    keep = {i: (t[0].cpu(), t[1].cpu()) for i, t in dev.items()}
    dev.clear()
    gc.collect()
    torch.cuda.empty_cache()
    scratch = torch.full((64 << 20,), 7, dtype=torch.uint8, device="cuda")  # reuse of freed memory, if any
    del scratch
    assert_close(run(), reference(X, Y0, idx, {i: (keep[i][0], keep[i][1], cpu[i][2]) if i < 3 else cpu[i]
                                               for i in range(6)}), "after the caller dropped its names")
    assert engine.device_errors() == 0
    # Eviction drops the reference; the id's tokens are then skipped.
    engine.evict_adapter(0)
    assert engine._lib.wp_has_adapter(engine._handle, 0) == 0
    Y = run()
    assert engine.device_errors() != 0
    rest = {i: (keep[i][0], keep[i][1], cpu[i][2]) if i < 3 else cpu[i] for i in range(1, 6)}
    assert_close(Y, reference(X, Y0, idx, rest), "after evicting a borrowed adapter")


def test_by_reference_prefetch_and_checks():
    announce("borrowed adapter staged; argument checks")
    engine = WarpPipeEngine()
    A = randn((R, D), 40, DT, 0.02).cuda()
    B = randn((O, R), 41, DT, 0.02).cuda()
    engine.register_adapter(7, A, B, 0.75, rank=R, copy=False)
    assert engine.prefetch_adapter(7) >= 0
    assert engine.wait_prefetch(7)
    idx = np.full(T, 7)
    X = randn((T, D), 42, DT)
    Y0 = randn((T, O), 43, DT)
    assert engine.build_seg_bounds(torch.from_numpy(idx).cuda())
    Y = Y0.cuda()
    engine.shrink_expand(X.cuda(), Y, O, R)
    torch.cuda.synchronize()
    assert_close(Y, reference(X, Y0, idx, {7: (A.cpu(), B.cpu(), 0.75)}), "staged from a borrowed adapter")
    assert engine.device_errors() == 0
    with pytest.raises(RuntimeError, match="CUDA tensors"):
        engine.register_adapter(8, A.cpu(), B.cpu(), 1.0, rank=R, copy=False)
    with pytest.raises(RuntimeError, match="aligned"):
        flat = torch.zeros(R * D + 1, dtype=DT, device="cuda")
        engine.register_adapter(8, flat[1:].view(R, D), B, 1.0, rank=R, copy=False)
