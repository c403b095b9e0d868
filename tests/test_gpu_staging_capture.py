"""GPU: staging slots consumed inside captured steps, the adapter table's
device-side publication, its dtype check, and the partial buffer's repair
after a wait gives up.

The reference consumes a ready staging slot when the segment table is built
(csrc/dispatch/segment_builder.cpp:36-42; the kernels then read the staged
pointers, warp_pipe_r32.cu:81,162).  Here the prefetch stream publishes the
slot on the device once its copy has landed, every build_seg_bounds (captured
or not) writes ready publications into the adapter table, and a release
writes the registered entry back in stream order.  Every output is checked
against the CPU oracle on the same inputs."""
import pytest
import torch

from adapterslotsplusplus_amd import WarpPipeConfig, WarpPipeEngine, _lib
from oracle import bgmv
from oracle import segments as so
from tests.helpers import announce, assert_close, randn

pytestmark = pytest.mark.gpu

T, D, O, R = 128, 2048, 2048, 32
DT = torch.bfloat16
HOT = list(range(28))                       # device-resident tenants
COLD = [list(range(28, 32)), list(range(32, 36))]  # host-resident, staged per step


def register_all(engine, seed=0):
    adapters = {}
    for i in HOT + COLD[0] + COLD[1]:
        A = randn((R, D), seed + 2 * i, DT, 0.02)
        B = randn((O, R), seed + 2 * i + 1, DT, 0.02)
        alpha = 0.5 + 0.01 * i
        host = i >= 28
        engine.register_adapter(i, A if host else A.cuda(), B if host else B.cuda(), alpha, rank=R)
        adapters[i] = (A, B, alpha)
    return adapters


def routing(step):
    """32 request groups of 4 tokens: 28 hot tenants and this step's 4 cold ones."""
    tenants = HOT + COLD[step % 2]
    g = torch.Generator().manual_seed(1000 + step)
    order = torch.randperm(32, generator=g)
    return torch.repeat_interleave(torch.tensor(tenants)[order], 4)


def reference(adapters, X, Y0, idx):
    segs = so.seg_bounds(idx.tolist()).tolist()
    H = bgmv.shrink(X, segs, adapters, R, T)
    return bgmv.expand(H, Y0, segs, adapters)


def test_captured_step_consumes_staged_adapters_between_replays():
    """A cfg5-shaped step (build_seg_bounds + shrink_expand over the adapter
    store) captured once.  Between replays, the next step's cold adapters are
    prefetched one step ahead into free slots, the stream waits for them, and
    the previous step's are released; slots are reused every other step.  No
    host synchronisation between steps: each step's output is copied aside in
    stream order and all are checked at the end."""
    engine = WarpPipeEngine()
    adapters = register_all(engine)
    X = randn((T, D), 7, DT)
    Y0 = randn((T, O), 8, DT)
    Xd, Y, Y0d = X.cuda(), Y0.cuda(), Y0.cuda()
    idx_buf = routing(0).cuda()
    for a in COLD[0]:
        assert engine.prefetch_adapter(a) >= 0
        assert engine.wait_prefetch(a)

    def step():
        engine.build_seg_bounds(idx_buf)
        engine.shrink_expand(Xd, Y, O, R)

    Y.copy_(Y0d)
    step()
    torch.cuda.synchronize()
    assert_close(Y, reference(adapters, X, Y0, routing(0)), "eager step 0")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    n_steps = 8
    outs = [torch.empty_like(Y) for _ in range(n_steps)]
    routes = [routing(s) for s in range(n_steps)]
    routes_d = [r.cuda() for r in routes]
    announce("captured step with cold adapters staged between replays")
    for s in range(n_steps):
        # Odd steps use the per-id calls, even steps the batched ones.
        if s + 1 < n_steps:
            nxt = COLD[(s + 1) % 2]
            slots = engine.prefetch_adapters(nxt) if s % 2 == 0 else [engine.prefetch_adapter(a) for a in nxt]
            assert all(sl >= 0 for sl in slots), f"step {s}: no free slot for the next step ({slots})"
        if s % 2 == 0:
            assert engine.wait_prefetches(COLD[s % 2]), f"step {s}: a cold adapter holds no slot"
        else:
            for a in COLD[s % 2]:
                assert engine.wait_prefetch(a), f"step {s}: adapter {a} holds no slot"
        idx_buf.copy_(routes_d[s])
        Y.copy_(Y0d)
        graph.replay()
        outs[s].copy_(Y)
        if s % 2 == 0:
            engine.release_prefetches(COLD[s % 2])
        else:
            for a in COLD[s % 2]:
                engine.release_prefetch(a)
    torch.cuda.synchronize()
    for s in range(n_steps):
        assert_close(outs[s], reference(adapters, X, Y0, routes[s]), f"replay {s}")
    assert engine.device_errors() == 0


def test_release_landing_after_the_next_fill_of_its_slot():
    """A release held behind a bounded spin on the compute stream while the
    slot's next fill (the same adapters, the same slot indices) is copied and
    published on the prefetch stream: the release retires only its own fill,
    so the next step still uses the new one.  (Emptying the publication at
    release, as a plain clear would, loses the newer fill here.)"""
    if not hasattr(torch.cuda, "_sleep"):
        pytest.skip("torch.cuda._sleep is not available")
    import time

    engine = WarpPipeEngine()
    adapters = register_all(engine, seed=40)
    X = randn((T, D), 41, DT)
    Y0 = randn((T, O), 42, DT)
    Xd = X.cuda()
    idx = routing(0)
    ref = reference(adapters, X, Y0, idx)
    slots0 = engine.prefetch_adapters(COLD[0])
    assert engine.wait_prefetches(COLD[0])
    assert engine.build_seg_bounds(idx.cuda())
    Y = Y0.cuda()
    engine.shrink_expand(Xd, Y, O, R)
    torch.cuda.synchronize()
    assert_close(Y, ref, "first fill")
    announce("release held behind a spin while the slots are filled again")
    torch.cuda._sleep(100_000_000)
    engine.release_prefetches(COLD[0])
    released = torch.cuda.Event()
    released.record()
    slots1 = engine.prefetch_adapters(COLD[0])
    assert sorted(slots1) == sorted(slots0), (slots0, slots1)
    t0 = time.time()
    while not all(engine.is_prefetch_ready(a) for a in COLD[0]):
        assert time.time() - t0 < 10, "the second fill did not land"
        time.sleep(1e-4)
    # The order this test is about: the new fills landed first.
    assert not released.query(), "the spin ended before the second fill landed"
    assert engine.wait_prefetches(COLD[0])
    assert engine.build_seg_bounds(idx.cuda())
    Y = Y0.cuda()
    engine.shrink_expand(Xd, Y, O, R)
    torch.cuda.synchronize()
    assert_close(Y, ref, "second fill")
    assert engine.device_errors() == 0


def test_unstaged_cold_adapter_is_skipped_and_flagged():
    """Negative control of the test above: a replay that routes to cold
    adapters nobody staged skips their tokens and flags them (device error 2);
    the hot tenants' tokens are still applied."""
    engine = WarpPipeEngine()
    adapters = register_all(engine)
    X = randn((T, D), 17, DT)
    Y0 = randn((T, O), 18, DT)
    Xd, Y = X.cuda(), Y0.cuda()
    idx = routing(1)
    announce("replay routed to unstaged cold adapters")
    assert engine.build_seg_bounds(idx.cuda())
    engine.shrink_expand(Xd, Y, O, R)
    torch.cuda.synchronize()
    assert engine.device_errors() & _lib.DEVICE_ERR_UNREGISTERED
    hot_only = torch.where(torch.tensor([int(v) in HOT for v in idx]), idx, torch.full_like(idx, -1))
    assert_close(Y, reference(adapters, X, Y0, hot_only), "hot tokens only")


def test_eager_call_uses_a_prefetch_that_landed_after_the_plan():
    """build_seg_bounds before the prefetch; once the copy has landed, an eager
    call on that table uses the staged copy."""
    engine = WarpPipeEngine()
    adapters = register_all(engine)
    X = randn((T, D), 27, DT)
    Y0 = randn((T, O), 28, DT)
    idx = routing(0)
    assert engine.build_seg_bounds(idx.cuda())
    for a in COLD[0]:
        assert engine.prefetch_adapter(a) >= 0
    torch.cuda.synchronize()
    assert all(engine.is_prefetch_ready(a) for a in COLD[0])
    Y = Y0.cuda()
    announce("eager call after the prefetch landed")
    engine.shrink_expand(X.cuda(), Y, O, R)
    H = engine.shrink(X.cuda(), D, R, T)
    torch.cuda.synchronize()
    assert_close(Y, reference(adapters, X, Y0, idx), "eager shrink_expand")
    assert_close(H, bgmv.shrink(X, so.seg_bounds(idx.tolist()).tolist(), adapters, R, T), "eager shrink")
    assert engine.device_errors() == 0


def test_release_returns_device_adapters_to_their_registered_copy():
    """A device-resident adapter staged D2D and released: calls before and
    after the release give the same bits (the staged copy is bitwise the
    registered one), and evicting it afterwards leaves its tokens untouched."""
    engine = WarpPipeEngine()
    adapters = register_all(engine)
    X = randn((T, D), 37, DT)
    Y0 = randn((T, O), 38, DT)
    idx = torch.repeat_interleave(torch.tensor(HOT[:16]), 8)
    assert engine.build_seg_bounds(idx.cuda())
    Y1, Y2, Y3 = Y0.cuda(), Y0.cuda(), Y0.cuda()
    announce("staged vs registered copy of device adapters")
    for a in HOT[:8]:
        assert engine.prefetch_adapter(a) >= 0
        assert engine.wait_prefetch(a)
    assert engine.build_seg_bounds(idx.cuda())
    engine.shrink_expand(X.cuda(), Y1, O, R)
    for a in HOT[:8]:
        engine.release_prefetch(a)
    engine.shrink_expand(X.cuda(), Y2, O, R)
    engine.evict_adapter(HOT[0])
    engine.shrink_expand(X.cuda(), Y3, O, R)
    torch.cuda.synchronize()
    assert torch.equal(Y1.cpu(), Y2.cpu())
    assert_close(Y1, reference(adapters, X, Y0, idx), "staged")
    rest = torch.where(idx == HOT[0], torch.full_like(idx, -1), idx)
    assert_close(Y3, reference(adapters, X, Y0, rest), "after evicting adapter 0")
    assert engine.device_errors() & _lib.DEVICE_ERR_UNREGISTERED


def test_table_entry_dtype_is_checked():
    """A bf16 adapter reached by an fp16 call through a build_seg_bounds table
    is skipped and flagged as a shape mismatch (device error 4), not
    reinterpreted."""
    engine = WarpPipeEngine()
    A = randn((R, 256), 1, torch.bfloat16, 0.02)
    B = randn((256, R), 2, torch.bfloat16, 0.02)
    engine.register_adapter(0, A.cuda(), B.cuda(), 1.0, rank=R)
    X = randn((16, 256), 3, torch.float16)
    Y0 = randn((16, 256), 4, torch.float16)
    Y = Y0.cuda()
    announce("fp16 call on a bf16 table entry")
    assert engine.build_seg_bounds(torch.zeros(16, dtype=torch.int64, device="cuda"))
    engine.shrink_expand(X.cuda(), Y, 256, R)
    torch.cuda.synchronize()
    assert engine.device_errors() & _lib.DEVICE_ERR_SHAPE
    assert torch.equal(Y.cpu(), Y0)


def test_table_does_not_move_after_capture():
    """The adapter table is sized at engine creation: an adapter registered
    after a step was captured, under an id far above the others, is applied
    on replay."""
    engine = WarpPipeEngine(WarpPipeConfig(max_adapter_ids=70000))
    adapters = {}
    for i in range(4):
        A, B = randn((R, 512), 10 + i, DT, 0.02), randn((512, R), 20 + i, DT, 0.02)
        engine.register_adapter(i, A.cuda(), B.cuda(), 1.0, rank=R)
        adapters[i] = (A, B, 1.0)
    X = randn((64, 512), 5, DT)
    Y0 = randn((64, 512), 6, DT)
    Xd, Y, Y0d = X.cuda(), Y0.cuda(), Y0.cuda()
    idx_buf = torch.arange(64, device="cuda") % 4

    def step():
        engine.build_seg_bounds(idx_buf)
        engine.shrink_expand(Xd, Y, 512, R)

    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    announce("adapter 65000 registered after capture")
    A, B = randn((R, 512), 40, DT, 0.02), randn((512, R), 41, DT, 0.02)
    engine.register_adapter(65000, A.cuda(), B.cuda(), 2.0, rank=R)
    adapters[65000] = (A, B, 2.0)
    idx = torch.tensor([65000 if t % 4 == 3 else t % 4 for t in range(64)])
    idx_buf.copy_(idx.cuda())
    Y.copy_(Y0d)
    graph.replay()
    torch.cuda.synchronize()
    segs = so.seg_bounds(idx.tolist()).tolist()
    assert_close(Y, bgmv.expand(bgmv.shrink(X, segs, adapters, R, 64), Y0, segs, adapters), "replay")
    assert engine.device_errors() == 0


def test_give_up_poisons_until_the_next_plan_build():
    """A wait on partials that gives up (forced from the host with a spin
    limit of 0, so every kernel still exits) flags device error 8 and poisons
    the partial buffer: the next call skips its work rather than read words a
    late shrink workgroup may have left; the next build_seg_bounds repairs the
    buffer, and calls after it are exact again -- without anyone reading the
    device errors in between."""
    engine = WarpPipeEngine()
    L, d, o = 8, 4096, 4096
    wa = randn((L, 1, R, d), 50, DT, 0.02)
    wb = randn((L, 1, o, R), 51, DT, 0.02)
    X = randn((T, d), 52, DT)
    Y0 = randn((T, o), 53, DT)
    wad, wbd, Xd = wa.cuda(), wb.cuda(), X.cuda()
    idx = torch.randint(0, L, (T,), generator=torch.Generator().manual_seed(54))
    segs = so.seg_bounds(idx.tolist()).tolist()
    ref = bgmv.add_lora(Y0, X, wa, wb, 0.5, segs)
    assert engine.build_seg_bounds(idx.cuda())
    announce("call with spin limit 0 (gives up)")
    engine.set_spin_limit(0)
    Y_bad = Y0.cuda()
    assert engine.add_lora_packed(Y_bad, Xd, wad, wbd, 0.5)
    engine.set_spin_limit(None)
    announce("call after the give-up, same plan: skipped")
    Y_skip = Y0.cuda()
    assert engine.add_lora_packed(Y_skip, Xd, wad, wbd, 0.5)
    torch.cuda.synchronize()
    assert torch.equal(Y_skip.cpu(), Y0), "a call on the poisoned buffer wrote y"
    announce("plan rebuilt: repaired")
    assert engine.build_seg_bounds(idx.cuda())
    for k in range(3):
        Y = Y0.cuda()
        assert engine.add_lora_packed(Y, Xd, wad, wbd, 0.5)
        torch.cuda.synchronize()
        assert_close(Y, ref, f"call {k} after the repair")
    assert engine.device_errors() & _lib.DEVICE_ERR_SPIN
    Y = Y0.cuda()
    assert engine.add_lora_packed(Y, Xd, wad, wbd, 0.5)
    torch.cuda.synchronize()
    assert_close(Y, ref, "after reading the errors")
    assert engine.device_errors() == 0


def test_staging_calls_refused_under_capture():
    engine = WarpPipeEngine()
    register_all(engine)
    assert engine.prefetch_adapter(28) >= 0
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    announce("release / wait / register during capture")
    with pytest.raises(RuntimeError, match="capture"):
        with torch.cuda.graph(graph, stream=s):
            engine.release_prefetch(28)
    with pytest.raises(RuntimeError, match="capture"):
        with torch.cuda.graph(torch.cuda.CUDAGraph(), stream=s):
            engine.wait_prefetch(28)
    assert engine.is_prefetch_ready(28)
