"""ScorePrefetchPolicy bookkeeping against a stand-in engine (CPU): ranking,
releases before prefetches, the slot limit, ids the engine cannot stage."""
from types import SimpleNamespace

from adapterslotsplusplus_amd.prefetch_policy import ScorePrefetchPolicy


class FakeEngine:
    def __init__(self, slots, known):
        self.config = SimpleNamespace(num_staging_slots=slots)
        self.known = set(known)
        self.slots = [None] * slots
        self.log = []

    def prefetch_adapter(self, aid, layer=None):
        self.log.append(("prefetch", aid))
        if aid not in self.known:
            return -1
        if aid in self.slots:
            return self.slots.index(aid)
        if None not in self.slots:
            return -1
        i = self.slots.index(None)
        self.slots[i] = aid
        return i

    def release_prefetch(self, aid, layer=None):
        self.log.append(("release", aid))
        if aid in self.slots:
            self.slots[self.slots.index(aid)] = None

    def is_prefetch_ready(self, aid, layer=None):
        return aid in self.slots


def test_top_scores_are_staged_and_the_rest_released():
    eng = FakeEngine(3, range(10))
    pol = ScorePrefetchPolicy(eng)
    assert pol.update({1: 0.1, 2: 0.9, 3: 0.5, 4: 0.7}) == [2, 4, 3]
    assert set(pol.staged) == {2, 3, 4}
    assert pol.ready(2) and not pol.ready(1)
    eng.log.clear()
    # 1 rises above 3: 3 is released before 1 is prefetched (its slot is needed).
    assert pol.update({1: 0.8, 2: 0.9, 3: 0.5, 4: 0.7}) == [1]
    assert eng.log == [("release", 3), ("prefetch", 1)]
    assert set(pol.staged) == {1, 2, 4}


def test_must_ids_come_first_and_ties_break_by_id():
    eng = FakeEngine(2, range(10))
    pol = ScorePrefetchPolicy(eng)
    assert pol.ranking({5: 1.0, 3: 1.0, 7: 2.0}, must=[9]) == [9, 7, 3, 5]
    assert pol.update({5: 1.0, 3: 1.0, 7: 2.0}, must=[9]) == [9, 7]


def test_unknown_ids_and_slot_limit():
    eng = FakeEngine(4, [1, 2])
    pol = ScorePrefetchPolicy(eng, slots=2)
    assert pol.update({1: 3.0, 8: 2.0, 2: 1.0}) == [1]      # 8 is not registered
    assert set(pol.staged) == {1}
    pol.release_all()
    assert pol.staged == {} and eng.slots == [None] * 4
    assert ScorePrefetchPolicy(eng, slots=0).update({1: 1.0}) == []
