"""Pins the segment-table oracle (oracle/seg_oracle.c) before it is trusted.

  * the known-answer tables derived from the reference's own test index lists
    (tests/golden/seg_bounds_kat.json, segment_table_kat.json);
  * an independent restatement (itertools.groupby over the ids) on random
    inputs, including negative ids and runs far longer than 32;
  * invariants the rule fixes: token order, disjoint coverage of exactly the
    tokens with id >= 0, pieces of <= 32 tokens, breaks only at run boundaries
    or every 32 tokens from a run start;
  * the by-adapter grouping against a stable sort.
A planted mistake (splitting at 31) is shown to fail the KATs.
"""
import itertools
import json
import os

import numpy as np
import pytest

from oracle import segments as so

MAXSEG = 32


def groupby_table(idx, piece=MAXSEG):
    """Independent restatement: itertools.groupby over consecutive equal ids."""
    out = []
    pos = 0
    for key, grp in itertools.groupby(list(idx)):
        n = len(list(grp))
        if key >= 0:
            for s in range(0, n, piece):
                out.append((int(key), pos + s, min(piece, n - s)))
        pos += n
    return out


def load(golden_dir, name):
    with open(os.path.join(golden_dir, name)) as f:
        return json.load(f)


def test_seg_bounds_known_answers(golden_dir):
    kat = load(golden_dir, "seg_bounds_kat.json")
    assert len(kat["cases"]) == 10
    for case in kat["cases"]:
        got = so.seg_bounds(case["indices"]).tolist()
        assert got == case["segments"], case["source"]


def test_planted_split_mistake_fails_known_answers(golden_dir):
    # Splitting runs at 31 instead of 32 must be caught by the KATs.
    kat = load(golden_dir, "seg_bounds_kat.json")
    mismatches = sum(groupby_table(c["indices"], piece=31) != [tuple(s) for s in c["segments"]] for c in kat["cases"])
    assert mismatches >= 2


def test_groupby_restatement_matches_known_answers(golden_dir):
    kat = load(golden_dir, "seg_bounds_kat.json")
    for case in kat["cases"]:
        assert groupby_table(case["indices"]) == [tuple(s) for s in case["segments"]], case["source"]


@pytest.mark.parametrize("T", [0, 1, 2, 31, 32, 33, 64, 255, 256, 257, 1000, 4096, 8192])
def test_seg_bounds_matches_independent_restatement(T):
    rng = np.random.default_rng(1000 + T)
    for trial in range(6):
        kind = trial % 3
        if kind == 0:    # short runs over a few ids, with -1 gaps
            idx = rng.integers(-1, 4, size=T)
        elif kind == 1:  # long runs (many > 32)
            vals = rng.integers(-2, 6, size=max(1, T // 40 + 1))
            lens = rng.integers(1, 120, size=vals.size)
            idx = np.repeat(vals, lens)[:T]
            if idx.size < T:
                idx = np.concatenate([idx, np.full(T - idx.size, 7)])
        else:            # large ids, mostly distinct
            idx = rng.integers(-1, 1 << 20, size=T)
        got = [tuple(r) for r in so.seg_bounds(idx).tolist()]
        assert got == groupby_table(idx.tolist())


@pytest.mark.parametrize("seed", range(8))
def test_seg_bounds_invariants(seed):
    rng = np.random.default_rng(seed)
    T = int(rng.integers(1, 3000))
    idx = np.repeat(rng.integers(-1, 5, size=T), rng.integers(1, 70, size=T))[:T]
    segs = so.seg_bounds(idx)
    covered = np.zeros(T, dtype=np.int64)
    prev_end = 0
    for aid, st, cnt in segs.tolist():
        assert 1 <= cnt <= MAXSEG
        assert st >= prev_end  # token order, disjoint
        prev_end = st + cnt
        assert np.all(idx[st:st + cnt] == aid)
        covered[st:st + cnt] += 1
        # a piece starts at a run start or 32k tokens after one
        run_start = st
        while run_start > 0 and idx[run_start - 1] == aid:
            run_start -= 1
        assert (st - run_start) % MAXSEG == 0
        # a short piece ends its run
        if cnt < MAXSEG:
            assert st + cnt == T or idx[st + cnt] != aid
    assert np.array_equal(covered, (idx >= 0).astype(np.int64))


def test_segment_table_known_answers(golden_dir):
    kat = load(golden_dir, "segment_table_kat.json")
    for case in kat["cases"]:
        got = so.segment_table(case["ids"], case["offsets"]).tolist()
        assert got == case["segments"], case["source"]
    k = kat["generated_cases"][0]["k"]
    got = so.segment_table(list(range(k)), list(range(k + 1))).tolist()
    assert got == [[i, i, 1] for i in range(k)]


def test_segment_table_errors(golden_dir):
    kat = load(golden_dir, "segment_table_kat.json")
    e0, e1 = kat["error_cases"]
    with pytest.raises(RuntimeError, match="K\\+1"):
        so.segment_table(e0["ids"], e0["offsets"])
    k = e1["k"]
    with pytest.raises(RuntimeError, match="capacity"):
        so.segment_table(list(range(k)), list(range(k + 1)))


@pytest.mark.parametrize("seed", range(5))
def test_group_tokens_is_stable_sort(seed):
    rng = np.random.default_rng(seed)
    T = int(rng.integers(1, 5000))
    idx = rng.integers(-1, 40, size=T)
    perm, gid, goff = so.group_tokens(idx)
    valid = np.nonzero(idx >= 0)[0]
    order = valid[np.argsort(idx[valid], kind="stable")]
    assert np.array_equal(perm, order)
    assert np.array_equal(gid, np.unique(idx[idx >= 0]))
    for g in range(gid.size):
        assert np.all(idx[perm[goff[g]:goff[g + 1]]] == gid[g])
