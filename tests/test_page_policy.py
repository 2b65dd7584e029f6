"""The paged KV pool's page policy (host C++ in the library) against the
restatement of swamp-engine/src/cache.rs in oracle/page_policy.py, on
hand-worked cases and random operation sequences (CPU)."""
import random

import pytest

import nyion_hip as nh
import page_policy as ref

C, E, R = nh.PAGE_CREATE, nh.PAGE_EVICT, nh.PAGE_RELOAD


def test_lru_eviction_and_reload_by_hand():
    """Limit 2: page 2 evicts the least recent page 0 into slot 0; bringing 0
    back evicts page 1 (now least recent) into slot 1 (the cursor moved past
    slot 0) and reuses the block page 1 left."""
    p = nh.PagePolicy(2, 4, 8)
    assert p.ensure(0) == (0, [(C, 0, 0, -1)])
    assert p.ensure(1) == (0, [(C, 1, 1, -1)])
    assert p.ensure(2) == (0, [(E, 0, 0, 0), (C, 2, 0, -1)])
    assert p.ensure(0) == (0, [(E, 1, 1, 1), (R, 0, 1, 0)])
    assert p.lru() == [0, 2]
    assert p.state(1)[:2] == (nh.PAGE_COLD, 1) and p.state(0)[:2] == (nh.PAGE_HOT, 1)


def test_creates_pages_in_order():
    """ensure_page of page 3 on an empty cache creates 0, 1, 2, 3 (cache.rs:
    530-535)."""
    p = nh.PagePolicy(8, 4, 16)
    rc, ev = p.ensure(3)
    assert rc == 0 and [e[:2] for e in ev] == [(C, 0), (C, 1), (C, 2), (C, 3)]
    assert p.lru() == [3, 2, 1, 0]


def test_importance_picks_the_victim():
    """Tail-first candidates 0 (5.0), 1 (0.1), 2 (0.0), 3 (0.0): the first
    strictly lowest is page 2."""
    p = nh.PagePolicy(4, 8, 16)
    p.ensure(0, 3)
    p.record(0, 5.0)
    p.record(1, 0.1)
    rc, ev = p.ensure(4)
    assert rc == 0 and ev == [(E, 2, 2, 0), (C, 4, 2, -1)]


def test_candidate_window_is_eight_pages():
    """Ten hot pages, page 9 (most recent) the least important: only the tail
    and the seven before it (pages 0..7) are candidates, all equal, so the
    tail goes."""
    p = nh.PagePolicy(10, 16, 32)
    p.ensure(0, 9)
    for q in range(9):
        p.record(q, 1.0)
    rc, ev = p.ensure(10)
    assert rc == 0 and ev[0] == (E, 0, 0, 0)


def test_full_cold_tier_is_an_error_and_changes_nothing():
    p = nh.PagePolicy(1, 1, 8)
    p.ensure(0)
    assert p.ensure(1) == (0, [(E, 0, 0, 0), (C, 1, 0, -1)])
    rc, ev = p.ensure(2)
    assert rc == nh.ERR_OOM and ev == []
    assert p.state(1)[:2] == (nh.PAGE_HOT, 0) and p.state(2)[0] == nh.PAGE_UNMAPPED


def test_range_larger_than_hot_tier_is_rejected():
    p = nh.PagePolicy(2, 4, 8)
    rc, ev = p.ensure(0, 2)
    assert rc == nh.ERR_INVALID and ev == []


def test_importance_rules():
    p = nh.PagePolicy(2, 4, 8)
    p.record(0, 1.0)  # not created yet: ignored (cache.rs:566-568)
    p.ensure(0)
    assert p.state(0)[2] == 0.0
    p.record(0, 0.5)
    p.ensure(1)
    # tail 0 (0.5) vs page 1 (0.0): the less important page 1 goes, not the tail
    assert p.ensure(2) == (0, [(E, 1, 1, 0), (C, 2, 1, -1)])
    p.record(1, 0.25)  # a cold page keeps collecting
    assert p.state(1) == (nh.PAGE_COLD, 0, 0.25)
    # back in: candidates tail 0 (0.5), then 2 (0.0): page 2 goes
    assert p.ensure(1) == (0, [(E, 2, 1, 1), (R, 1, 1, 0)])
    assert p.state(1) == (nh.PAGE_HOT, 1, 0.25) and p.state(0)[2] == 0.5
    p.reset()
    assert all(p.state(q)[2] == 0.0 for q in range(3))


def test_range_pages_are_not_evicted_while_made_hot():
    """Limit 4: ensure(0, 3), page 0 made important, then ensure(4, 7).  Each
    new page of 4..7 evicts the least important unprotected page; creating
    page 7 finds only page 0 (5.0) outside the range (4, 5, 6 are
    protected), so page 0 goes and all of 4..7 end hot.  Without the
    protection page 4 (importance 0) would be evicted by its own range."""
    want_ev = [(E, 1, 1, 0), (C, 4, 1, -1), (E, 2, 2, 1), (C, 5, 2, -1),
               (E, 3, 3, 2), (C, 6, 3, -1), (E, 0, 0, 3), (C, 7, 0, -1)]
    p = nh.PagePolicy(4, 8, 16)
    p.ensure(0, 3)
    p.record(0, 5.0)
    assert p.ensure(4, 7) == (0, want_ev)
    assert all(p.state(q)[0] == nh.PAGE_HOT for q in range(4, 8))
    assert p.lru() == [7, 6, 5, 4]
    r = ref.PagePolicy(4, 8, 16)
    r.ensure(0, 3)
    r.record(0, 5.0)
    assert r.ensure(4, 7) == (True, want_ev)
    assert r.lru == [7, 6, 5, 4]


@pytest.mark.parametrize("hot,cold,pages,seed", [(1, 3, 8, 0), (2, 2, 12, 1), (4, 8, 32, 2),
                                                 (8, 64, 64, 3), (10, 5, 40, 4), (16, 200, 200, 5)])
def test_random_sequences_match_restatement(hot, cold, pages, seed):
    rng = random.Random(seed)
    got = nh.PagePolicy(hot, cold, pages)
    want = ref.PagePolicy(hot, cold, pages)
    for _ in range(400):
        op = rng.random()
        if op < 0.7:
            first = rng.randrange(pages)
            last = min(pages - 1, first + rng.randrange(hot + 1))  # sometimes one too many
            rc, ev = got.ensure(first, last)
            ok, wev = want.ensure(first, last)
            assert ev == wev and (rc == 0) == ok, (first, last, ev, wev, rc)
        elif op < 0.95:
            q, w = rng.randrange(pages), rng.choice([0.0, 0.002, 0.5, 1.0, rng.random()])
            got.record(q, w)
            want.record(q, w)
        else:
            got.reset()
            want.reset()
        assert got.lru() == want.lru
        for q in range(pages):
            st, where, imp = got.state(q)
            assert (st, where) == (want.state[q], want.where[q]) and imp == want.importance[q]


def test_restatement_on_the_hand_worked_cases():
    """The same hand-worked expectations, on the oracle restatement itself."""
    p = ref.PagePolicy(2, 4, 8)
    assert p.ensure(0) == (True, [(C, 0, 0, -1)])
    assert p.ensure(1) == (True, [(C, 1, 1, -1)])
    assert p.ensure(2) == (True, [(E, 0, 0, 0), (C, 2, 0, -1)])
    assert p.ensure(0) == (True, [(E, 1, 1, 1), (R, 0, 1, 0)])
    assert p.lru == [0, 2]
    q = ref.PagePolicy(4, 8, 16)
    q.ensure(0, 3)
    q.record(0, 5.0)
    q.record(1, 0.1)
    assert q.ensure(4) == (True, [(E, 2, 2, 0), (C, 4, 2, -1)])
    w = ref.PagePolicy(10, 16, 32)
    w.ensure(0, 9)
    for k in range(9):
        w.record(k, 1.0)
    assert w.ensure(10)[1][0] == (E, 0, 0, 0)
    f = ref.PagePolicy(1, 1, 8)
    f.ensure(0)
    f.ensure(1)
    assert f.ensure(2) == (False, [])
