"""CPU: the host side of the routing capture (tools/routecap/routecap.py): which ring slots a
poll keeps, the file round trip, and capture -> routing counts -> warm-start profile."""
from __future__ import annotations

import numpy as np
import pytest


@pytest.fixture(scope="module")
def rc(pkg):
    from importlib import import_module
    return import_module(pkg.__name__ + ".routecap")


def test_complete_slots_keeps_finished_steps_in_order(rc):
    ring = 8
    steps = np.full(ring, -1, np.int64)
    for v in range(1, 6):                      # steps 1..5 written, 5 still in progress
        steps[v % ring] = v
    assert [int(steps[s]) for s in rc.complete_slots(steps, 5, -1)] == [1, 2, 3, 4]
    assert [int(steps[s]) for s in rc.complete_slots(steps, 5, 3)] == [4]
    assert rc.complete_slots(steps, 1, -1) == []          # only step 1, unfinished


def test_complete_slots_after_a_wrap(rc):
    ring = 8
    steps = np.full(ring, -1, np.int64)
    for v in range(1, 20):                     # slots now hold steps 12..19
        steps[v % ring] = v
    kept = [int(steps[s]) for s in rc.complete_slots(steps, 19, 4)]
    assert kept == list(range(12, 19))         # 5..11 were overwritten before this poll


def _routes(rng, n, L, maxrows, k, E, rows):
    ids = np.full((n, L, maxrows * k), -1, np.int16)
    for t in range(n):
        for li in range(L):
            ids[t, li, :rows * k] = rng.integers(0, E, rows * k)
    return dict(steps=np.arange(1, n + 1, dtype=np.int64), ids=ids, nlayer=np.int64(L),
                topk=np.int64(k), maxrows=np.int64(maxrows), ring=np.int64(64),
                ctr=np.int64(n + 1), lost_to_wrap=np.int64(0))


def test_routes_file_round_trip(rc, tmp_path):
    r = _routes(np.random.default_rng(0), 6, 3, 4, 10, 512, 2)
    p = tmp_path / "routes_rank0.npz"
    with open(p, "wb") as fh:
        np.savez(fh, **r)
    back = rc.load_routes(p)
    assert set(back) == set(r)
    for k in r:
        assert np.array_equal(back[k], r[k]) and back[k].dtype == r[k].dtype


def test_counts_and_profile_from_routes(rc, pkg):
    E, L, k = 64, 3, 4
    r = _routes(np.random.default_rng(1), 50, L, 8, k, E, 5)
    r["ids"][0, 1, 0] = E + 3                  # out of range: not counted
    c = rc.decode_counts(r, E)
    ids = r["ids"].astype(np.int64)
    for li in range(L):                        # brute force
        v = ids[:, li].ravel()
        for e in range(E):
            assert c[li, e] == int((v == e).sum())
    assert c.sum() == 50 * L * 5 * k - 1
    prof = rc.hot_profile_from_routes(r, E, source="capture")
    for li in range(L):
        ranked, counts = prof.layers[li]
        assert np.array_equal(counts, np.sort(c[li])[::-1])
        assert all(c[li, a] > c[li, b] or (c[li, a] == c[li, b] and a < b)
                   for a, b in zip(ranked[:-1], ranked[1:]))
    assert prof.decode_tokens == int(c.sum()) // (L * k)
