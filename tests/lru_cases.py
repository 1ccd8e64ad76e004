"""Shared LRU test cases: the reference's suites, re-expressed as data.

Suites follow tests/lru/test_lru.py:176-197 (policy), tests/lru/test_victim_equiv.py:48-81,
137-159 (victim cases) and tests/lru/test_fused.py:265-280 (geometries). Only the generators
are mirrored here -- inputs, not algorithms.
"""
from __future__ import annotations

import numpy as np

from oracle import lru as olru
from conftest import load_pkg
otrace = load_pkg().traces

# (name, E, S, generator(rng, n) -> ids [rows, k], nsteps, max_distinct, max_inserts)
def _skew(rng, n):
    p = otrace.zipf_p(512, 1.1)
    return np.stack([rng.choice(512, size=10, replace=False, p=p) for _ in range(5)])


def _padded(rng, n):
    a = rng.choice(64, size=(4, 10), replace=True)
    a[2:] = -1
    return a


POLICY_SUITES = [
    ("tiny-churn", 32, 8, lambda rng, n: rng.choice(32, size=(2, 5), replace=True), 200, 8, 8),
    ("skewed-512", 512, 257, _skew, 300, 128, 64),
    ("insert-capped", 128, 32, lambda rng, n: rng.choice(128, size=(8, 10), replace=True),
     150, 128, 4),
    ("read-through", 128, 32, lambda rng, n: rng.choice(128, size=(16, 10), replace=True),
     60, 8, 16),
    ("padded-rows", 64, 16, _padded, 120, 64, 16),
    # beyond the reference: ids >= E must be ignored like -1
    ("out-of-range", 64, 16,
     lambda rng, n: np.where(rng.random((4, 10)) < 0.2, 64 + rng.integers(0, 5, (4, 10)),
                             rng.choice(64, size=(4, 10))), 60, 64, 16),
]


def policy_start(E, S, seed=0, maxi=64):
    """tests/lru/test_lru.py:148-154: random hot set in slots 0.., zero stamps, step 0."""
    rng = np.random.default_rng(seed)
    hot = sorted(rng.choice(E, S, replace=False).tolist())
    return rng, olru.make_state(E, S, hot, cap=maxi, miss_fill=-7)


# tests/lru/test_victim_equiv.py:137-159
VICTIM_CASES = [
    ("prod B=1", dict(E=512, S=257, mk=50, k_cold=2, maxi=64, seed=1)),
    ("prod B=4", dict(E=512, S=257, mk=200, k_cold=13, maxi=64, seed=2)),
    ("at the cliff", dict(E=512, S=257, mk=50, k_cold=14, maxi=64, seed=3)),
    ("past the cliff", dict(E=512, S=257, mk=120, k_cold=40, maxi=64, seed=4)),
    ("zero misses", dict(E=512, S=257, mk=50, k_cold=0, maxi=64, seed=5)),
    ("serial n=4", dict(E=512, S=257, mk=50, k_cold=4, maxi=64, seed=18)),
    ("rank n=5", dict(E=512, S=257, mk=50, k_cold=5, maxi=64, seed=19)),
    ("serial, ev=0", dict(E=512, S=24, mk=60, k_cold=3, maxi=64, seed=20)),
    ("serial, ev=2", dict(E=512, S=26, mk=60, k_cold=4, maxi=64, seed=21)),
    ("capped by maxi", dict(E=512, S=257, mk=300, k_cold=200, maxi=8, seed=6)),
    ("tiny maxi", dict(E=512, S=257, mk=100, k_cold=60, maxi=3, seed=15)),
    ("empty slots", dict(E=512, S=257, mk=50, k_cold=10, maxi=64, seed=7, empty=100)),
    ("stamp ties", dict(E=512, S=257, mk=50, k_cold=12, maxi=64, seed=8, tie=True)),
    ("tiny cache", dict(E=512, S=16, mk=50, k_cold=30, maxi=64, seed=9)),
    ("evict-all", dict(E=512, S=24, mk=60, k_cold=50, maxi=64, seed=16)),
    ("evict exhausted", dict(E=512, S=40, mk=200, k_cold=60, maxi=64, seed=10)),
    ("S=1024", dict(E=1024, S=1024, mk=400, k_cold=100, maxi=64, seed=11, resident=600)),
    ("maxi=1024", dict(E=1024, S=1024, mk=900, k_cold=500, maxi=1024, seed=17, resident=400)),
    ("maxi=1", dict(E=512, S=257, mk=50, k_cold=20, maxi=1, seed=12)),
    # beyond the reference: huge stamps (the 64-bit key search path), and k = 64 storms
    ("stamps >= 2^43", dict(E=512, S=257, mk=200, k_cold=40, maxi=64, seed=22, big=True)),
    ("storm 64", dict(E=512, S=257, mk=200, k_cold=64, maxi=64, seed=23)),
]


def victim_case(E, S, mk, k_cold, maxi, seed, resident=None, empty=0, tie=False, big=False):
    """-> (ids int32 [mk], LruState) as tests/lru/test_victim_equiv.py:49-81 builds them."""
    rng = np.random.default_rng(seed)
    nres = S - empty if resident is None else resident
    hot = np.sort(rng.choice(E, nres, replace=False))
    cold = np.setdiff1d(np.arange(E), hot)
    k = min(k_cold, len(cold))
    nh = min(mk - k, len(hot))
    routed = np.concatenate([rng.choice(cold, k, replace=False),
                             rng.choice(hot, nh, replace=False)])
    if len(routed) < mk:
        routed = np.concatenate([routed, rng.choice(routed, mk - len(routed))])
    rng.shuffle(routed)
    ids = routed[:mk].astype(np.int32)
    stamps = np.zeros(S, np.int64) if tie else rng.permutation(S).astype(np.int64) + 1
    if big:
        stamps = stamps + (np.int64(1) << np.int64(50))
    st = olru.make_state(E, S, hot, stamps, step=int(stamps.max()) + 1, cap=maxi,
                         max_distinct=E, max_inserts=maxi)
    return ids, st


def c1_trace():
    """The LRU-only workload: E=512, S=257, top-10, 5 rows/step, 64 steps, warm start."""
    ids, perm0 = otrace.zipf_trace(seed=0, E=512, rows=5, k=10, steps=64)
    hot, rank = otrace.warm_hot(perm0, 257)
    return ids, olru.warm_start(512, 257, hot, rank)
