"""Seeded synthetic routing traces: the workload generator of the benchmark, the smoke test and
the tests (pure numpy; no kernel involved).

zipf_trace(): the LRU-only workload -- E experts, `rows` routing rows per step, top-k drawn
without replacement from p(rank r) ~ r^-s over a seeded random permutation of the experts,
with `reshuffle` positions of the permutation re-shuffled among themselves every `every`
steps. It mirrors the skewed generator of tests/lru/test_lru.py:181-185, plus the
permutation and its drift. All draws come from one numpy PCG64 stream, in this order:
    perm = rng.permutation(E)
    for each step n:
        if n > 0 and n % every == 0:
            pos = rng.choice(E, reshuffle, replace=False); perm[pos] = perm[rng.permutation(pos)]
        for each row: perm[rng.choice(E, k, replace=False, p=p)]
warm_hot(): the initial hot set = the S hottest of the initial permutation, with its ranks.
profile_trace(): rows drawn from one layer's routing counts of a hot profile (hot_profile.py).

layer_trace(): the many-layer step harness's routing: one zipf_trace per layer, seed
base + layer, exponent `s` and `corr` tuned so that the cache sees the insert rate a real
decode trace shows (5-13 inserts per layer per step at 20 rows). With corr > 0 each row
after the first re-uses each of the first row's experts with probability corr (rows of
one decode step are correlated through the shared context), the remaining ones drawn from
the Zipf law without replacement.
"""
from __future__ import annotations

import numpy as np


def zipf_p(E: int, s: float) -> np.ndarray:
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    return p / p.sum()


def zipf_trace(seed: int = 0, E: int = 512, rows: int = 5, k: int = 10, steps: int = 64,
               s: float = 1.1, every: int = 8, reshuffle: int = 26, corr: float = 0.0):
    """-> (ids int32 [steps, rows*k], initial permutation int64 [E])."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(E)
    perm0 = perm.copy()
    p = zipf_p(E, s)
    out = np.empty((steps, rows * k), np.int32)
    for n in range(steps):
        if n > 0 and every > 0 and n % every == 0 and reshuffle > 0:
            pos = rng.choice(E, reshuffle, replace=False)
            perm[pos] = perm[rng.permutation(pos)]
        step_rows = []
        first = None
        for r in range(rows):
            if corr > 0 and first is not None:
                chosen = first[rng.random(k) < corr].tolist()
                while len(chosen) < k:
                    for c in perm[rng.choice(E, k - len(chosen), replace=False, p=p)].tolist():
                        if c not in chosen and len(chosen) < k:
                            chosen.append(c)
                row = np.array(chosen, np.int64)
            else:
                row = perm[rng.choice(E, k, replace=False, p=p)]
            if first is None:
                first = row
            step_rows.append(row)
        out[n] = np.concatenate(step_rows)
    return out, perm0


def warm_hot(perm0: np.ndarray, S: int):
    """The S hottest experts of the initial permutation and their profile ranks."""
    hot = np.sort(perm0[:S])
    rank = {int(e): i for i, e in enumerate(perm0.tolist())}
    return hot, rank


def layer_trace(layer: int, steps: int, rows: int = 20, E: int = 512, k: int = 10,
                s: float = 1.1, corr: float = 0.0, base: int = 1000):
    return zipf_trace(seed=base + layer, E=E, rows=rows, k=k, steps=steps, s=s, corr=corr)


def insert_storm_ids(rng: np.random.Generator, hot: np.ndarray, E: int, mk: int,
                     k: int) -> np.ndarray:
    """Routing with exactly k distinct non-resident experts among mk ids (the rest drawn from
    the resident set), shuffled: the insert-count sweep of tests/lru/bench_victim.py:43-79."""
    hot = np.asarray(hot)
    cold = np.setdiff1d(np.arange(E), hot)
    k = min(k, len(cold))
    nh = min(mk - k, len(hot))
    routed = np.concatenate([rng.choice(cold, k, replace=False),
                             rng.choice(hot, nh, replace=False)])
    if len(routed) < mk:
        routed = np.concatenate([routed, rng.choice(routed, mk - len(routed))])
    rng.shuffle(routed)
    return routed[:mk].astype(np.int32)


def profile_trace(ranked: np.ndarray, counts: np.ndarray, E: int, seed: int = 0, rows: int = 20,
                  k: int = 10, steps: int = 64) -> np.ndarray:
    """A routing trace whose per-expert frequencies follow one layer of a hot profile: each
    row draws k distinct experts without replacement with p(e) proportional to the layer's
    routing count of e (experts the profile never saw are never drawn). One numpy PCG64
    stream. -> ids int32 [steps, rows * k]."""
    p = np.zeros(E, np.float64)
    p[np.asarray(ranked, np.int64)] = np.asarray(counts, np.float64)
    if (p > 0).sum() < k:
        raise ValueError("the profile layer routes fewer than k experts")
    p /= p.sum()
    rng = np.random.default_rng(seed)
    out = np.empty((steps, rows * k), np.int32)
    for n in range(steps):
        out[n] = np.concatenate([rng.choice(E, k, replace=False, p=p) for _ in range(rows)])
    return out
