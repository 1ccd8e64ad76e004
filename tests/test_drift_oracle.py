"""Host-link traffic of the LRU and static arms under drifting routing, on the CPU oracle.

The bench's `pcie_drift` leg measures this with the device kernel; the kernel's state is
bit-exact against oracle.lru (test_gpu_lru.py), so the property it reports is checked here
on the oracle: on the headline's Zipf(1.1) layer traces (26 of 512 permutation positions
re-shuffled every 8 steps, 20 correlated rows), a cache that cannot insert (static arm,
max_inserts 0) leaves more and more routed experts cold as the popularity drifts away from
its warm set, while the LRU keeps its per-step traffic (inserted + cold experts) flat.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import lru as olru

E, S, TOPK, ROWS, STEPS, WIN = 512, 257, 10, 20, 400, 50


def arm_traffic(trace, hot, rank, max_inserts):
    """Per step: experts inserted + distinct routed experts left cold after the manager."""
    st = olru.warm_start(E, S, hot, rank, max_inserts=max_inserts)
    out = []
    for t in range(trace.shape[0]):
        ids = trace[t].reshape(-1)
        n_ins = olru.manage(st, ids)
        routed = np.unique(ids[(ids >= 0) & (ids < E)])
        out.append(n_ins + int((st.map_cold[routed] >= 0).sum()))
    return np.asarray(out, np.float64)


@pytest.mark.parametrize("layer", [0, 7, 31])
def test_static_arm_goes_stale_lru_stays_flat(pkg, layer):
    tr, perm0 = pkg.traces.zipf_trace(seed=1000 + layer, E=E, rows=ROWS, k=TOPK, steps=STEPS,
                                      s=1.1, corr=0.7)
    trace = tr.reshape(STEPS, ROWS, TOPK)
    hot, rank = pkg.traces.warm_hot(perm0, S)
    lru = arm_traffic(trace, hot, rank, 64)
    static = arm_traffic(trace, hot, rank, 0)
    first, last = slice(0, WIN), slice(STEPS - WIN, STEPS)
    # the static arm never inserts: its traffic is its cold experts, which grow with the drift
    assert static[last].mean() > 1.8 * static[first].mean()
    # the LRU's traffic stays within 25% of where it started ...
    assert abs(lru[last].mean() - lru[first].mean()) < 0.25 * lru[first].mean()
    # ... and ends well under the stale static arm's
    assert lru[last].mean() < 0.7 * static[last].mean()


def test_no_drift_keeps_static_arm_flat(pkg):
    """The control: the same trace generator with the drift switched off (reshuffle 0) leaves
    the static arm's cold count where it started, so the growth above is the drift's."""
    tr, perm0 = pkg.traces.zipf_trace(seed=1000, E=E, rows=ROWS, k=TOPK, steps=STEPS, s=1.1,
                                      corr=0.7, reshuffle=0)
    trace = tr.reshape(STEPS, ROWS, TOPK)
    hot, rank = pkg.traces.warm_hot(perm0, S)
    static = arm_traffic(trace, hot, rank, 0)
    first, last = slice(0, WIN), slice(STEPS - WIN, STEPS)
    assert abs(static[last].mean() - static[first].mean()) < 0.25 * static[first].mean()
