"""GPU: the device cache against the oracle over a long drifting trace (the replay of
tests/lru/test_trace_replay.py, which runs the reference's whole captured trace through its
kernel; docs/LOCALITY.md:203-215).

Four layers of the 52-layer decode workload (Zipf(1.1) over a seeded permutation of 512
experts, seed 1000 + layer, 20 correlated rows of top-10 per step, 26 permutation positions
re-shuffled every 8 steps) run 400 steps through the fused LRU kernel (manager + both aligns)
in both arms: the LRU (up to 64 inserts per step) and the static arm (max_inserts 0). At every
step the kernel's insert count n_miss and its count of distinct routed experts left cold equal
the oracle's; every 50 steps, and at the last, the whole cache state, the miss list and both
align outputs are bit-exact. Those two counts are what the bench's pcie_drift leg turns into
host-link bytes, so this pins its figures. The drift itself shows on the device counts too:
the static arm's cold experts grow, the LRU's traffic stays flat.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import gpu_case, load_pkg
from oracle import lru as olru

trace = load_pkg().traces
torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda"
E, S, TOPK, ROWS, STEPS, EVERY, WIN = 512, 257, 10, 20, 400, 50, 50
LAYERS = (0, 7, 31, 51)


def _cold_count(map_cold: np.ndarray, ids: np.ndarray) -> int:
    routed = np.unique(ids[(ids >= 0) & (ids < E)])
    return int((map_cold[routed] >= 0).sum())


@pytest.mark.parametrize("max_inserts", [64, 0])
@pytest.mark.parametrize("layer", LAYERS)
def test_kernel_tracks_oracle_over_400_drifting_steps(pkg, layer, max_inserts):
    tr, perm0 = trace.zipf_trace(seed=1000 + layer, E=E, rows=ROWS, k=TOPK, steps=STEPS, s=1.1,
                                 corr=0.7)
    hot, rank = trace.warm_hot(perm0, S)
    cache = pkg.LruCache.build(E, hot, rank, DEV, max_inserts=max_inserts)
    st = olru.warm_start(E, S, hot, rank, max_inserts=max_inserts)
    assert cache.max_inserts == st.max_inserts and cache.max_distinct == st.max_distinct
    mk = ROWS * TOPK
    L, NB = olru.align_sizes(mk, E, 16)
    out = cache.alloc_align(mk)
    ids_dev = torch.from_numpy(tr).to(DEV)
    ins, cold = [], []
    for t in range(STEPS):
        ids = tr[t]
        if t % EVERY == 0:
            gpu_case(f"drift layer {layer} max_inserts {max_inserts} steps {t}..")
        cache.fused(ids_dev[t], out=out)
        want = olru.fused(st, ids, 16, L, NB)
        n_miss = int(cache.n_miss.item())
        got_cold = _cold_count(cache.map_cold.cpu().numpy(), ids)
        assert n_miss == int(st.n_miss[0]), (t, n_miss, int(st.n_miss[0]))
        assert got_cold == _cold_count(st.map_cold, ids), t
        ins.append(n_miss)
        cold.append(got_cold)
        if t % EVERY == EVERY - 1 or t == STEPS - 1:
            for name, g in zip(olru.LruState.NAMES, cache.state()):
                if name == "routed":
                    continue
                g = g.cpu().numpy()
                w = getattr(st, name)
                if name == "miss":
                    g, w = g[:n_miss], w[:n_miss]
                assert np.array_equal(g, w), (t, name)
            for i, (g, w) in enumerate(zip(out, want)):
                assert np.array_equal(g.cpu().numpy(), np.asarray(w)), (t, "align", i)
    ins, cold = np.asarray(ins, float), np.asarray(cold, float)
    first, last = slice(0, WIN), slice(STEPS - WIN, STEPS)
    if max_inserts == 0:
        assert ins.sum() == 0
        assert cold[last].mean() > 1.5 * cold[first].mean(), (cold[first].mean(),
                                                               cold[last].mean())
    else:
        traffic = ins + cold
        assert abs(traffic[last].mean() - traffic[first].mean()) < 0.3 * traffic[first].mean()
