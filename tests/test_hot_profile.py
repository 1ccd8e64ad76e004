"""Hot profiles: the on-disk warm-start format and the global budget split (CPU).

The fixture tests/golden/hot_profile.json is the reference's own profile file
(profiles/hot_profile.json: decode routing counts of 48 layers x 512 experts). It pins:
  * the reader (every layer a permutation of the experts, counts non-increasing);
  * the writer: rebuilding the [layer, expert] count matrix from the file and running
    build() gives the file's rankings, counts and decode_tokens exactly (the reference wrote
    it with a stable descending argsort, tools/routecap/build_hot_profile.py:14-20);
  * the water-fill against a brute force that sorts (fraction, position) tuples in Python --
    an independent statement of "the highest fractions, ties in layer then rank order"
    (r4d_mxfp4_moe.py.lru.diff:100-126) -- at several budgets, and its invariants.
"""
from __future__ import annotations

import json
import pathlib

import numpy as np
import pytest

GOLDEN = pathlib.Path(__file__).parent / "golden" / "hot_profile.json"
PER_EXPERT = 5_899_680      # w13 + s13 + w2 + s2 of one fp8 expert at hidden 2560, I 768


@pytest.fixture(scope="module")
def hp(pkg):
    return pkg.hot_profile


@pytest.fixture(scope="module")
def prof(hp):
    return hp.load(GOLDEN)


def count_matrix(prof):
    E = max(len(r) for r, _ in prof.layers.values())
    m = np.zeros((len(prof.layers), E), np.float64)
    for row, (r, c) in enumerate(prof.layers.values()):
        m[row, r] = c
    return m


def test_fixture_reads(prof):
    assert len(prof.layers) == 48 and prof.decode_tokens == 11279
    for r, c in prof.layers.values():
        assert sorted(r.tolist()) == list(range(512))
        assert (np.diff(c) <= 0).all()


def test_build_reproduces_the_reference_file(hp, prof):
    m = count_matrix(prof)
    rebuilt = hp.build(m, layer_ids=list(prof.layers), source="x")
    assert rebuilt.decode_tokens == prof.decode_tokens
    assert list(rebuilt.layers) == list(prof.layers)
    for li in prof.layers:
        assert np.array_equal(rebuilt.layers[li][0], prof.layers[li][0])
        assert np.array_equal(rebuilt.layers[li][1], prof.layers[li][1])


def test_save_load_roundtrip_with_ties(hp, tmp_path):
    rng = np.random.default_rng(0)
    m = rng.integers(0, 4, size=(5, 40)).astype(np.float64)     # many ties
    p = hp.build(m, source="t")
    path = tmp_path / "p.json"
    hp.save(p, path)
    q = hp.load(path)
    assert json.loads(path.read_text())["layers"].keys() == {str(i) for i in range(5)}
    for li in range(5):
        order = sorted(range(40), key=lambda e: (-m[li, e], e))  # stable: ties by expert id
        assert q.layers[li][0].tolist() == order
        assert q.layers[li][1].tolist() == [m[li, e] for e in order]


def brute_sets(prof, budget):
    items = []
    pos = 0
    for li, (r, c) in prof.layers.items():
        tot = float(c.sum())
        for e, x in zip(r.tolist(), c.tolist()):
            items.append((-(x / tot), pos, li, e))
            pos += 1
    items.sort()
    out = {li: [] for li in prof.layers}
    for _, _, li, e in items[:budget]:
        out[li].append(e)
    return {li: sorted(v) for li, v in out.items()}


@pytest.mark.parametrize("gb", [0.001, 1.0, 10.0, 50.0, 100.0, 300.0])
def test_water_fill_vs_brute_force(hp, prof, gb):
    sets = hp.hot_sets(prof, PER_EXPERT, gb)
    budget = hp.budget_experts(gb, PER_EXPERT)
    assert budget == int(gb * 1e9) // PER_EXPERT
    assert sets == brute_sets(prof, budget)
    assert sum(len(v) for v in sets.values()) == min(budget, 48 * 512)
    for li, (r, _) in prof.layers.items():        # a layer keeps a prefix of its ranking
        n = len(sets[li])
        assert sorted(r[:n].tolist()) == sets[li]


def test_water_fill_small_cases_by_hand(hp):
    # layer 0: fractions .5 .3 .2; layer 1: .6 .4 -> order (1,a) .6, (0,x) .5, (1,b) .4, ...
    p = hp.HotProfile({0: (np.array([7, 3, 5]), np.array([5.0, 3.0, 2.0])),
                       1: (np.array([1, 9]), np.array([6.0, 4.0]))})
    assert hp.hot_sets(p, 10**9, 1.0) == {0: [], 1: [1]}
    assert hp.hot_sets(p, 10**9, 2.0) == {0: [7], 1: [1]}
    assert hp.hot_sets(p, 10**9, 3.0) == {0: [7], 1: [1, 9]}
    assert hp.hot_sets(p, 10**9, 4.0) == {0: [3, 7], 1: [1, 9]}
    assert hp.hot_sets(p, 10**9, 9.0) == {0: [3, 5, 7], 1: [1, 9]}
    assert abs(hp.coverage(p, 10**9, 3.0) - (0.6 + 0.5 + 0.4) / 2) < 1e-12
    # equal fractions: layer order first
    q = hp.HotProfile({4: (np.array([2]), np.array([1.0])), 0: (np.array([8]), np.array([3.0]))})
    assert hp.hot_sets(q, 10**9, 1.0) == {4: [2], 0: []}


def test_coverage_monotone_and_bounded(hp, prof):
    cov = [hp.coverage(prof, PER_EXPERT, gb) for gb in (1, 10, 50, 100, 200, 400)]
    assert all(0.0 <= c <= 1.0 + 1e-12 for c in cov)
    assert all(b >= a for a, b in zip(cov, cov[1:]))
    assert abs(cov[-1] - 1.0) < 1e-12


def test_rank_and_errors(hp, prof):
    r = prof.rank(0)
    assert r[int(prof.layers[0][0][0])] == 0 and len(r) == 512
    assert prof.rank(999) is None
    bad = hp.HotProfile({0: (np.array([1, 2]), np.array([0.0, 0.0]))})
    with pytest.raises(ValueError, match="no routing counts"):
        hp.hot_sets(bad, 10, 1.0)
    with pytest.raises(ValueError):
        hp.budget_experts(1.0, 0)


def test_environment_entry_points(hp, monkeypatch):
    monkeypatch.delenv(hp.ENV_PROFILE, raising=False)
    monkeypatch.delenv(hp.ENV_GB, raising=False)
    assert hp.hot_profile() is None
    assert hp.hot_ids_for_layer(3, PER_EXPERT) is None
    assert hp.profile_rank_for_layer(3) is None
    monkeypatch.setenv(hp.ENV_PROFILE, str(GOLDEN))
    with pytest.raises(ValueError, match="VLLM_R4D_HOT_GB"):
        hp.hot_ids_for_layer(3, PER_EXPERT)
    monkeypatch.setenv(hp.ENV_GB, "50")
    prof = hp.load(GOLDEN)
    assert hp.hot_ids_for_layer(3, PER_EXPERT) == hp.hot_sets(prof, PER_EXPERT, 50.0)[3]
    assert hp.hot_ids_for_layer(4242, PER_EXPERT) is None
    assert hp.profile_rank_for_layer(3) == prof.rank(3)


def test_profile_trace(pkg, prof):
    r, c = prof.layers[5]
    tr = pkg.traces.profile_trace(r, c, 512, seed=3, rows=20, k=10, steps=30)
    assert tr.shape == (30, 200)
    rows = tr.reshape(-1, 10)
    assert all(len(set(x.tolist())) == 10 for x in rows)
    never = set(r[c == 0].tolist())
    assert not never & set(tr.ravel().tolist())
    again = pkg.traces.profile_trace(r, c, 512, seed=3, rows=20, k=10, steps=30)
    assert np.array_equal(tr, again)
    # the layer's 64 most routed experts are drawn far more often than its bottom half
    freq = np.bincount(tr.ravel(), minlength=512)
    assert freq[r[:64]].mean() > 3 * freq[r[256:]].mean()
