"""CPU: pin the LRU oracle before trusting it.

* numpy restatement (oracle/lru.py, sort-based victims, vectorised align) against the serial C
  restatement (oracle/lru_oracle.c, argmin per insert, cursor align) on every suite of
  tests/lru/test_lru.py, every case of tests/lru/test_victim_equiv.py and the align geometries
  of tests/lru/test_fused.py -- two different algorithms for the same contract;
* hand-worked known answers on tiny caches (ties, empty slots, read-through, padding, cap);
* brute force: on tiny caches, the victims equal the lexicographically smallest (stamp, slot)
  evictable slots found by enumerating all subsets;
* the invariants of tests/lru/test_lru.py:138-145 after every step;
* the committed golden fixture reproduces;
* planted mistakes in a copy of the oracle are caught by these comparisons.
"""
from __future__ import annotations

import itertools
import pathlib

import numpy as np
import pytest

from lru_cases import POLICY_SUITES, VICTIM_CASES, c1_trace, policy_start, victim_case
from oracle import clru, lru
from conftest import load_pkg
otrace = load_pkg().traces

BS = 16


def same_state(a: lru.LruState, b: lru.LruState):
    for n in lru.LruState.NAMES:
        assert np.array_equal(getattr(a, n), getattr(b, n)), n


@pytest.mark.parametrize("suite", POLICY_SUITES, ids=[s[0] for s in POLICY_SUITES])
def test_policy_numpy_vs_c(suite):
    name, E, S, gen, nsteps, md, mi = suite
    rng, a = policy_start(E, S, maxi=mi)
    b = a.copy()
    for n in range(nsteps):
        ids = gen(rng, n).ravel().astype(np.int32)
        na = lru.manage(a, ids, md, mi)
        nb = clru.manage(b, ids, md, mi)
        assert na == nb
        same_state(a, b)
        assert not lru.check_invariants(a), (name, n)


@pytest.mark.parametrize("case", VICTIM_CASES, ids=[c[0] for c in VICTIM_CASES])
def test_victim_cases_numpy_vs_c(case):
    name, kw = case
    ids, a = victim_case(**kw)
    b = a.copy()
    oa = lru.fused(a, ids, BS)
    ob = clru.fused(b, ids, BS)
    same_state(a, b)
    for x, y in zip(oa, ob):
        assert np.array_equal(x, y)


@pytest.mark.parametrize("rows", [1, 4, 20, 40, 205, 400])
def test_align_geometries_numpy_vs_c(rows):
    E, S = 512, 257
    rng = np.random.default_rng(rows)
    p = otrace.zipf_p(E, 1.1)
    _, a = victim_case(E=E, S=S, mk=10, k_cold=0, maxi=64, seed=3)
    a.max_distinct = 128
    b = a.copy()
    for _ in range(4):
        ids = np.concatenate([rng.choice(E, 10, replace=False, p=p) for _ in range(rows)])
        oa = lru.fused(a, ids, BS)
        ob = clru.fused(b, ids, BS)
        same_state(a, b)
        for x, y in zip(oa, ob):
            assert np.array_equal(x, y)
        mk = ids.size
        hot = oa[0][:oa[2][0]]
        cold = oa[3][:oa[5][0]]
        tok = np.sort(np.concatenate([hot[hot != mk], cold[cold != mk]]))
        assert np.array_equal(tok, np.arange(mk))      # partition (test_fused.py:186-195)


def test_golden_fixture_reproduces():
    gold = np.load(pathlib.Path(__file__).parent / "golden" / "lru_c1.npz")
    ids, s = c1_trace()
    assert np.array_equal(gold["ids"], ids)
    names = ("sorted_hot", "eids_hot", "npad_hot", "sorted_cold", "eids_cold", "npad_cold")
    for n in range(ids.shape[0]):
        out = lru.fused(s, ids[n], BS)
        for k, x in zip(names, out):
            assert np.array_equal(gold[f"{k}_{n}"], x), (n, k)
        for k in lru.LruState.NAMES:
            assert np.array_equal(gold[f"{k}_{n}"], getattr(s, k)), (n, k)


def test_c1_insert_rate():
    """The seeded LRU workload inserts about 6 experts a step (between 4 and 8 on average)."""
    ids, s = c1_trace()
    nm = [lru.manage(s, ids[n]) for n in range(ids.shape[0])]
    assert 4 <= np.mean(nm) <= 8


# ---- known answers ----------------------------------------------------------------------
def test_known_answer_tie_and_empty():
    # E=8, S=4: slots hold experts [1, 3, -1, 6]; stamps [5, 2, 2, 7]; step 7.
    # routing {1, 0, 4}: 1 is a hit (slot 0 -> stamp 8); misses 0 and 4 (ascending).
    # evictable: slot 1 (3, stamp 2), slot 2 (empty, stamp 2), slot 3 (6, stamp 7).
    # keys (2,1) < (2,2) < (7,3): miss 0 -> slot 1 (evicts 3), miss 4 -> slot 2.
    s = lru.make_state(8, 4, [1, 3], cap=4)
    s.slot_expert[:] = [1, 3, -1, 6]
    s.table[:] = -1
    s.table[[1, 3, 6]] = [0, 1, 3]
    s.map_cold[:] = np.arange(8)
    s.map_cold[[1, 3, 6]] = -1
    s.slot_stamp[:] = [5, 2, 2, 7]
    s.step[0] = 7
    s.max_distinct = 8
    c = s.copy()
    assert lru.manage(s, np.array([1, 0, 4])) == 2
    assert clru.manage(c, np.array([1, 0, 4])) == 2
    same_state(s, c)
    assert s.miss[:2].tolist() == [[0, 1], [4, 2]]
    assert s.slot_expert.tolist() == [1, 0, 4, 6]
    assert s.slot_stamp.tolist() == [8, 8, 8, 7]
    assert s.table.tolist() == [1, 0, -1, -1, 2, -1, 3, -1]
    assert s.map_cold.tolist() == [-1, -1, 2, 3, -1, 5, -1, 7]
    assert s.routed.tolist() == [1, 1, 0, 0, 1, 0, 0, 0]


def test_known_answer_read_through_and_cap():
    s = lru.make_state(16, 4, [0, 1, 2, 3], stamps=[4, 3, 2, 1], step=4, cap=2)
    s.max_distinct = 2
    before = s.copy()
    assert lru.manage(s, np.array([5, 6, 7])) == 0          # 3 distinct > 2: read through
    for n in ("table", "map_cold", "slot_expert", "slot_stamp"):
        assert np.array_equal(getattr(s, n), getattr(before, n))
    assert s.step[0] == 5
    s.max_distinct = 16
    # misses 5,6,7,8 capped at 2 -> 5 and 6 only, into the two oldest slots 3 (stamp 1), 2
    assert lru.manage(s, np.array([8, 7, 6, 5, -1, 99])) == 2
    assert s.miss.tolist() == [[5, 3], [6, 2]]
    assert s.table[7] == -1 and s.table[8] == -1 and s.map_cold[7] == 7


def test_known_answer_nothing_evictable():
    # every resident expert routed: misses cannot be installed, n_miss = 0, miss experts set
    s = lru.make_state(8, 2, [0, 1], stamps=[1, 2], step=2, cap=4)
    c = s.copy()
    assert lru.manage(s, np.array([0, 1, 5])) == 0
    assert clru.manage(c, np.array([0, 1, 5])) == 0
    same_state(s, c)
    assert s.miss[0, 0] == 5 and s.slot_stamp.tolist() == [3, 3]


def test_brute_force_victims_tiny():
    """Victims == the nins smallest evictable (stamp, slot) pairs by exhaustive search."""
    rng = np.random.default_rng(5)
    for trial in range(300):
        E, S = int(rng.integers(4, 10)), int(rng.integers(1, 6))
        nres = int(rng.integers(0, min(E, S) + 1))
        hot = np.sort(rng.choice(E, nres, replace=False))
        st = rng.integers(0, 4, S).astype(np.int64)
        s = lru.make_state(E, S, hot, st, step=5, cap=8, max_distinct=E)
        ids = rng.integers(-1, E, int(rng.integers(0, 8)))
        ev = [i for i in range(S)
              if s.slot_expert[i] < 0 or s.slot_expert[i] not in set(ids[ids >= 0].tolist())]
        routed = sorted(set(ids[(ids >= 0)].tolist()))
        nmiss = sum(1 for e in routed if s.table[e] < 0)
        k = min(nmiss, 8, len(ev))
        best = None
        for comb in itertools.combinations(ev, k):
            key = sorted((int(s.slot_stamp[i]), i) for i in comb)
            if best is None or key < best:
                best = key
        want = [i for _, i in best] if best else []
        c = s.copy()
        got = lru.manage(s, ids)
        clru.manage(c, ids)
        same_state(s, c)
        assert got == k
        assert s.miss[:got, 1].tolist() == want, trial


# ---- warm start (_build_lru, r4d_mxfp4_moe.py.lru.diff:502-541): hand-worked answers -------
# E = 8, hot set {6, 1, 4, 3, 7}; the layer's profile ranks experts 4, 7, 1, 6, 3, 0, 2, 5
# (0 = most often routed). Slots take the hot ids in ascending order: [1, 3, 4, 6, 7]. The
# hottest (4, slot 2) gets stamp S = 5, then 7 (slot 4) 4, 1 (slot 0) 3, 6 (slot 3) 2 and the
# coldest, 3 (slot 1), 1. Every value below was worked out by hand from that rule.
WS_HOT = [6, 1, 4, 3, 7]
WS_RANK = {e: i for i, e in enumerate([4, 7, 1, 6, 3, 0, 2, 5])}


def test_known_answer_warm_start_profile():
    s = lru.warm_start(8, 5, WS_HOT, WS_RANK)
    assert s.slot_expert.tolist() == [1, 3, 4, 6, 7]
    assert s.slot_stamp.tolist() == [3, 1, 5, 2, 4]
    assert s.table.tolist() == [-1, 0, -1, 1, 2, -1, 3, 4]
    assert s.map_cold.tolist() == [0, -1, 2, -1, -1, 5, -1, -1]
    assert s.step.tolist() == [5]
    assert s.max_distinct == 2                  # max(1, int(5 * 0.5))
    assert s.max_inserts == 5 and s.miss.shape == (5, 2)   # cap = min(64, S)
    assert (s.miss == -1).all() and s.n_miss.tolist() == [0]
    assert not lru.check_invariants(s)


def test_known_answer_warm_start_evicts_coldest_first():
    """The first misses after a warm start take the profile's coldest slots, in rank order:
    a stamp rule turned upside down would evict the hottest expert (4) first."""
    s = lru.warm_start(8, 5, WS_HOT, WS_RANK)
    s.max_distinct = 8
    assert lru.manage(s, np.array([0, 4])) == 1     # 4 hits (slot 2), 0 misses
    assert s.miss[0].tolist() == [0, 1]              # into slot 1: expert 3, stamp 1
    assert s.slot_expert.tolist() == [1, 0, 4, 6, 7]
    assert s.slot_stamp.tolist() == [3, 6, 6, 2, 4]
    assert lru.manage(s, np.array([2, 5])) == 2      # next oldest: slot 3 (2), slot 0 (3)
    assert s.miss[:2].tolist() == [[2, 3], [5, 0]]
    c = lru.warm_start(8, 5, WS_HOT, WS_RANK)
    c.max_distinct = 8
    clru.manage(c, np.array([0, 4]))
    clru.manage(c, np.array([2, 5]))
    same_state(s, c)


def test_known_answer_warm_start_edges():
    # no profile: zero stamps, so ties go by slot (lowest id first); S = 1 reads through above 1
    s = lru.warm_start(8, 3, [5, 2, 7], None)
    assert s.slot_expert.tolist() == [2, 5, 7] and s.slot_stamp.tolist() == [0, 0, 0]
    assert s.max_distinct == 1 and s.step.tolist() == [3]
    one = lru.warm_start(4, 1, [3], {3: 0})
    assert one.slot_stamp.tolist() == [1] and one.max_distinct == 1 and one.max_inserts == 1
    # experts missing from the profile rank after every ranked one (rank = len(rank)), so
    # they get the lowest stamps; among themselves, slot order
    part = lru.warm_start(8, 4, [0, 2, 5, 6], {6: 0, 2: 1})
    assert part.slot_stamp.tolist() == [2, 3, 1, 4]
    # the production geometry: S = 257 -> max_distinct 128, cap 64, stamps a permutation of
    # 1..257 with the hottest at S
    rank = {e: i for i, e in enumerate(np.random.default_rng(7).permutation(512).tolist())}
    hot = sorted(rank, key=rank.get)[:257]
    big = lru.warm_start(512, 257, hot, rank)
    assert big.max_distinct == 128 and big.max_inserts == 64
    assert sorted(big.slot_stamp.tolist()) == list(range(1, 258))
    hottest = min(hot, key=rank.get)
    assert big.slot_stamp[big.table[hottest]] == 257
    assert list(big.slot_expert) == sorted(hot)


def test_product_warm_start_known_answer():
    """LruCache.build (the product's _build_lru) on the CPU gives the hand-worked state."""
    c = load_pkg().LruCache.build(8, WS_HOT, WS_RANK, "cpu")
    assert c.slot_expert.tolist() == [1, 3, 4, 6, 7]
    assert c.slot_stamp.tolist() == [3, 1, 5, 2, 4]
    assert c.table.tolist() == [-1, 0, -1, 1, 2, -1, 3, 4]
    assert c.map_cold.tolist() == [0, -1, 2, -1, -1, 5, -1, -1]
    assert c.step.tolist() == [5] and c.max_distinct == 2 and c.max_inserts == 5
    assert tuple(c.miss.shape) == (5, 2)


def test_planted_warm_start_mistakes_are_caught():
    """Reversed stamps, unsorted slots and a wrong step each fail the hand-worked answers."""
    good = lru.warm_start(8, 5, WS_HOT, WS_RANK)
    rev = good.copy()
    rev.slot_stamp[:] = 6 - good.slot_stamp              # hottest -> 1, coldest -> S
    assert rev.slot_stamp.tolist() != [3, 1, 5, 2, 4]
    rev.max_distinct = 8
    lru.manage(rev, np.array([0, 4]))
    assert rev.miss[0].tolist() == [0, 4]                # evicts expert 7 (2nd hottest), not 3
    unsorted = lru.make_state(8, 5, WS_HOT, good.slot_stamp, step=5)
    assert unsorted.slot_expert.tolist() != [1, 3, 4, 6, 7]


# ---- align sizes (r4d_mxfp4_moe.py.lru.diff:290-296): the worst case, by brute force -------
def _worst_npad(mk: int, E: int, bs: int) -> int:
    """Largest num_post_pad any routing of mk ids (each in [-1, E)) can produce, over every
    multiset of ids."""
    best = 0
    for ids in itertools.combinations_with_replacement(range(-1, E), mk):
        cnt = np.bincount(np.array([i for i in ids if i >= 0], np.int64), minlength=E)
        best = max(best, int(((cnt + bs - 1) // bs * bs).sum()))
    return best


@pytest.mark.parametrize("E", [1, 2, 3, 5])
@pytest.mark.parametrize("bs", [1, 2, 4, 16])
def test_align_sizes_brute_force(E, bs):
    """L must hold the worst routing's padded run (else the kernel would write past it), and
    be tight: it exceeds that worst case by (mk - E) mod bs < bs when mk >= E, by nothing
    when mk < E. NB = ceil(L / bs) blocks."""
    for mk in range(1, 8):
        L, NB = lru.align_sizes(mk, E, bs)
        worst = _worst_npad(mk, E, bs)
        assert worst <= L, (mk, E, bs)
        assert L - worst == ((mk - E) % bs if mk >= E else 0), (mk, E, bs, L, worst)
        assert (NB - 1) * bs < L <= NB * bs
        # the worst routing through the oracle's align fills exactly `worst` entries
        if mk < E:
            ids = np.arange(mk)
        else:
            extra = (mk - E) // bs * bs
            ids = np.concatenate([np.arange(E), np.zeros(extra, np.int64),
                                  np.full(mk - E - extra, -1)])
        out = lru.align(ids, E, E, np.arange(E, dtype=np.int32), bs, L, NB)
        assert int(out[2][0]) == worst and int(out[5][0]) == 0


def test_align_sizes_known_answers():
    # C1 / C2: 5 tokens x top-10 over 512 experts; C3: 20 tokens; a 4096-token prefill chunk
    assert lru.align_sizes(50, 512, 16) == (800, 50)
    assert lru.align_sizes(200, 512, 16) == (3200, 200)
    assert lru.align_sizes(40960, 512, 16) == (40960 + 512 * 15, (40960 + 512 * 15) // 16)
    assert lru.align_sizes(512, 512, 16) == (512 + 512 * 15, 512)
    assert lru.align_sizes(7, 3, 4) == (16, 4)


# ---- planted mistakes must be caught ------------------------------------------------------
def _planted(kind):
    """A copy of the numpy manager with one plausible mistake."""
    def manage(s, ids, md=None, mi=None):
        md = s.max_distinct if md is None else md
        mi = s.max_inserts if mi is None else mi
        ids = np.asarray(ids, np.int64).ravel()
        s.step[0] += 1
        st = s.step[0]
        s.n_miss[0] = 0
        routed = np.zeros(s.E, np.uint8)
        routed[ids[(ids >= 0) & (ids < s.E)]] = 1
        s.routed[:] = routed
        if routed.sum() > md:
            return 0
        rexp = np.nonzero(routed)[0]
        sl = s.table[rexp]
        if kind != "no-refresh":
            s.slot_stamp[sl[sl >= 0]] = st
        misses = rexp[sl < 0]
        if kind == "desc-miss":
            misses = misses[::-1]
        nins = min(len(misses), mi)
        key = lru.victim_keys(s.slot_expert, s.slot_stamp, routed)
        if kind == "slot-desc-tiebreak":
            key = np.where(key == lru.LLONG_MAX, key,
                           (s.slot_stamp << 20) | (s.S - 1 - np.arange(s.S)))
        cand = np.nonzero(key != lru.LLONG_MAX)[0]
        vic = cand[np.argsort(key[cand], kind="stable")][:nins]
        for r, v in enumerate(vic.tolist()):
            e = int(misses[r])
            old = int(s.slot_expert[v])
            if old >= 0:
                s.table[old] = -1
                s.map_cold[old] = old
            s.slot_expert[v] = e
            s.slot_stamp[v] = st
            s.table[e] = v
            s.map_cold[e] = -1
            s.miss[r] = (e, v)
        s.n_miss[0] = len(vic)
        return len(vic)
    return manage


@pytest.mark.parametrize("kind", ["no-refresh", "desc-miss", "slot-desc-tiebreak"])
def test_planted_mistakes_are_caught(kind):
    bad = _planted(kind)
    caught = False
    for name, kw in VICTIM_CASES:
        ids, a = victim_case(**kw)
        b = a.copy()
        bad(a, ids)
        clru.manage(b, ids)
        if any(not np.array_equal(getattr(a, n), getattr(b, n)) for n in lru.LruState.NAMES):
            caught = True
            break
    assert caught, kind


def test_align_comparator_bites():
    """tests/lru/test_fused.py:366-388: a per-bucket multiset comparison fails on 3
    perturbations (npad, an expert id, a duplicated token)."""
    ids, s = c1_trace()
    o = lru.fused(s, ids[0], BS)

    def same(a, b):
        gs, ge, gn = a
        rs, re_, rn = b
        if gn[0] != rn[0] or not np.array_equal(ge, re_):
            return False
        n = int(gn[0])
        by = lambda s_, e_: {int(k): sorted(s_[:n][np.repeat(e_[:n // BS], BS) == k].tolist())
                             for k in np.unique(e_[:n // BS])}
        return by(gs, ge) == by(rs, re_)

    assert same(o[0:3], o[0:3])
    caught = 0
    for k in range(3):
        p = [x.copy() for x in o[0:3]]
        if k == 0:
            p[2] += BS
        elif k == 1:
            p[1][0] = -7
        else:
            p[0][0] = p[0][1]
        caught += not same(p, o[0:3])
    assert caught == 3
