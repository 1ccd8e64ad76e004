"""numpy restatement of the device LRU expert cache (test infrastructure only).

Follows, function by function:
  manage()      kernels/lru/r4d_lru.hip:187-269 (lru_manage_k) with the victim rule of
                :79-185 (pickVictims/installVictim)
  align()       kernels/lru/r4d_lru.hip:502-575 (phases 1-5 of lru_fused_k) with the
                moe_align_block_size contract restated in tests/k1/moe_ref_harness.py:104-137
                and the sizes of patches/.../r4d_mxfp4_moe.py.lru.diff:290-296
  fused()       kernels/lru/r4d_lru.hip:418-575 (manager, then both align outputs)
  gather()      kernels/lru/r4d_lru.hip:271-301 (index copy of six per-expert buffers)
  warm_start()  patches/.../r4d_mxfp4_moe.py.lru.diff:502-541 (_build_lru)

Parity pins (tests/test_oracle_lru.py):
  * against the independent serial C restatement (oracle/lru_oracle.c, argmin per insert as in
    kernels/lru/r4d_lru_pre_victim.hip) on every suite of tests/lru/test_lru.py:176-197 and all
    19 cases of tests/lru/test_victim_equiv.py:137-159;
  * against brute force (every permutation / every subset) on tiny E and S;
  * against the invariants of tests/lru/test_lru.py:138-145 and test_slots_prod.py:183-197;
  * against the committed golden fixtures (tests/golden/);
  * warm_start(): hand-worked states for a 5-slot profile (stamps, slots, table, step, cap,
    read-through threshold), the first evictions after it taking the profile's coldest slots,
    and the edges (no profile, S = 1, experts missing from the profile, S = 257);
  * align_sizes(): against the worst num_post_pad over every routing of tiny E / mk / bs
    (brute force): L holds it and exceeds it by (mk - E) mod bs at most.
Align order: stable (ascending token index inside a bucket) at every mk. That equals the
reference's deterministic path (mk <= 256, r4d_lru.hip:542-562) and is one member of the
per-bucket multiset class its atomic-cursor path (mk > 256) produces.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

SLOT_BITS = 20          # r4d_lru.hip:29
LLONG_MAX = np.int64(2**63 - 1)
MAXS = 1024             # r4d_lru.hip:76
MAXE = 1024             # r4d_lru.hip:328
MAXINS = 1024           # r4d_lru.hip:77


@dataclass
class LruState:
    """The eight tensors the manager owns (r4d_lru.hip:187-199)."""
    table: np.ndarray          # int32 [E]   expert -> slot or -1
    map_cold: np.ndarray       # int32 [E]   expert -> expert when not resident, else -1
    slot_expert: np.ndarray    # int32 [S]   slot -> expert or -1
    slot_stamp: np.ndarray     # int64 [S]   slot -> step it was last routed
    routed: np.ndarray         # uint8 [E]   scratch: routed this step
    step: np.ndarray           # int64 [1]
    miss: np.ndarray           # int32 [cap, 2] (expert, slot)
    n_miss: np.ndarray         # int32 [1]
    max_distinct: int = 0
    max_inserts: int = 0

    @property
    def E(self) -> int:
        return int(self.table.shape[0])

    @property
    def S(self) -> int:
        return int(self.slot_expert.shape[0])

    NAMES = ("table", "map_cold", "slot_expert", "slot_stamp", "routed", "step", "miss",
             "n_miss")

    def copy(self) -> "LruState":
        return LruState(*(getattr(self, n).copy() for n in self.NAMES),
                        max_distinct=self.max_distinct, max_inserts=self.max_inserts)

    def arrays(self) -> dict:
        return {n: getattr(self, n) for n in self.NAMES}


def align_sizes(mk: int, num_experts: int, block_size: int) -> tuple[int, int]:
    """sorted_ids / expert_ids lengths vLLM's moe_align_block_size wrapper allocates
    (patches/.../r4d_mxfp4_moe.py.lru.diff:290-296)."""
    n = mk + num_experts * (block_size - 1)
    if mk < num_experts:
        n = min(mk * block_size, n)
    return n, (n + block_size - 1) // block_size


def make_state(E: int, S: int, hot: np.ndarray, stamps: np.ndarray | None = None,
               step: int = 0, cap: int = 64, max_distinct: int | None = None,
               max_inserts: int | None = None, miss_fill: int = -1) -> LruState:
    """Cache with `hot` (ascending ids) in slots 0..len(hot)-1 (tests/lru/test_lru.py:53-72)."""
    hot = np.asarray(hot, dtype=np.int64)
    table = np.full(E, -1, np.int32)
    table[hot] = np.arange(len(hot), dtype=np.int32)
    map_cold = np.arange(E, dtype=np.int32)
    map_cold[hot] = -1
    se = np.full(S, -1, np.int32)
    se[:len(hot)] = hot
    st = np.zeros(S, np.int64) if stamps is None else np.asarray(stamps, np.int64).copy()
    return LruState(table, map_cold, se, st, np.zeros(E, np.uint8),
                    np.array([step], np.int64), np.full((cap, 2), miss_fill, np.int32),
                    np.zeros(1, np.int32),
                    max_distinct=E if max_distinct is None else max_distinct,
                    max_inserts=cap if max_inserts is None else max_inserts)


def warm_start(E: int, S: int, hot_ids, rank: dict | None, thresh: float = 0.5,
               max_inserts: int = 64) -> LruState:
    """_build_lru (patches/.../r4d_mxfp4_moe.py.lru.diff:502-541).

    Slot i holds the i-th smallest hot id; stamps = S - argsort(argsort(profile rank)), so the
    hottest expert gets S and the coldest 1 (zeros when there is no profile); step = S;
    max_distinct = max(1, int(S * thresh)); cap = min(max_inserts, S)."""
    hot = np.sort(np.asarray(hot_ids, np.int64))
    assert len(hot) == S
    if rank is None:
        stamps = np.zeros(S, np.int64)
    else:
        r = np.array([rank.get(int(e), len(rank)) for e in hot], np.int64)
        stamps = S - np.argsort(np.argsort(r, kind="stable"), kind="stable")
    cap = min(max_inserts, S)
    return make_state(E, S, hot, stamps, step=S, cap=cap,
                      max_distinct=max(1, int(S * thresh)), max_inserts=cap)


def victim_keys(se: np.ndarray, st: np.ndarray, routed: np.ndarray) -> np.ndarray:
    """(stamp << 20) | slot, or LLONG_MAX for a slot whose expert is routed this step
    (r4d_lru.hip:124-130). Computed with int64 wrap-around, exactly as the device shift."""
    E = routed.shape[0]
    S = se.shape[0]
    idx = np.arange(S, dtype=np.int64)
    with np.errstate(over="ignore"):
        key = (st.astype(np.int64) << np.int64(SLOT_BITS)) | idx
    safe = np.clip(se, 0, E - 1)
    busy = (se >= 0) & (se < E) & (routed[safe] != 0)
    return np.where(busy, LLONG_MAX, key)


def manage(s: LruState, topk_ids: np.ndarray, max_distinct: int | None = None,
           max_inserts: int | None = None) -> int:
    """One lru_manage_k call (r4d_lru.hip:187-269) on state `s`, in place. Returns n_miss.

    1. step += 1; n_miss = 0; routed = experts named by ids in [0, E) (:208-220)
    2. distinct > max_distinct -> read-through: nothing else changes (:222-226)
    3. hits refresh slot_stamp[table[e]] = step (:228-238)
    4. misses in ascending expert id, the first nins = min(#miss, max_inserts) written to
       miss[j, 0] (:239-251)
    5. victims = the nins smallest victim keys of the slots evictable on entry, ascending;
       rank r installs miss r (:79-185); n_miss = number installed (:264-268)
    """
    md = s.max_distinct if max_distinct is None else max_distinct
    mi = s.max_inserts if max_inserts is None else max_inserts
    E, S = s.E, s.S
    ids = np.asarray(topk_ids, dtype=np.int64).reshape(-1)
    s.step[0] += 1
    st = s.step[0]
    s.n_miss[0] = 0
    routed = np.zeros(E, np.uint8)
    routed[ids[(ids >= 0) & (ids < E)]] = 1
    s.routed[:] = routed
    if int(routed.sum()) > md:
        return 0
    rexp = np.nonzero(routed)[0]
    slots = s.table[rexp]
    hit = slots >= 0
    s.slot_stamp[slots[hit]] = st
    misses = rexp[~hit]
    nins = min(len(misses), mi)
    if nins <= 0:
        return 0
    missf = s.miss.reshape(-1)
    missf[0:2 * nins:2] = misses[:nins]
    key = victim_keys(s.slot_expert, s.slot_stamp, routed)
    cand = np.nonzero(key != LLONG_MAX)[0]
    order = cand[np.argsort(key[cand], kind="stable")]
    vic = order[:nins]
    for r, sl in enumerate(vic.tolist()):
        e = int(misses[r])
        old = int(s.slot_expert[sl])
        if old >= 0:
            s.table[old] = -1
            s.map_cold[old] = old
        s.slot_expert[sl] = e
        s.slot_stamp[sl] = st
        s.table[e] = sl
        s.map_cold[e] = -1
        missf[2 * r + 1] = sl
    s.n_miss[0] = len(vic)
    return len(vic)


def align(topk_ids: np.ndarray, E: int, S: int, table: np.ndarray, bs: int, L: int,
          NB: int) -> tuple[np.ndarray, ...]:
    """Both moe_align_block_size outputs from one table (r4d_lru.hip:502-575).

    A valid token (id in [0, E)) whose expert sits in slot s (0 <= table[e] < S) goes to hot
    bucket s, any other valid token to cold bucket e. Each bucket's run of flat token
    indices, ascending, is padded up to a multiple of bs with the sentinel mk; buckets are
    laid out in bucket order; expert_ids[b] names the bucket of block b and is -1 past npad.
    Returns (sorted_hot, eids_hot, npad_hot, sorted_cold, eids_cold, npad_cold)."""
    ids = np.asarray(topk_ids, dtype=np.int64).reshape(-1)
    mk = ids.shape[0]
    valid = (ids >= 0) & (ids < E)
    slot = np.full(mk, -1, np.int64)
    slot[valid] = table[ids[valid]]
    hot = valid & (slot >= 0) & (slot < S)
    cold = valid & ~hot
    out = []
    for mask, key, nbk in ((hot, slot, S), (cold, ids, E)):
        sorted_ids = np.full(L, mk, np.int32)
        eids = np.full(NB, -1, np.int32)
        tok = np.nonzero(mask)[0]
        k = key[tok]
        order = np.argsort(k, kind="stable")
        tok, k = tok[order], k[order]
        cnt = np.bincount(k, minlength=nbk).astype(np.int64) if len(k) else np.zeros(nbk, np.int64)
        padded = (cnt + bs - 1) // bs * bs
        cum = np.concatenate([[0], np.cumsum(padded)])
        pos = cum[k] + (np.arange(len(k)) - np.concatenate([[0], np.cumsum(cnt)])[k])
        sorted_ids[pos] = tok
        for b in np.nonzero(cnt)[0]:
            eids[cum[b] // bs:cum[b + 1] // bs] = b
        out += [sorted_ids, eids, np.array([cum[-1]], np.int32)]
    return tuple(out)


def fused(s: LruState, topk_ids: np.ndarray, bs: int, L: int | None = None,
          NB: int | None = None, max_distinct: int | None = None,
          max_inserts: int | None = None) -> tuple[np.ndarray, ...]:
    """lru_fused_k (r4d_lru.hip:418-575): manage(), then align() from the updated table."""
    ids = np.asarray(topk_ids).reshape(-1)
    if L is None or NB is None:
        L, NB = align_sizes(ids.shape[0], s.E, bs)
    manage(s, ids, max_distinct, max_inserts)
    return align(ids, s.E, s.S, s.table, bs, L, NB)


def gather(dsts: list[np.ndarray], srcs: list[np.ndarray], miss: np.ndarray,
           n_miss: int) -> None:
    """lru_gather_k (r4d_lru.hip:271-301): for j < n_miss copy expert miss[j,0]'s slab of every
    buffer into slot miss[j,1]. Buffers are [rows, bytes_per_row] uint8 views."""
    m = np.asarray(miss).reshape(-1, 2)
    for j in range(int(n_miss)):
        e, sl = int(m[j, 0]), int(m[j, 1])
        for d, src in zip(dsts, srcs):
            d[sl] = src[e]


def check_invariants(s: LruState) -> list[str]:
    """tests/lru/test_lru.py:138-145 and test_slots_prod.py:183-197."""
    bad = []
    t, c, se = s.table, s.map_cold, s.slot_expert
    E = s.E
    if not (((t >= 0) & (c == -1)) | ((t < 0) & (c == np.arange(E)))).all():
        bad.append("table/map_cold not complementary")
    live = se[se >= 0]
    if len(np.unique(live)) != len(live):
        bad.append("duplicate expert in slots")
    if not (t[live] == np.nonzero(se >= 0)[0]).all():
        bad.append("table/slot mismatch")
    if int((t >= 0).sum()) != len(live):
        bad.append("resident count != live slots")
    return bad
