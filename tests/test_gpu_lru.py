"""GPU parity of the device LRU (r4d_lru_manage / r4d_lru_fused / r4d_lru_gather) through the
C-ABI, against the numpy oracle and against the reference's own kernel compiled from
/root/reference by oracle/Makefile (oracle/_ref/librlu_ref.so, when present).

Mirrors tests/lru/test_lru.py (policy suites + gather byte identity), tests/lru/test_fused.py
(fused vs manager + align, edges, HIP-graph replay, negative control) and
tests/lru/test_victim_equiv.py (19 victim cases), all bit-exact.
"""
from __future__ import annotations

import ctypes
import pathlib

import numpy as np
import pytest

from conftest import gpu_case
from lru_cases import POLICY_SUITES, VICTIM_CASES, c1_trace, policy_start, victim_case
from oracle import fp8
from oracle import lru as olru

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda"
BS = 16
REF_SO = pathlib.Path(__file__).resolve().parent.parent / "oracle" / "_ref" / "librlu_ref.so"
NAMES = olru.LruState.NAMES


def to_dev(s: olru.LruState) -> dict:
    return {n: torch.from_numpy(np.ascontiguousarray(getattr(s, n))).to(DEV) for n in NAMES}


def from_dev(d: dict, like: olru.LruState) -> olru.LruState:
    out = like.copy()
    for n in NAMES:
        getattr(out, n)[...] = d[n].cpu().numpy()
    return out


def assert_state(got: dict, want: olru.LruState, tag: str, skip=("routed",)):
    for n in NAMES:
        if n in skip:
            continue
        g = got[n].cpu().numpy()
        w = getattr(want, n)
        assert np.array_equal(g, w), f"{tag}: '{n}' differs in {int((g != w).sum())} entries"


def call(libh, fn, ids_t, d, md, mi, out=None, bs=BS):
    args = [ctypes.c_void_p(d[n].data_ptr()) for n in NAMES]
    E, S = d["table"].numel(), d["slot_expert"].numel()
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if fn == "manage":
        rc = libh.r4d_lru_manage(ctypes.c_void_p(ids_t.data_ptr()), ids_t.numel(), E, S, md, mi,
                                 *args, st)
    else:
        rc = libh.r4d_lru_fused(ctypes.c_void_p(ids_t.data_ptr()), ids_t.numel(), E, S, md, mi,
                                *args, bs, out[0].numel(), out[1].numel(),
                                *[ctypes.c_void_p(o.data_ptr()) for o in out], st)
    assert rc == 0, f"{fn} rc={rc}"


def new_out(mk, E, bs=BS, fill=None):
    L, NB = olru.align_sizes(mk, E, bs)
    mk_ = lambda n: (torch.empty(n, dtype=torch.int32, device=DEV) if fill is None
                     else torch.full((n,), fill, dtype=torch.int32, device=DEV))
    return [mk_(L), mk_(NB), mk_(1), mk_(L), mk_(NB), mk_(1)]


@pytest.fixture(scope="module")
def mine(pkg):
    return pkg.lib()


@pytest.fixture(scope="module")
def ref():
    if not REF_SO.exists():
        pytest.skip("reference library not built (oracle/Makefile ref needs /root/reference)")
    h = ctypes.CDLL(str(REF_SO))
    P, I = ctypes.c_void_p, ctypes.c_int
    h.r4d_lru_manage.restype = I
    h.r4d_lru_manage.argtypes = [P] + [I] * 5 + [P] * 9
    h.r4d_lru_fused.restype = I
    h.r4d_lru_fused.argtypes = [P] + [I] * 5 + [P] * 8 + [I] * 3 + [P] * 7
    return h


@pytest.mark.parametrize("suite", POLICY_SUITES, ids=[s[0] for s in POLICY_SUITES])
def test_policy_manage_vs_oracle(mine, suite):
    """tests/lru/test_lru.py:148-169: every field after every step."""
    name, E, S, gen, nsteps, md, mi = suite
    rng, s = policy_start(E, S, maxi=mi)
    d = to_dev(s)
    for n in range(nsteps):
        ids = gen(rng, n).ravel().astype(np.int32)
        olru.manage(s, ids, md, mi)
        gpu_case(f"policy {name} step {n} E={E} S={S} mk={ids.size}") if n == 0 else None
        call(mine, "manage", torch.from_numpy(ids).to(DEV), d, md, mi)
        torch.cuda.synchronize()
        assert_state(d, s, f"{name} step {n}", skip=())
        assert not olru.check_invariants(s)


def test_c1_fused_vs_oracle_and_golden(mine):
    """The 64-step LRU workload (E=512, S=257, top-10, 5 rows): state and both align outputs
    bit-exact against the oracle after every step, and against the committed fixture."""
    ids_all, s = c1_trace()
    gold = np.load(pathlib.Path(__file__).parent / "golden" / "lru_c1.npz")
    d = to_dev(s)
    mk = ids_all.shape[1]
    for n in range(ids_all.shape[0]):
        want = olru.fused(s, ids_all[n], BS)
        out = new_out(mk, 512, fill=-12345)
        gpu_case(f"c1 fused step {n}") if n == 0 else None
        call(mine, "fused", torch.from_numpy(ids_all[n]).to(DEV), d, s.max_distinct,
             s.max_inserts, out)
        torch.cuda.synchronize()
        assert_state(d, s, f"c1 step {n}", skip=())
        for i, (g, w) in enumerate(zip(out, want)):
            assert np.array_equal(g.cpu().numpy(), w), f"c1 step {n}: align output {i}"
        for i, name in enumerate(("sorted_hot", "eids_hot", "npad_hot", "sorted_cold",
                                  "eids_cold", "npad_cold")):
            assert np.array_equal(out[i].cpu().numpy(), gold[f"{name}_{n}"]), (n, name)
        for name in NAMES:
            assert np.array_equal(d[name].cpu().numpy(), gold[f"{name}_{n}"]), (n, name)


@pytest.mark.parametrize("case", VICTIM_CASES, ids=[c[0] for c in VICTIM_CASES])
@pytest.mark.parametrize("fn", ["manage", "fused"])
def test_victim_cases_vs_oracle(mine, case, fn):
    """tests/lru/test_victim_equiv.py:137-182 against the oracle (full state, all outputs)."""
    name, kw = case
    ids, s = victim_case(**kw)
    d = to_dev(s)
    gpu_case(f"victim {name} {fn} E={s.E} S={s.S} mk={ids.size} maxi={kw['maxi']}")
    out = new_out(ids.size, s.E, fill=-12345) if fn == "fused" else None
    call(mine, fn, torch.from_numpy(ids).to(DEV), d, s.max_distinct, s.max_inserts, out)
    torch.cuda.synchronize()
    want = olru.fused(s, ids, BS) if fn == "fused" else olru.manage(s, ids)
    assert_state(d, s, name, skip=())
    if fn == "fused":
        for i, (g, w) in enumerate(zip(out, want)):
            assert np.array_equal(g.cpu().numpy(), w), f"{name}: align output {i}"


def _cmp_align_multiset(g, r, mk, bs=BS):
    """tests/lru/test_fused.py:133-173: npad and expert_ids exact, sorted_ids as a multiset per
    bucket, sentinel past npad."""
    gs, ge, gn = [x.cpu().numpy() for x in g]
    rs, re_, rn = [x.cpu().numpy() for x in r]
    assert gn[0] == rn[0]
    assert np.array_equal(ge, re_)
    n = int(gn[0])
    by = lambda s_, e_: {int(k): sorted(s_[:n][np.repeat(e_[:n // bs], bs) == k].tolist())
                         for k in np.unique(e_[:n // bs])}
    assert by(gs, ge) == by(rs, re_)
    assert (gs[n:] == mk).all() and (rs[n:] == mk).all()


@pytest.mark.parametrize("case", VICTIM_CASES, ids=[c[0] for c in VICTIM_CASES])
def test_victim_cases_vs_reference_kernel(mine, ref, case):
    """Same pristine state through this library and through the reference kernel compiled
    from kernels/lru/r4d_lru.hip: the whole state bit-exact; align exact when mk <= 256 (the
    reference's deterministic path), per-bucket multiset above (its atomic cursors)."""
    name, kw = case
    ids, s = victim_case(**kw)
    ids_t = torch.from_numpy(ids).to(DEV)
    for fn in ("manage", "fused"):
        a, b = to_dev(s), to_dev(s)
        oa = new_out(ids.size, s.E, fill=-12345) if fn == "fused" else None
        ob = new_out(ids.size, s.E, fill=-12345) if fn == "fused" else None
        gpu_case(f"vs-ref {name} {fn}")
        call(mine, fn, ids_t, a, s.max_distinct, s.max_inserts, oa)
        call(ref, fn, ids_t, b, s.max_distinct, s.max_inserts, ob)
        torch.cuda.synchronize()
        for n in NAMES:
            assert torch.equal(a[n], b[n]), f"{name}/{fn}: '{n}' differs from the reference"
        if fn == "fused":
            if ids.size <= 256:
                for i in range(6):
                    assert torch.equal(oa[i], ob[i]), f"{name}: align output {i}"
            else:
                _cmp_align_multiset(oa[0:3], ob[0:3], ids.size)
                _cmp_align_multiset(oa[3:6], ob[3:6], ids.size)


@pytest.mark.parametrize("rows", [40, 205])
def test_chunked_sizes_vs_reference_kernel(mine, ref, rows):
    """tests/lru/test_fused.py:265-280's largest sizes (mk 400 and 2050) through both kernels
    from the same state, 3 steps with inserts: state bit-exact, buckets equal as multisets
    (the reference places above 256 ids with atomic cursors). At mk 2050 this library ranks
    the ids in its many-workgroup placement kernel."""
    E, S = 512, 257
    rng = np.random.default_rng(rows)
    _, s = victim_case(E=E, S=S, mk=10, k_cold=0, maxi=64, seed=9)
    s.max_distinct = E
    a, b = to_dev(s), to_dev(s)
    for n in range(3):
        pool = rng.choice(E, 350, replace=False)
        ids = np.concatenate([rng.choice(pool, 10, replace=False)
                              for _ in range(rows)]).astype(np.int32)
        ids_t = torch.from_numpy(ids).to(DEV)
        oa, ob = new_out(ids.size, E, fill=-12345), new_out(ids.size, E, fill=-12345)
        gpu_case(f"vs-ref chunked rows={rows} step {n}")
        call(mine, "fused", ids_t, a, s.max_distinct, s.max_inserts, oa)
        call(ref, "fused", ids_t, b, s.max_distinct, s.max_inserts, ob)
        torch.cuda.synchronize()
        for nm in NAMES:
            assert torch.equal(a[nm], b[nm]), f"rows={rows} step {n}: '{nm}'"
        assert int(a["n_miss"].item()) > 0
        _cmp_align_multiset(oa[0:3], ob[0:3], ids.size)
        _cmp_align_multiset(oa[3:6], ob[3:6], ids.size)


def test_c1_trace_vs_reference_kernel(mine, ref):
    """The 64-step trace through both kernels, side by side: identical state every step."""
    ids_all, s = c1_trace()
    a, b = to_dev(s), to_dev(s)
    for n in range(ids_all.shape[0]):
        ids_t = torch.from_numpy(ids_all[n]).to(DEV)
        oa, ob = new_out(50, 512), new_out(50, 512)
        call(mine, "fused", ids_t, a, s.max_distinct, s.max_inserts, oa)
        call(ref, "fused", ids_t, b, s.max_distinct, s.max_inserts, ob)
        torch.cuda.synchronize()
        for nm in NAMES:
            assert torch.equal(a[nm], b[nm]), f"step {n}: '{nm}'"
        for i in range(6):
            assert torch.equal(oa[i], ob[i]), f"step {n}: align output {i}"


@pytest.mark.parametrize("rows", [1, 4, 20, 40, 205, 4096])
def test_fused_geometries(mine, rows):
    """tests/lru/test_fused.py:265-280: mk = 10 .. 2050 incl. the chunked placement path, and
    a 4096-token prefill chunk (mk = 40960)."""
    E, S = 512, 257
    rng = np.random.default_rng(7)
    from conftest import load_pkg
    otrace = load_pkg().traces
    p = otrace.zipf_p(E, 1.1)
    _, s = victim_case(E=E, S=S, mk=10, k_cold=0, maxi=64, seed=3)
    s.max_distinct = max(1, int(S * 0.5))
    d = to_dev(s)
    for n in range(6):
        ids = np.concatenate([rng.choice(E, 10, replace=False, p=p)
                              for _ in range(rows)]).astype(np.int32)
        want = olru.fused(s, ids, BS)
        out = new_out(ids.size, E, fill=-12345)
        gpu_case(f"geometry rows={rows} step {n}") if n == 0 else None
        call(mine, "fused", torch.from_numpy(ids).to(DEV), d, s.max_distinct, s.max_inserts,
             out)
        torch.cuda.synchronize()
        assert_state(d, s, f"rows={rows} step {n}", skip=())
        for i, (g, w) in enumerate(zip(out, want)):
            assert np.array_equal(g.cpu().numpy(), w), f"rows={rows} step {n}: output {i}"
        # hot + cold partition [0, mk) (tests/lru/test_fused.py:186-195)
        hot = out[0].cpu().numpy()[:int(out[2].item())]
        cold = out[3].cpu().numpy()[:int(out[5].item())]
        tok = np.sort(np.concatenate([hot[hot != ids.size], cold[cold != ids.size]]))
        assert np.array_equal(tok, np.arange(ids.size))


PLACE_CASES = [
    # (tag, mk, bs, L override, NB override, invalid-id fraction)
    ("just-past-threshold", 1537, 16, None, None, 0.0),
    ("past-threshold-2049", 2049, 16, None, None, 0.0),
    ("ragged-with-invalid-ids", 9001, 16, None, None, 0.05),
    # fewer expert-id blocks than L needs (the library bounds the writes; the reference
    # writes past them): the single-workgroup placement
    ("L-past-the-blocks", 9000, 16, 9000 + 512 * 15, 100, 0.0),
    ("runtime-bs-64", 5000, 64, None, None, 0.02),
    ("ids-not-16-byte-aligned", 7003, 16, None, None, 0.01),
    ("ids-not-16-byte-aligned-single-workgroup", 1001, 16, None, None, 0.01),
    ("single-workgroup-vector-count", 1500, 16, None, None, 0.02),
]


@pytest.mark.parametrize("case", PLACE_CASES, ids=[c[0] for c in PLACE_CASES])
def test_fused_parallel_placement(mine, case):
    """Above 1536 tokens the align's tokens are ranked by many workgroups; the outputs and the
    state stay bit-exact against the oracle: ids outside [0, E) skipped, a runtime block size,
    and a short expert-id array (NB * bs < L), which keeps the single-workgroup placement."""
    tag, mk, bs, L, NB, bad = case
    E, S = 512, 257
    rng = np.random.default_rng(11)
    _, s = victim_case(E=E, S=S, mk=10, k_cold=0, maxi=64, seed=5)
    s.max_distinct = E
    d = to_dev(s)
    L0, NB0 = olru.align_sizes(mk, E, bs)
    L, NB = L or L0, NB or NB0
    for n in range(3):
        pool = rng.choice(E, 350, replace=False)      # leaves unrouted residents to evict
        ids = rng.choice(pool, mk).astype(np.int32)
        nbad = int(bad * mk)
        if nbad:
            at = rng.choice(mk, nbad, replace=False)
            ids[at] = rng.choice(np.array([-1, E, E + 7, -100], np.int32), nbad)
        want = olru.fused(s, ids, bs, L=L, NB=NB)
        out = [torch.full((n_,), -12345, dtype=torch.int32, device=DEV)
               for n_ in (L, NB, 1, L, NB, 1)]
        gpu_case(f"placement {tag} mk={mk} bs={bs} L={L} NB={NB} step {n}")
        ids_t = torch.from_numpy(ids).to(DEV)
        if "aligned" in tag:                          # a view one element into its buffer
            buf = torch.zeros(mk + 1, dtype=torch.int32, device=DEV)
            buf[1:] = ids_t
            ids_t = buf[1:]
            assert ids_t.data_ptr() % 16 == 4
        call(mine, "fused", ids_t, d, s.max_distinct, s.max_inserts, out, bs=bs)
        torch.cuda.synchronize()
        assert_state(d, s, f"{tag} step {n}", skip=())
        for i, (g, w) in enumerate(zip(out, want)):
            assert np.array_equal(g.cpu().numpy(), w), f"{tag} step {n}: output {i}"


def test_fused_prefill_size_graph_replay(mine):
    """A prefill-sized fused call (8200 ids: two launches, the second ranking the ids) captured
    once as a HIP graph and replayed with new routing: each replay's state and outputs equal an
    eager call on a twin state, with eager work and synchronizations between replays."""
    E, S, mk = 512, 257, 8200
    rng = np.random.default_rng(21)
    _, s = victim_case(E=E, S=S, mk=10, k_cold=0, maxi=64, seed=13)
    s.max_distinct = E
    a, b = to_dev(s), to_dev(s)
    ids_st = torch.zeros(mk, dtype=torch.int32, device=DEV)
    oa, ob = new_out(mk, E), new_out(mk, E)
    first = torch.from_numpy(rng.choice(rng.choice(E, 350, replace=False), mk)
                             .astype(np.int32)).to(DEV)
    ids_st.copy_(first)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):                   # step 0 eager on both, off the capture
        call(mine, "fused", ids_st, a, s.max_distinct, s.max_inserts, oa)
        call(mine, "fused", first, b, s.max_distinct, s.max_inserts, ob)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(mine, "fused", ids_st, a, s.max_distinct, s.max_inserts, oa)
    for n in range(3):
        ids = torch.from_numpy(rng.choice(rng.choice(E, 350, replace=False), mk)
                               .astype(np.int32)).to(DEV)
        ids_st.copy_(ids)
        gpu_case(f"prefill-size graph replay {n}")
        g.replay()
        call(mine, "fused", ids, b, s.max_distinct, s.max_inserts, ob)
        torch.cuda.synchronize()
        for nm in NAMES:
            assert torch.equal(a[nm], b[nm]), f"replay {n}: '{nm}'"
        for i in range(6):
            assert torch.equal(oa[i], ob[i]), f"replay {n}: align output {i}"
        assert int(a["n_miss"].item()) > 0
        for o in oa:                                # eager work between replays
            o.fill_(-7)
        torch.cuda.synchronize()
    del g


def test_fused_edges(mine):
    """tests/lru/test_fused.py:282-293: forced read-through and a zero-miss replay."""
    ids_all, s = c1_trace()
    d = to_dev(s)
    for md, tag in ((0, "read-through"), (s.max_distinct, "warm"), (s.max_distinct, "zero-miss")):
        out = new_out(50, 512, fill=-12345)
        want = olru.fused(s, ids_all[0], BS, max_distinct=md)
        gpu_case(f"edge {tag}")
        call(mine, "fused", torch.from_numpy(ids_all[0]).to(DEV), d, md, s.max_inserts, out)
        torch.cuda.synchronize()
        assert_state(d, s, tag, skip=())
        for i, (g, w) in enumerate(zip(out, want)):
            assert np.array_equal(g.cpu().numpy(), w), f"{tag}: output {i}"
        if tag == "zero-miss":
            assert int(d["n_miss"].item()) == 0


def test_fused_graph_replay(mine):
    """tests/lru/test_fused.py:295-364: 12 replays of a captured call with changing routing
    equal 12 eager calls, state and outputs; a zero-insert step after an inserting one leaves
    no stale output."""
    ids_all, s0 = c1_trace()
    mk = ids_all.shape[1]
    ids_static = torch.zeros(mk, dtype=torch.int32, device=DEV)
    out = new_out(mk, 512)
    d = to_dev(s0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ids_static.copy_(torch.from_numpy(ids_all[0]))
        call(mine, "fused", ids_static, d, s0.max_distinct, s0.max_inserts, out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    gpu_case("graph capture of r4d_lru_fused")
    with torch.cuda.graph(g):
        call(mine, "fused", ids_static, d, s0.max_distinct, s0.max_inserts, out)
    torch.cuda.synchronize()
    fresh = to_dev(s0)
    for n in NAMES:
        d[n].copy_(fresh[n])
    s = s0.copy()
    seq = list(range(12)) + [11]          # the last replay repeats routing: zero inserts
    for k, n in enumerate(seq):
        ids_static.copy_(torch.from_numpy(ids_all[n]))
        g.replay()
        torch.cuda.synchronize()
        want = olru.fused(s, ids_all[n], BS)
        assert_state(d, s, f"replay {k}", skip=())
        for i, (gg, w) in enumerate(zip(out, want)):
            assert np.array_equal(gg.cpu().numpy(), w), f"replay {k}: output {i}"
    assert int(d["n_miss"].item()) == 0


def _uva(nbytes):
    t = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    hip = ctypes.CDLL("libamdhip64.so")
    dp = ctypes.c_void_p()
    rc = hip.hipHostGetDevicePointer(ctypes.byref(dp), ctypes.c_void_p(t.data_ptr()),
                                     ctypes.c_uint(0))
    assert rc == 0, f"hipHostGetDevicePointer rc={rc}"
    return t, dp.value


def test_gather_bytes_from_pinned_host(pkg):
    """tests/lru/test_lru.py:210-258: 40 steps of manage + gather from pinned host memory;
    every inserted slab of all six buffers byte-equal to its source."""
    E, S = 512, 257
    sizes = [3932160 // 16, 1966080 // 16, 960, 480, 960, 480]   # fp8 layer, scaled down
    g = torch.Generator().manual_seed(1)
    src_h, src_d, dst = [], [], []
    for b in sizes:
        h, dp = _uva(E * b)
        h.copy_(torch.randint(0, 256, (E * b,), dtype=torch.uint8, generator=g))
        src_h.append(h)
        src_d.append(dp)
        dst.append(torch.zeros(S * b, dtype=torch.uint8, device=DEV))
    _, s = victim_case(E=E, S=S, mk=50, k_cold=0, maxi=64, seed=3)
    s.max_distinct = 128
    d = to_dev(s)
    rng = np.random.default_rng(11)
    views_d = [x.view(S, b) for x, b in zip(dst, sizes)]
    views_s = [x.view(E, b) for x, b in zip(src_h, sizes)]
    for n in range(40):
        ids = np.concatenate([rng.choice(E, 10, replace=False) for _ in range(5)]).astype(np.int32)
        olru.manage(s, ids)
        gpu_case(f"gather step {n}") if n == 0 else None
        call(pkg.lib(), "manage", torch.from_numpy(ids).to(DEV), d, s.max_distinct,
             s.max_inserts)
        pkg._r4d_lru_gather(views_d, views_s, d["miss"], d["n_miss"], 8, 16, src_ptrs=src_d)
        torch.cuda.synchronize()
        assert_state(d, s, f"gather step {n}", skip=())
        nm = int(s.n_miss[0])
        for e, sl in s.miss[:nm].tolist():
            for i in range(6):
                assert torch.equal(views_d[i][sl].cpu(), views_s[i][e]), (n, e, sl, i)


def test_gather_rejects_bad_sizes(pkg):
    d = torch.zeros(64, dtype=torch.uint8, device=DEV).view(4, 16)
    bad = torch.zeros(4, 8, dtype=torch.uint8, device=DEV)
    m = torch.zeros(4, 2, dtype=torch.int32, device=DEV)
    nm = torch.zeros(1, dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError):
        pkg._r4d_lru_gather([bad] * 6, [bad] * 6, m, nm, 8, 16)
    with pytest.raises(RuntimeError):
        pkg._r4d_lru_gather([d] * 6, [d] * 6, m, nm, 0, 16)


@pytest.mark.parametrize("rows", [5, 7, 20, 4100])
def test_fused_quant_equals_fused_then_quant(pkg, rows):
    """rlu_lru_fused_quant == r4d_lru_fused followed by rlu_quant_fp8_group(group 128), bit for
    bit: cache state, both align outputs, e4m3 codes and scales; a row count that leaves a
    quant workgroup part-used, and a prefill-sized chunk (8200 ids: the parallel placement)."""
    from importlib import import_module
    ops = import_module(pkg.__name__ + ".ops")
    ids_all, s = c1_trace()
    rng = np.random.default_rng(rows)
    E, S = 512, 257
    a = pkg.LruCache.build(E, s.slot_expert.tolist(), None, DEV)
    b = pkg.LruCache.build(E, s.slot_expert.tolist(), None, DEV)
    for t, (sa, sb) in enumerate(zip(a.state(), b.state())):
        sa.copy_(torch.from_numpy(np.ascontiguousarray(getattr(s, NAMES[t]))).to(DEV))
        sb.copy_(sa)
    x = torch.from_numpy(fp8.bf16_round(rng.standard_normal((rows, 2560)).astype(np.float32)
                                        * 3)).to(torch.bfloat16).to(DEV)
    for n in range(3):
        ids = np.concatenate([ids_all[n + k % 4] for k in range(rows // 5)]).astype(np.int32)
        idt = torch.from_numpy(ids).to(DEV)
        oa, ob = a.alloc_align(ids.size), b.alloc_align(ids.size)
        q1 = torch.empty((rows, 2560), dtype=torch.float8_e4m3fn, device=DEV)
        s1 = torch.empty((rows, 20), dtype=torch.float32, device=DEV)
        gpu_case(f"fused quant rows={rows} step {n}")
        a.fused_quant(idt, oa, x, q1, s1)
        b.fused(idt, out=ob)
        q2, s2 = ops.fp8_quant_group(x, 128)
        torch.cuda.synchronize()
        for ta, tb in zip(a.state(), b.state()):
            assert torch.equal(ta, tb)
        for ta, tb in zip(oa, ob):
            assert torch.equal(ta, tb)
        assert torch.equal(q1.view(torch.uint8), q2.view(torch.uint8))
        assert torch.equal(s1, s2)


@pytest.mark.parametrize("rows,seed", [(5, 1), (20, 2), (20, 3)])
def test_split_fresh_partitions_the_hot_align(pkg, rows, seed):
    """rlu_lru_split_fresh on the fused kernel's own outputs, over steps of a Zipf trace: each
    block of eids_hot lands in exactly one bucket (-1 blocks in neither); a block is in the
    installed bucket exactly when its slot changed hands this step (slot_expert before the
    step differs), i.e. when the gather writes it."""
    from importlib import import_module
    lru = import_module(pkg.__name__ + ".lru")
    E, S, steps = 128, 100, 4
    tr, perm0 = pkg.traces.zipf_trace(seed=seed, E=E, rows=rows, k=10, steps=steps, s=1.1,
                                      corr=0.7 if rows >= 20 else 0.0)
    hot, rank = pkg.traces.warm_hot(perm0, S)
    cache = lru.LruCache.build(E, hot, rank, DEV, thresh=1.0)
    out = cache.alloc_align(rows * 10, BS)
    res, new = torch.empty_like(out[1]), torch.empty_like(out[1])
    seen_new = 0
    for t in range(steps):
        gpu_case(f"split_fresh rows={rows} seed={seed} step {t}")
        before = cache.slot_expert.cpu().numpy().copy()
        cache.fused(torch.from_numpy(tr[t]).to(DEV), out=out, block_size=BS)
        lru.split_fresh(out[1], cache.miss, cache.n_miss, S, res, new)
        torch.cuda.synchronize()
        eids = out[1].cpu().numpy()
        r, n = res.cpu().numpy(), new.cpu().numpy()
        after = cache.slot_expert.cpu().numpy()
        live = eids >= 0
        assert (r[~live] == -1).all() and (n[~live] == -1).all()
        changed = np.zeros(S, bool)
        changed[before != after] = True
        for b in np.nonzero(live)[0]:
            s = eids[b]
            if changed[s]:
                assert n[b] == s and r[b] == -1, (t, b)
                seen_new += 1
            else:
                assert r[b] == s and n[b] == -1, (t, b)
    assert seen_new > 0, "the trace must install experts"


def test_split_fresh_clamps_to_the_miss_capacity(pkg):
    """n_miss larger than the miss buffer reads only the buffer; bad sizes return -1."""
    from importlib import import_module
    lru = import_module(pkg.__name__ + ".lru")
    lib = pkg._lib.lib()
    eids = torch.tensor([3, 5, 7, 3, -1, -1], dtype=torch.int32, device=DEV)
    miss = torch.tensor([[9, 5], [11, 7]], dtype=torch.int32, device=DEV)
    n_miss = torch.tensor([7], dtype=torch.int32, device=DEV)
    res, new = torch.empty_like(eids), torch.empty_like(eids)
    gpu_case("split_fresh clamp")
    lru.split_fresh(eids, miss, n_miss, 8, res, new)
    torch.cuda.synchronize()
    assert res.tolist() == [3, -1, -1, 3, -1, -1]
    assert new.tolist() == [-1, 5, 7, -1, -1, -1]
    n_miss.fill_(0)
    lru.split_fresh(eids, miss, n_miss, 8, res, new)
    torch.cuda.synchronize()
    assert res.tolist() == eids.tolist() and new.tolist() == [-1] * 6
    P = ctypes.c_void_p
    for nb, cap, S in ((-1, 2, 8), (6, -1, 8), (6, 2, 0), (6, 2, 1025)):
        assert lib.rlu_lru_split_fresh(P(eids.data_ptr()), nb, P(miss.data_ptr()),
                                       P(n_miss.data_ptr()), cap, S, P(res.data_ptr()),
                                       P(new.data_ptr()), None) == -1


def test_multilayer_graph_fused_and_gather(pkg, mine):
    """tests/lru/test_graph_lru.py:102-158: several layers of (fused manager + align, then the
    miss gather on a side stream) captured as one HIP graph and replayed 20 times with new
    routing: after every replay each layer's cache state and align outputs equal the oracle's,
    and every slot of every layer holds its expert's bytes in all six buffers (the slot
    audit of tests/lru/test_slots_prod.py:199-207)."""
    L, E, S, rows, steps = 8, 128, 64, 5, 21
    sizes = [4096, 2048, 64, 32, 64, 32]
    g = torch.Generator().manual_seed(5)
    src_h, src_d = [], []
    for b in sizes:
        h, dp = _uva(E * b)
        h.copy_(torch.randint(0, 256, (E * b,), dtype=torch.uint8, generator=g))
        src_h.append(h.view(E, b))
        src_d.append(dp)
    layers = []
    for l in range(L):
        tr, perm0 = pkg.traces.zipf_trace(seed=700 + l, E=E, rows=rows, k=10, steps=steps,
                                          s=1.1)
        hot, rank = pkg.traces.warm_hot(perm0, S)
        st = olru.warm_start(E, S, hot, rank, thresh=1.0)    # 5-10 inserts a step
        d = to_dev(st)
        slots = [torch.empty((S, b), dtype=torch.uint8, device=DEV) for b in sizes]
        idx = torch.from_numpy(st.slot_expert.astype(np.int64))
        for i in range(6):
            slots[i].copy_(src_h[i].index_select(0, idx))
        layers.append(dict(tr=tr, st=st, d=d, slots=slots, out=new_out(rows * 10, E),
                           ids=torch.zeros(rows * 10, dtype=torch.int32, device=DEV)))
    side = torch.cuda.Stream()

    def step():
        cur = torch.cuda.current_stream()
        for ly in layers:
            call(mine, "fused", ly["ids"], ly["d"], ly["st"].max_distinct, ly["st"].max_inserts,
                 ly["out"])
            side.wait_stream(cur)
            with torch.cuda.stream(side):
                pkg._r4d_lru_gather(ly["slots"], src_h, ly["d"]["miss"], ly["d"]["n_miss"], 4,
                                    32, src_ptrs=src_d)
            cur.wait_stream(side)

    def check(n, tag):
        inserts = 0
        for l, ly in enumerate(layers):
            want = olru.fused(ly["st"], ly["tr"][n], BS)
            inserts += int(ly["st"].n_miss[0])
            assert_state(ly["d"], ly["st"], f"{tag} layer {l}", skip=())
            for i, (gg, w) in enumerate(zip(ly["out"], want)):
                assert np.array_equal(gg.cpu().numpy(), w), f"{tag} layer {l}: output {i}"
            idx = torch.from_numpy(ly["st"].slot_expert.astype(np.int64))
            for i in range(6):
                assert torch.equal(ly["slots"][i].cpu(), src_h[i].index_select(0, idx)), \
                    f"{tag} layer {l}: buffer {i}"
        return inserts

    # step 0 eager on a side stream (loads the kernels), then capture, then 20 replays
    gpu_case("multi-layer graph: eager step 0")
    for ly in layers:
        ly["ids"].copy_(torch.from_numpy(ly["tr"][0]))
    s0 = torch.cuda.Stream()
    s0.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s0):
        step()
    torch.cuda.current_stream().wait_stream(s0)
    torch.cuda.synchronize()
    check(0, "eager step 0")
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        step()
    torch.cuda.synchronize()
    total = 0
    for n in range(1, steps):
        gpu_case(f"multi-layer graph replay {n}")
        for ly in layers:
            ly["ids"].copy_(torch.from_numpy(ly["tr"][n]))
        gr.replay()
        torch.cuda.synchronize()
        total += check(n, f"replay {n}")
    assert total > 0, "the traces must insert"
    del gr


def test_manage_negative_mk_is_no_tokens(mine, ref):
    """kernels/lru/r4d_lru.hip:583-587 launches for any mk; its loops over mk ids then run zero
    times: step advances, n_miss = 0, nothing else changes. The same here, side by side."""
    ids, s = victim_case(E=512, S=257, mk=50, k_cold=5, maxi=64, seed=4)
    want = s.copy()
    olru.manage(want, np.zeros(0, np.int32))
    ids_t = torch.from_numpy(ids.astype(np.int32)).to(DEV)
    for libh, tag in ((mine, "mine"), (ref, "ref")):
        d = to_dev(s)
        args = [ctypes.c_void_p(d[n].data_ptr()) for n in NAMES]
        gpu_case(f"manage mk=-5 ({tag})")
        rc = libh.r4d_lru_manage(ctypes.c_void_p(ids_t.data_ptr()), -5, 512, 257,
                                 s.max_distinct, s.max_inserts, *args,
                                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert rc == 0
        torch.cuda.synchronize()
        assert_state(d, want, f"mk<0 {tag}")
