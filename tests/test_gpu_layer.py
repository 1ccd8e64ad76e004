"""GPU: LruMoELayer.apply (the _apply_split path, r4d_mxfp4_moe.py.lru.diff:659-696) end to end
against the oracle pipeline, over consecutive decode steps of Zipf routing with misses.

Per step:
* the cache state after the step equals oracle.lru.fused's, bit for bit (table, map_cold,
  slot_expert, slot_stamp, step, miss, n_miss);
* residency: after the side-stream gather every slot holds the bytes of the expert its
  slot_expert entry names, in all four per-expert buffers (w13, s13, w2, s2);
* the layer output is within 2e-2 of max|ref| of the oracle pipeline: group-128 quant, float64
  gate_up GEMM over the row-major weights, bf16, SiLU-mul-quant, float64 down GEMM x routed
  weights, bf16, moe_sum -- computed with every expert resident (the hot/cold partition must not
  change the result).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import gpu_case
from oracle import fp8, gemm as ogemm
from oracle import lru as olru
from conftest import load_pkg
trace = load_pkg().traces

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 2e-2
E, S, H, I, TOPK = 128, 100, 2560, 768, 10   # read-through above 50 distinct


@pytest.fixture(scope="module")
def ops(pkg):
    from importlib import import_module
    return import_module(pkg.__name__ + ".ops")


@pytest.fixture(scope="module")
def pool(pkg, ops):
    """E experts: row-major e4m3 copies for the oracle, fragment-order pinned host copies for
    the layer (the gather source and the cold GEMM operand)."""
    g = torch.Generator(device=DEV).manual_seed(7)
    out = {}
    for name, (n, k) in (("w13", (2 * I, H)), ("w2", (H, I))):
        w = torch.randn(E, n, k, device=DEV, generator=g) * 0.02
        b = w.reshape(E, n // 128, 128, k // 128, 128)
        ws = (b.abs().amax(dim=(2, 4)).clamp(min=1e-12) / 448.0).float()
        wq = (b / ws[:, :, None, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn).reshape(E, n, k)
        del w, b
        out[name + "_np"] = wq.view(torch.uint8).cpu().numpy()
        out[name + "s_np"] = ws.cpu().numpy()
        t = ops.shuffle_fp8_weight(wq.contiguous())
        h = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
        h.copy_(t)
        hs = torch.empty(ws.shape, dtype=torch.float32, pin_memory=True)
        hs.copy_(ws)
        out[name], out[name + "s"] = h, hs
    return out


def oracle_layer(x, ids, tw, pool):
    """The pipeline of apply() on the CPU with every expert resident."""
    M = x.shape[0]
    mtk = ids.size
    L, NB = olru.align_sizes(mtk, E, 16)
    s, e, n = olru.align(ids.reshape(-1), E, E, np.arange(E, dtype=np.int32), 16, L, NB)[:3]
    qx, xs = fp8.group_quant(x, 128)
    y1 = ogemm.moe_gemm(qx, xs, pool["w13_np"], pool["w13s_np"], s, e, n, mtk, TOPK)
    _, q2, s2 = fp8.silu_mul_quant(fp8.bf16_round(y1.astype(np.float32)), 128)
    y2 = ogemm.moe_gemm(q2, s2, pool["w2_np"], pool["w2s_np"], s, e, n, mtk, 1,
                        tw=tw.reshape(-1))
    return ogemm.moe_sum(fp8.bf16_round(y2.astype(np.float32)), M, TOPK)


@pytest.mark.parametrize("M", [5, 20])
def test_layer_steps_vs_oracle(pkg, pool, M):
    steps = 4
    tr, perm0 = trace.zipf_trace(seed=300 + M, E=E, rows=M, k=TOPK, steps=steps, s=1.1,
                                 corr=0.7 if M >= 20 else 0.0)
    ids_all = tr.reshape(steps, M, TOPK).astype(np.int32)
    hot, rank = trace.warm_hot(perm0, S)
    full = pkg.ExpertWeights(pool["w13"], pool["w13s"], pool["w2"], pool["w2s"])
    layer = pkg.LruMoELayer(full, hot, rank, M, TOPK, DEV)
    st = olru.warm_start(E, S, hot, rank)
    rng = np.random.default_rng(M)
    side = torch.cuda.Stream()
    total_miss = 0
    for t in range(steps):
        ids = ids_all[t]
        x = fp8.bf16_round(rng.standard_normal((M, H)).astype(np.float32))
        tw = rng.random((M, TOPK)).astype(np.float32)
        out = torch.empty((M, H), dtype=torch.bfloat16, device=DEV)
        gpu_case(f"layer M={M} step {t}")
        layer.apply(out, torch.from_numpy(x).to(torch.bfloat16).to(DEV),
                    torch.from_numpy(tw).to(DEV), torch.from_numpy(ids).to(DEV),
                    gather=True, side=side)
        torch.cuda.synchronize()
        olru.fused(st, ids.reshape(-1), 16)
        for name, got in zip(olru.LruState.NAMES, layer.cache.state()):
            if name == "routed":
                continue
            assert np.array_equal(got.cpu().numpy(), getattr(st, name)), (t, name)
        total_miss += int(st.n_miss[0])
        # residency: slot s holds slot_expert[s]'s bytes in all four buffers
        se = st.slot_expert
        live = np.nonzero(se >= 0)[0]
        idx = torch.from_numpy(se[live].astype(np.int64))
        for name in ("w13", "w13s", "w2", "w2s"):
            src = pool[name].index_select(0, idx)
            dst = getattr(layer.slots, {"w13": "w13", "w13s": "s13", "w2": "w2",
                                        "w2s": "s2"}[name])[torch.from_numpy(live).to(DEV)]
            assert torch.equal(src.view(torch.uint8).reshape(len(live), -1),
                               dst.cpu().view(torch.uint8).reshape(len(live), -1)), (t, name)
        ref = oracle_layer(x, ids, tw, pool)
        got = out.float().cpu().numpy()
        err = ogemm.rel_err(got, ref)
        assert err <= TOL, f"step {t}: rel err {err:.3e}"
    assert total_miss > 0, "the trace must exercise the miss path"


def test_layer_static_arm(pkg, pool):
    """max_inserts = 0 (the static hot/cold arm, r4d_mxfp4_moe.py.static.diff; the README's
    MAX_INSERTS=0 ablation): no insert ever, the warm-start set stays in its slots, every
    other routed expert is computed from the full tensor; state (stamps, step) and output
    match the oracle with the same cap."""
    M, steps = 5, 3
    tr, perm0 = trace.zipf_trace(seed=55, E=E, rows=M, k=TOPK, steps=steps, s=1.1)
    ids_all = tr.reshape(steps, M, TOPK).astype(np.int32)
    hot, rank = trace.warm_hot(perm0, S)
    full = pkg.ExpertWeights(pool["w13"], pool["w13s"], pool["w2"], pool["w2s"])
    layer = pkg.LruMoELayer(full, hot, rank, M, TOPK, DEV, max_inserts=0)
    st = olru.warm_start(E, S, hot, rank, max_inserts=0)
    se0 = layer.cache.slot_expert.cpu().numpy().copy()
    rng = np.random.default_rng(55)
    cold_rows = 0
    for t in range(steps):
        ids = ids_all[t]
        cold_rows += int((~np.isin(ids, hot)).sum())
        x = fp8.bf16_round(rng.standard_normal((M, H)).astype(np.float32))
        tw = rng.random((M, TOPK)).astype(np.float32)
        out = torch.empty((M, H), dtype=torch.bfloat16, device=DEV)
        gpu_case(f"static arm step {t}")
        layer.apply(out, torch.from_numpy(x).to(torch.bfloat16).to(DEV),
                    torch.from_numpy(tw).to(DEV), torch.from_numpy(ids).to(DEV), gather=True)
        torch.cuda.synchronize()
        olru.fused(st, ids.reshape(-1), 16)
        for name, got in zip(olru.LruState.NAMES, layer.cache.state()):
            if name == "routed":
                continue
            assert np.array_equal(got.cpu().numpy(), getattr(st, name)), (t, name)
        assert int(layer.cache.n_miss.item()) == 0
        assert np.array_equal(layer.cache.slot_expert.cpu().numpy(), se0)
        err = ogemm.rel_err(out.float().cpu().numpy(), oracle_layer(x, ids, tw, pool))
        assert err <= TOL, f"step {t}: rel err {err:.3e}"
    assert cold_rows > 0, "the trace must route experts outside the resident set"


@pytest.mark.parametrize("M", [5, 20])
def test_layer_overlap_bit_identical(pkg, pool, M):
    """The three-way split (docs/REVIEW.md:281-301): resident and cold rows computed while the
    side stream gathers, installed rows after it. Two layers from the same warm start, one
    with the overlap and one without, see the same steps: outputs equal bit for bit, cache
    states equal, and the output stays within 2e-2 of the oracle pipeline."""
    steps = 4
    tr, perm0 = trace.zipf_trace(seed=400 + M, E=E, rows=M, k=TOPK, steps=steps, s=1.1,
                                 corr=0.7 if M >= 20 else 0.0)
    ids_all = tr.reshape(steps, M, TOPK).astype(np.int32)
    hot, rank = trace.warm_hot(perm0, S)
    full = pkg.ExpertWeights(pool["w13"], pool["w13s"], pool["w2"], pool["w2s"])
    a = pkg.LruMoELayer(full, hot, rank, M, TOPK, DEV)
    b = pkg.LruMoELayer(full, hot, rank, M, TOPK, DEV)
    rng = np.random.default_rng(400 + M)
    side = torch.cuda.Stream()
    installs = 0
    for t in range(steps):
        ids = ids_all[t]
        x = fp8.bf16_round(rng.standard_normal((M, H)).astype(np.float32))
        tw = rng.random((M, TOPK)).astype(np.float32)
        xd = torch.from_numpy(x).to(torch.bfloat16).to(DEV)
        twd, idd = torch.from_numpy(tw).to(DEV), torch.from_numpy(ids).to(DEV)
        oa = torch.empty((M, H), dtype=torch.bfloat16, device=DEV)
        ob = torch.empty((M, H), dtype=torch.bfloat16, device=DEV)
        gpu_case(f"overlap layer M={M} step {t}")
        a.apply(oa, xd, twd, idd, gather=True, side=side, overlap=True)
        b.apply(ob, xd, twd, idd, gather=True, side=side, overlap=False)
        torch.cuda.synchronize()
        installs += int(a.cache.n_miss.item())
        assert torch.equal(oa.view(torch.int16), ob.view(torch.int16)), f"step {t}"
        for name, ga, gb in zip(olru.LruState.NAMES, a.cache.state(), b.cache.state()):
            assert torch.equal(ga, gb), (t, name)
        err = ogemm.rel_err(oa.float().cpu().numpy(), oracle_layer(x, ids, tw, pool))
        assert err <= TOL, f"step {t}: rel err {err:.3e}"
    assert installs > 0, "the trace must install experts"


def test_layer_overlap_graph_replay(pkg, pool):
    """The overlapped step captured once as a HIP graph (side-stream gather, event between its
    two launches, joins) and replayed with new routing: every replay's output and cache state
    equal an eager layer without the overlap, bit for bit, with eager work and
    synchronizations between the replays."""
    M, steps = 20, 5
    tr, perm0 = trace.zipf_trace(seed=77, E=E, rows=M, k=TOPK, steps=steps, s=1.1, corr=0.7)
    ids_all = tr.reshape(steps, M, TOPK).astype(np.int32)
    hot, rank = trace.warm_hot(perm0, S)
    full = pkg.ExpertWeights(pool["w13"], pool["w13s"], pool["w2"], pool["w2s"])
    a = pkg.LruMoELayer(full, hot, rank, M, TOPK, DEV)
    b = pkg.LruMoELayer(full, hot, rank, M, TOPK, DEV)
    rng = np.random.default_rng(77)
    xs = [torch.from_numpy(fp8.bf16_round(rng.standard_normal((M, H)).astype(np.float32)))
          .to(torch.bfloat16).to(DEV) for _ in range(steps)]
    tws = [torch.from_numpy(rng.random((M, TOPK)).astype(np.float32)).to(DEV)
           for _ in range(steps)]
    x_st, tw_st = torch.empty_like(xs[0]), torch.empty_like(tws[0])
    ids_st = torch.empty((M, TOPK), dtype=torch.int32, device=DEV)
    out_a = torch.empty((M, H), dtype=torch.bfloat16, device=DEV)
    out_b = torch.empty_like(out_a)
    side = torch.cuda.Stream()
    # the routing capture hook rides in the captured step too
    from importlib import import_module
    ring = import_module(pkg.__name__ + ".routecap").RouteRing(1, TOPK, DEV, ring=16, maxrows=M)
    a.route_capture = ring.fn(0)
    # step 0 eager on both (loads every kernel), then capture the overlapped step
    gpu_case("overlap graph: eager step 0")
    ids0 = torch.from_numpy(ids_all[0]).to(DEV)
    a.apply(out_a, xs[0], tws[0], ids0, gather=True, side=side, overlap=True)
    b.apply(out_b, xs[0], tws[0], ids0, gather=True, side=side, overlap=False)
    torch.cuda.synchronize()
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        a.apply(out_a, x_st, tw_st, ids_st, gather=True, side=side, overlap=True)
    torch.cuda.synchronize()
    installs = 0
    for t in range(1, steps):
        gpu_case(f"overlap graph: replay step {t}")
        ids = torch.from_numpy(ids_all[t]).to(DEV)
        x_st.copy_(xs[t])
        tw_st.copy_(tws[t])
        ids_st.copy_(ids)
        g.replay()
        b.apply(out_b, xs[t], tws[t], ids, gather=True, side=side, overlap=False)
        torch.cuda.synchronize()
        installs += int(a.cache.n_miss.item())
        assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16)), f"replay {t}"
        for name, ga, gb in zip(olru.LruState.NAMES, a.cache.state(), b.cache.state()):
            assert torch.equal(ga, gb), (t, name)
        assert torch.equal(a.slots.w2.view(torch.uint8), b.slots.w2.view(torch.uint8)), t
        out_a.zero_()                       # eager work between replays
        torch.cuda.synchronize()
    assert installs > 0, "the trace must install experts"
    ring.poll()                             # steps 1..steps-1 finished; the last is the newest
    got = ring.routes()
    assert list(got["steps"]) == list(range(1, steps))
    for t in range(steps - 1):
        assert np.array_equal(got["ids"][t, 0], ids_all[t].reshape(-1).astype(np.int16))
    assert np.array_equal(ring.ring_ids[0, steps % 16].cpu().numpy(),
                          ids_all[steps - 1].reshape(-1).astype(np.int16))
    del g


def test_layer_overlap_read_through_and_cold_rows(pkg, pool):
    """Overlap across read-through steps (more distinct experts than the gate: no install, the
    non-resident experts run cold in the overlapped phase) alternating with insert steps:
    outputs and states equal the serial order bit for bit, and the oracle within 2e-2."""
    M = 20
    ta, perm0 = trace.zipf_trace(seed=420, E=E, rows=M, k=TOPK, steps=4, s=1.1, corr=0.7)
    tb, _ = trace.zipf_trace(seed=500, E=E, rows=M, k=TOPK, steps=4, s=0.6)
    mix = np.stack([ta[0], tb[0], ta[1], tb[1], ta[2]]).reshape(5, M, TOPK).astype(np.int32)
    hot, rank = trace.warm_hot(perm0, S)
    full = pkg.ExpertWeights(pool["w13"], pool["w13s"], pool["w2"], pool["w2s"])
    a = pkg.LruMoELayer(full, hot, rank, M, TOPK, DEV)
    b = pkg.LruMoELayer(full, hot, rank, M, TOPK, DEV)
    st = olru.warm_start(E, S, hot, rank)
    rng = np.random.default_rng(420)
    side = torch.cuda.Stream()
    kinds = []
    for t in range(mix.shape[0]):
        ids = mix[t]
        x = fp8.bf16_round(rng.standard_normal((M, H)).astype(np.float32))
        tw = rng.random((M, TOPK)).astype(np.float32)
        xd = torch.from_numpy(x).to(torch.bfloat16).to(DEV)
        twd, idd = torch.from_numpy(tw).to(DEV), torch.from_numpy(ids).to(DEV)
        oa = torch.empty((M, H), dtype=torch.bfloat16, device=DEV)
        ob = torch.empty_like(oa)
        gpu_case(f"overlap read-through mix step {t}")
        a.apply(oa, xd, twd, idd, gather=True, side=side, overlap=True)
        b.apply(ob, xd, twd, idd, gather=True, side=side, overlap=False)
        torch.cuda.synchronize()
        olru.fused(st, ids.reshape(-1), 16)
        cold = int((st.map_cold[ids.reshape(-1)] >= 0).sum())
        kinds.append((int(st.n_miss[0]), cold))
        assert torch.equal(oa.view(torch.int16), ob.view(torch.int16)), f"step {t}"
        for name, ga in zip(olru.LruState.NAMES, a.cache.state()):
            if name == "routed":
                continue
            assert np.array_equal(ga.cpu().numpy(), getattr(st, name)), (t, name)
        err = ogemm.rel_err(oa.float().cpu().numpy(), oracle_layer(x, ids, tw, pool))
        assert err <= TOL, f"step {t}: rel err {err:.3e}"
    assert any(n > 0 and c == 0 for n, c in kinds), kinds      # insert steps
    assert any(n == 0 and c > 0 for n, c in kinds), kinds      # read-through, cold rows


def test_layer_prefill_read_through(pkg, pool):
    """A 2048-token chunk (20480 routed rows) through apply(): the layer runs the tiled prefill
    GEMM over the hot and the cold align (tests/lru/test_numerics_prod.py:44-48 runs the same
    read-through chunk through the split path). Step 1 routes uniformly over all 128 experts,
    past the read-through gate (50 distinct): no install, every non-resident expert is read
    from pinned host memory. Step 2 routes over 30 experts, 10 of them not resident: they are
    installed by the side-stream gather while the overlap runs. Per step: the state equals
    the oracle's bit for bit; the output equals a decode-kernel layer's (sk = 1, no overlap)
    bit for bit over all 2048 tokens; sampled tokens are within 2e-2 of the oracle pipeline."""
    M = 2048
    _, perm0 = trace.zipf_trace(seed=600, E=E, rows=20, k=TOPK, steps=1, s=1.1)
    hot, rank = trace.warm_hot(perm0, S)
    full = pkg.ExpertWeights(pool["w13"], pool["w13s"], pool["w2"], pool["w2s"])
    a = pkg.LruMoELayer(full, hot, rank, M, TOPK, DEV)
    b = pkg.LruMoELayer(full, hot, rank, M, TOPK, DEV, sk1=1, sk2=1, prefill_rows=1 << 30)
    assert a.prefill and not b.prefill
    st = olru.warm_start(E, S, hot, rank)
    rng = np.random.default_rng(600)
    cold = [e for e in range(E) if e not in set(hot)]
    narrow = np.array(sorted(list(hot[:20]) + cold[:10]), dtype=np.int32)
    side = torch.cuda.Stream()
    for t, pool_ids in enumerate((np.arange(E, dtype=np.int32), narrow)):
        ids = np.stack([rng.choice(pool_ids, TOPK, replace=False) for _ in range(M)]).astype(np.int32)
        x = fp8.bf16_round(rng.standard_normal((M, H)).astype(np.float32))
        tw = rng.random((M, TOPK)).astype(np.float32)
        xd = torch.from_numpy(x).to(torch.bfloat16).to(DEV)
        twd, idd = torch.from_numpy(tw).to(DEV), torch.from_numpy(ids).to(DEV)
        oa = torch.full((M, H), float("nan"), dtype=torch.bfloat16, device=DEV)
        ob = torch.full_like(oa, float("nan"))
        gpu_case(f"prefill layer step {t}: tiled")
        a.apply(oa, xd, twd, idd, gather=True, side=side)
        gpu_case(f"prefill layer step {t}: decode kernel")
        b.apply(ob, xd, twd, idd, gather=True, side=side)
        torch.cuda.synchronize()
        olru.fused(st, ids.reshape(-1), 16)
        for name, ga in zip(olru.LruState.NAMES, a.cache.state()):
            if name == "routed":
                continue
            assert np.array_equal(ga.cpu().numpy(), getattr(st, name)), (t, name)
        if t == 0:
            assert int(st.n_miss[0]) == 0 and (st.map_cold[ids.reshape(-1)] >= 0).any()
        else:
            assert int(st.n_miss[0]) == 10
        assert not torch.isnan(oa).any()
        assert torch.equal(oa.view(torch.int16), ob.view(torch.int16)), f"step {t}"
        pick = np.sort(rng.choice(M, 96, replace=False))
        ref = oracle_layer(x[pick], ids[pick], tw[pick], pool)
        err = ogemm.rel_err(oa.float().cpu().numpy()[pick], ref)
        assert err <= TOL, f"step {t}: rel err {err:.3e}"


def test_layer_prefill_threshold(pkg, pool):
    """The layer switches to the prefill kernels at PREFILL_ROWS_PER_EXPERT routed rows per
    expert (the measured crossover), counted on max_tokens x top_k: with 128 experts the
    last decode size is 76 tokens (760 rows < 768) and 77 tokens (770 rows) is the first
    prefill one; an explicit prefill_rows overrides it both ways."""
    moe = pkg.moe
    full = pkg.ExpertWeights(pool["w13"], pool["w13s"], pool["w2"], pool["w2s"])
    hot = list(range(S))
    slots = pkg.ExpertWeights(*[t[:S].to(DEV) for t in full.tensors()])   # slot i = expert i
    assert moe.PREFILL_ROWS_PER_EXPERT * E == 768
    mk = lambda M, **kw: pkg.LruMoELayer(full, hot, None, M, TOPK, DEV, slots=slots, **kw)
    assert not mk(76).prefill
    assert mk(77).prefill
    assert mk(20, prefill_rows=200).prefill and not mk(20, prefill_rows=201).prefill
    assert not mk(2048, prefill_rows=1 << 30).prefill


def test_layer_prefill_graph_replay(pkg, pool):
    """A prefill-sized step (256 tokens, 2560 routed rows: the tiled kernels, gate_up with the
    activation in its epilogue) captured once as a HIP graph with the overlapped gather and
    replayed with new routing -- alternately wide (read-through) and narrow (10 experts to
    install) -- equals an eager layer without the overlap, bit for bit, output and state."""
    M, steps = 256, 5
    _, perm0 = trace.zipf_trace(seed=610, E=E, rows=20, k=TOPK, steps=1, s=1.1)
    hot, rank = trace.warm_hot(perm0, S)
    full = pkg.ExpertWeights(pool["w13"], pool["w13s"], pool["w2"], pool["w2s"])
    a = pkg.LruMoELayer(full, hot, rank, M, TOPK, DEV)
    b = pkg.LruMoELayer(full, hot, rank, M, TOPK, DEV)
    assert a.prefill and a.fuse_act
    rng = np.random.default_rng(610)
    hs = set(int(e) for e in hot)
    cold = [e for e in range(E) if e not in hs]
    ids_all = []
    for t in range(steps):
        if t % 2:
            pool_ids = np.array(sorted(rng.choice(sorted(hs), 20, replace=False).tolist()
                                       + rng.choice(cold, 10, replace=False).tolist()), np.int32)
        else:
            pool_ids = np.arange(E, dtype=np.int32)
        ids_all.append(np.stack([rng.choice(pool_ids, TOPK, replace=False)
                                 for _ in range(M)]).astype(np.int32))
    xs = [torch.from_numpy(fp8.bf16_round(rng.standard_normal((M, H)).astype(np.float32)))
          .to(torch.bfloat16).to(DEV) for _ in range(steps)]
    tws = [torch.from_numpy(rng.random((M, TOPK)).astype(np.float32)).to(DEV)
           for _ in range(steps)]
    x_st, tw_st = torch.empty_like(xs[0]), torch.empty_like(tws[0])
    ids_st = torch.empty((M, TOPK), dtype=torch.int32, device=DEV)
    out_a = torch.empty((M, H), dtype=torch.bfloat16, device=DEV)
    out_b = torch.empty_like(out_a)
    side = torch.cuda.Stream()
    gpu_case("prefill graph: eager step 0")
    ids0 = torch.from_numpy(ids_all[0]).to(DEV)
    a.apply(out_a, xs[0], tws[0], ids0, gather=True, side=side, overlap=True)
    b.apply(out_b, xs[0], tws[0], ids0, gather=True, side=side, overlap=False)
    torch.cuda.synchronize()
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        a.apply(out_a, x_st, tw_st, ids_st, gather=True, side=side, overlap=True)
    torch.cuda.synchronize()
    installs = 0
    for t in range(1, steps):
        gpu_case(f"prefill graph: replay step {t}")
        ids = torch.from_numpy(ids_all[t]).to(DEV)
        x_st.copy_(xs[t])
        tw_st.copy_(tws[t])
        ids_st.copy_(ids)
        g.replay()
        b.apply(out_b, xs[t], tws[t], ids, gather=True, side=side, overlap=False)
        torch.cuda.synchronize()
        installs += int(a.cache.n_miss.item())
        assert not torch.isnan(out_a).any()
        assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16)), f"replay {t}"
        for name, ga, gb in zip(olru.LruState.NAMES, a.cache.state(), b.cache.state()):
            assert torch.equal(ga, gb), (t, name)
        out_a.zero_()                       # eager work between replays
        torch.cuda.synchronize()
    assert installs > 0, "the narrow steps must install experts"
    del g
