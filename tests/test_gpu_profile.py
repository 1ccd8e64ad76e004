"""GPU: an LRU MoE layer warm-started from the reference's hot profile (tests/golden/
hot_profile.json) -- LruMoELayer.from_profile, the hot_ids_for_layer / profile_rank_for_layer
path of r4d_mxfp4_moe.py.lru.diff:129-141 and 502-541 -- then run on a routing trace drawn
from the same layer's counts.

* the warm start equals the oracle's (oracle.lru.warm_start with the water-filled hot set and
  the profile ranks): table, map_cold, slot_expert, slot_stamp, step;
* each step's cache state equals oracle.lru.fused's bit for bit; residency holds after the
  gather; the layer output is within 2e-2 of max|ref| of the oracle pipeline.
Expert shapes are small (hidden 256, intermediate 256) so that all 512 experts of a layer fit
a quick test; the budget (1.65 GB of these 196,656-byte experts) gives each layer about the
share that 50 GB gives full-size experts.
"""
from __future__ import annotations

import pathlib

import numpy as np
import pytest

from conftest import gpu_case
from oracle import fp8, gemm as ogemm
from oracle import lru as olru

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 2e-2
E, H, I, TOPK = 512, 256, 256, 10
GOLDEN = pathlib.Path(__file__).parent / "golden" / "hot_profile.json"
BUDGET_GB = 1.65


@pytest.fixture(scope="module")
def small_pool(pkg):
    from importlib import import_module
    ops = import_module(pkg.__name__ + ".ops")
    g = torch.Generator(device=DEV).manual_seed(11)
    out = {}
    for name, (n, k) in (("w13", (2 * I, H)), ("w2", (H, I))):
        w = torch.randn(E, n, k, device=DEV, generator=g) * 0.05
        b = w.reshape(E, n // 128, 128, k // 128, 128)
        ws = (b.abs().amax(dim=(2, 4)).clamp(min=1e-12) / 448.0).float()
        wq = (b / ws[:, :, None, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn).reshape(E, n, k)
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


# 20 rows of this profile's (flat) routing exceed the read-through gate (more than S / 2
# distinct experts): no inserts, all misses run cold; 5 rows insert
@pytest.mark.parametrize("layer_idx,M,path", [(7, 20, "read-through"), (30, 5, "insert")])
def test_layer_from_profile(pkg, small_pool, layer_idx, M, path):
    hp = pkg.hot_profile
    prof = hp.load(GOLDEN)
    full = pkg.ExpertWeights(small_pool["w13"], small_pool["w13s"], small_pool["w2"],
                             small_pool["w2s"])
    assert full.per_expert_bytes() == 196_656
    hot = hp.hot_sets(prof, full.per_expert_bytes(), BUDGET_GB)[layer_idx]
    rank = prof.rank(layer_idx)
    assert 50 < len(hot) < 400
    gpu_case(f"profile layer {layer_idx}: warm start, {len(hot)} slots")
    layer = pkg.LruMoELayer.from_profile(full, prof, layer_idx, BUDGET_GB, M, TOPK, DEV)
    st = olru.warm_start(E, len(hot), hot, rank)
    for name, got in zip(olru.LruState.NAMES, layer.cache.state()):
        if name in ("routed", "miss", "n_miss"):
            continue
        assert np.array_equal(got.cpu().numpy(), getattr(st, name)), name
    ranked, counts = prof.layers[layer_idx]
    steps = 4
    tr = pkg.traces.profile_trace(ranked, counts, E, seed=layer_idx, rows=M, k=TOPK,
                                  steps=steps)
    rng = np.random.default_rng(layer_idx)
    side = torch.cuda.Stream()
    total_miss = 0
    read_through = 0
    for t in range(steps):
        ids = tr[t].reshape(M, TOPK)
        x = fp8.bf16_round(rng.standard_normal((M, H)).astype(np.float32))
        tw = rng.random((M, TOPK)).astype(np.float32)
        out = torch.empty((M, H), dtype=torch.bfloat16, device=DEV)
        gpu_case(f"profile layer {layer_idx} M={M} step {t}")
        layer.apply(out, torch.from_numpy(x).to(torch.bfloat16).to(DEV),
                    torch.from_numpy(tw).to(DEV), torch.from_numpy(ids).to(DEV),
                    gather=True, side=side)
        torch.cuda.synchronize()
        distinct = len(set(ids.reshape(-1).tolist()))
        read_through += distinct > max(1, int(len(hot) * 0.5))
        olru.fused(st, ids.reshape(-1), 16)
        for name, got in zip(olru.LruState.NAMES, layer.cache.state()):
            if name == "routed":
                continue
            assert np.array_equal(got.cpu().numpy(), getattr(st, name)), (t, name)
        total_miss += int(st.n_miss[0])
        se = st.slot_expert
        live = np.nonzero(se >= 0)[0]
        idx = torch.from_numpy(se[live].astype(np.int64))
        for name, slot_name in (("w13", "w13"), ("w13s", "s13"), ("w2", "w2"), ("w2s", "s2")):
            src = small_pool[name].index_select(0, idx)
            dst = getattr(layer.slots, slot_name)[torch.from_numpy(live).to(DEV)]
            assert torch.equal(src.view(torch.uint8).reshape(len(live), -1),
                               dst.cpu().view(torch.uint8).reshape(len(live), -1)), (t, name)
        err = ogemm.rel_err(out.float().cpu().numpy(), oracle_layer(x, ids, tw, small_pool))
        assert err <= TOL, f"step {t}: rel err {err:.3e}"
    if path == "insert":
        assert total_miss > 0, "the trace must exercise the insert path"
    else:
        assert read_through == steps and total_miss == 0
