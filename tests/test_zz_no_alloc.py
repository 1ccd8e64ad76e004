"""GPU: rlu_moe_gemm_fp8blk_tiled_noalloc -- the prefill grouped GEMM with its tile list in the
library's per-device scratch array -- called through the C-ABI, equals the existing entry points
(rlu_moe_gemm_tiles + rlu_moe_gemm_fp8blk_tiled with a caller workspace) bit for bit, on two
calls in a row, the second with a smaller input (fewer tokens, so fewer tiles than the first
call left in the scratch); gate_up without and down with routed weights; outputs poisoned
with NaN so an unwritten or stale row shows. Sizes past the scratch are refused unlaunched.
The Python wrapper passes pinned host weights by their device-visible address, and a gate_up +
down pair captured into a HIP graph reuses the scratch correctly over replays with new routing
and fewer live tokens.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import gpu_case

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda"
E, H, I, TOPK = 64, 2560, 768, 10
P = ctypes.c_void_p


def _experts(n, k, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randn(E, n, k, device=DEV, generator=g) * 0.02
    b = w.reshape(E, n // 128, 128, k // 128, 128)
    ws = (b.abs().amax(dim=(2, 4)).clamp(min=1e-12) / 448.0).float()
    wq = (b / ws[:, :, None, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    return wq.reshape(E, n, k).contiguous(), ws.contiguous()


@pytest.fixture(scope="module")
def weights(pkg):
    w13, s13 = _experts(2 * I, H, 11)
    w2, s2 = _experts(H, I, 12)
    return (pkg.ops.shuffle_fp8_weight(w13), s13, pkg.ops.shuffle_fp8_weight(w2), s2)


def _noalloc(pkg, y, a, s_, w, ws, al, tw, mtk, top_k):
    sh, eh, nh = al
    return pkg.lib().rlu_moe_gemm_fp8blk_tiled_noalloc(
        P(a.data_ptr()), P(s_.data_ptr()), P(w.data_ptr()), P(ws.data_ptr()), P(sh.data_ptr()),
        P(eh.data_ptr()), P(nh.data_ptr()), eh.numel(), P(0 if tw is None else tw.data_ptr()),
        P(y.data_ptr()), mtk, top_k, a.shape[1], y.shape[1], 0,
        P(torch.cuda.current_stream().cuda_stream))


def test_noalloc_equals_workspace_entry_two_calls(pkg, weights):
    w13, s13, w2, s2 = weights
    ops = pkg.ops
    for T in (1024, 300):                      # the second call is smaller
        rng = np.random.default_rng(T)
        ids = np.stack([rng.choice(E, TOPK, replace=False) for _ in range(T)]).astype(np.int32)
        mtk = ids.size
        cache = pkg.LruCache.build(E, range(E), None, DEV)
        al = cache.alloc_align(mtk)
        (sh, eh, nh), _ = cache.fused(torch.from_numpy(ids).to(DEV), out=al)
        g = torch.Generator(device=DEV).manual_seed(T)
        x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16)
        qx, xs = ops.fp8_quant_group(x)
        a2 = torch.randn(mtk, 2 * I, device=DEV, generator=g).to(torch.bfloat16)
        _, q2, sc2 = ops.silu_mul_quant(a2)
        tw = torch.rand(mtk, device=DEV, generator=g)
        for name, a, s_, w, ws, t_w, top_k, N in (("gate_up", qx, xs, w13, s13, None, TOPK, 2 * I),
                                                 ("down", q2, sc2, w2, s2, tw, 1, H)):
            y_ref = torch.full((mtk, N), float("nan"), dtype=torch.bfloat16, device=DEV)
            y = torch.full_like(y_ref, float("nan"))
            gpu_case(f"noalloc {name} T={T}: workspace entry")
            ops.moe_gemm_tiled(y_ref, a, s_, w, ws, sh, eh, nh, t_w, mtk, top_k)
            gpu_case(f"noalloc {name} T={T}: scratch entry")
            assert _noalloc(pkg, y, a, s_, w, ws, (sh, eh, nh), t_w, mtk, top_k) == 0
            torch.cuda.synchronize()
            assert not torch.isnan(y).any(), (name, T)
            assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16)), (name, T)


def test_noalloc_refuses_past_the_scratch(pkg, weights):
    w13, s13, _, _ = weights
    small = torch.zeros(16, dtype=torch.int32, device=DEV)
    y = torch.empty((16, 2 * I), dtype=torch.bfloat16, device=DEV)
    q = torch.zeros((16, H), dtype=torch.float8_e4m3fn, device=DEV)
    s_ = torch.ones((16, H // 128), dtype=torch.float32, device=DEV)
    f = pkg.lib().rlu_moe_gemm_fp8blk_tiled_noalloc
    st = P(torch.cuda.current_stream().cuda_stream)
    args = [P(q.data_ptr()), P(s_.data_ptr()), P(w13.data_ptr()), P(s13.data_ptr()),
            P(small.data_ptr()), P(small.data_ptr()), P(small.data_ptr())]
    assert f(*args, 8193, P(0), P(y.data_ptr()), 16, TOPK, H, 2 * I, 0, st) == -7
    assert f(*args, 0, P(0), P(y.data_ptr()), 16, TOPK, H, 2 * I, 0, st) == -1
    assert f(*args, 4, P(0), P(y.data_ptr()), 16, TOPK, H, 2 * I - 128, 0, st) == -2
    with pytest.raises(ValueError, match="scratch"):
        pkg.ops.moe_gemm_tiled_noalloc(y, q, s_, w13, s13, small, torch.zeros(
            8193, dtype=torch.int32, device=DEV), small, None, 16, TOPK)


def test_noalloc_pinned_weights_through_the_wrapper(pkg, weights):
    """ops.moe_gemm_tiled_noalloc passes the device-visible address of pinned host weights (the
    cold call's full expert tensor), as moe_gemm_tiled does: both equal bit for bit."""
    _, _, w2, s2 = weights
    ops = pkg.ops
    hw = torch.empty(w2.shape, dtype=w2.dtype, pin_memory=True)
    hw.copy_(w2)
    hs = torch.empty(s2.shape, dtype=s2.dtype, pin_memory=True)
    hs.copy_(s2)
    T = 48
    rng = np.random.default_rng(5)
    ids = np.stack([rng.choice(E, TOPK, replace=False) for _ in range(T)]).astype(np.int32)
    mtk = ids.size
    cache = pkg.LruCache.build(E, range(E), None, DEV)
    (sh, eh, nh), _ = cache.fused(torch.from_numpy(ids).to(DEV), out=cache.alloc_align(mtk))
    g = torch.Generator(device=DEV).manual_seed(6)
    _, q2, sc2 = ops.silu_mul_quant(torch.randn(mtk, 2 * I, device=DEV, generator=g)
                                    .to(torch.bfloat16))
    tw = torch.rand(mtk, device=DEV, generator=g)
    want = torch.full((mtk, H), float("nan"), dtype=torch.bfloat16, device=DEV)
    got = torch.full_like(want, float("nan"))
    gpu_case("noalloc pinned weights: workspace entry")
    ops.moe_gemm_tiled(want, q2, sc2, hw, hs, sh, eh, nh, tw, mtk, 1)
    gpu_case("noalloc pinned weights: scratch entry")
    ops.moe_gemm_tiled_noalloc(got, q2, sc2, hw, hs, sh, eh, nh, tw, mtk, 1)
    torch.cuda.synchronize()
    assert not torch.isnan(want).any()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_noalloc_pair_replayed_in_a_graph(pkg, weights):
    """What the entry is for: after one eager call (which looks up the scratch address), the
    fused align and a gate_up + down pair of no-alloc calls are captured into one HIP graph and
    replayed with new routing, some replays with fewer live tokens (the other rows' ids -1, so
    fewer blocks and tiles than the scratch last held). Eager work and synchronizations run
    between the replays; after each, both outputs equal the workspace entry run eagerly on that
    replay's align output, bit for bit (rows the align does not name stay NaN in both)."""
    w13, s13, w2, s2 = weights
    ops = pkg.ops
    T = 512
    mtk = T * TOPK
    cache = pkg.LruCache.build(E, range(E), None, DEV)
    al = cache.alloc_align(mtk)
    ids_dev = torch.empty((T, TOPK), dtype=torch.int32, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(77)
    qx, xs = ops.fp8_quant_group(torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16))
    _, q2, sc2 = ops.silu_mul_quant(torch.randn(mtk, 2 * I, device=DEV, generator=g)
                                    .to(torch.bfloat16))
    tw = torch.rand(mtk, device=DEV, generator=g)
    y1 = torch.empty((mtk, 2 * I), dtype=torch.bfloat16, device=DEV)
    y2 = torch.empty((mtk, H), dtype=torch.bfloat16, device=DEV)

    def routing(seed, live):
        rng = np.random.default_rng(seed)
        ids = np.stack([rng.choice(E, TOPK, replace=False) for _ in range(T)]).astype(np.int32)
        ids[live:] = -1
        return torch.from_numpy(ids)

    def body():
        cache.fused(ids_dev, out=al)
        ops.moe_gemm_tiled_noalloc(y1, qx, xs, w13, s13, al[0], al[1], al[2], None, mtk, TOPK)
        ops.moe_gemm_tiled_noalloc(y2, q2, sc2, w2, s2, al[0], al[1], al[2], tw, mtk, 1)

    ids_dev.copy_(routing(0, T))
    gpu_case("noalloc graph: eager first call")
    body()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    gpu_case("noalloc graph: capture")
    with torch.cuda.graph(graph):
        body()
    torch.cuda.synchronize()
    for rep, live in enumerate((T, 200, T, 37)):
        ids_dev.copy_(routing(rep + 1, live))
        y1.fill_(float("nan"))
        y2.fill_(float("nan"))
        gpu_case(f"noalloc graph: replay {rep} with {live} live tokens")
        graph.replay()
        torch.cuda.synchronize()
        r1 = torch.full_like(y1, float("nan"))
        r2 = torch.full_like(y2, float("nan"))
        ops.moe_gemm_tiled(r1, qx, xs, w13, s13, al[0], al[1], al[2], None, mtk, TOPK)
        ops.moe_gemm_tiled(r2, q2, sc2, w2, s2, al[0], al[1], al[2], tw, mtk, 1)
        torch.cuda.synchronize()
        assert not torch.isnan(r1[:live * TOPK]).any() and not torch.isnan(r2[:live * TOPK]).any()
        if live < T:
            assert torch.isnan(r2[live * TOPK:]).all()
        assert torch.equal(y1.view(torch.int16), r1.view(torch.int16)), (rep, live)
        assert torch.equal(y2.view(torch.int16), r2.view(torch.int16)), (rep, live)
