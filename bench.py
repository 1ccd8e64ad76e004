#!/usr/bin/env python3
"""MoE decode step on one MI355X: device LRU cache + align + fp8 grouped expert GEMMs.

Workload (the 52-layer decode step): 52 MoE layers, E=512 experts of hidden 2560 /
intermediate 768 (w13 [1536, 2560], w2 [2560, 768], fp8 e4m3 with 128x128 float32 block scales,
weights ~N(0, 0.02) before quantization), S=257 HBM slots per layer warm-started from the
hottest experts of each layer's routing, top-10 routing of B=4 streams x 5 rows (MTP-4) = 20
tokens per step from a seeded Zipf(1.1) trace per layer (seed 1000 + layer, rows correlated so a
layer sees 5-13 misses per step). Per layer and step: r4d_lru_fused (manager + both aligns),
group-128 activation quant, gate_up GEMM (hot slots + cold tensor) with the SiLU-mul in its
epilogue, down GEMM with routed weights (quantizing the activation per workgroup, as
silu_mul_quant does), moe_sum -- captured once as a HIP graph and replayed with new routing.

`value` is ms per 52-layer step with every input resident in HBM: the miss gather, which reads
pinned host memory over PCIe, is timed in a second graph and reported as
`e2e_with_gather_ms_per_step` (the gather overlapped with the GEMMs of the rows already
resident; `e2e_no_overlap_ms_per_step` is the same steps with the gather in front of every
GEMM); the same step at B=1 (5 tokens) is `b1_ms_per_step`, with the gather
`b1_e2e_with_gather_ms_per_step`. The
static hot/cold arm (inserts disabled: the warm-start set stays resident and every other
routed expert is read over PCIe by the GEMMs, every step) is `e2e_static_arm_ms_per_step`.
`pcie_mb_per_step` counts the host-link bytes of both arms (experts inserted + distinct routed
experts left cold, from the device state after each step) on this trace and on routing drawn
from the reference's hot profile (`profile_trace`: tests/golden/hot_profile.json);
`pcie_drift` counts them over 400 steps of the drifting Zipf traces (the caches alone).
`step_frac` is the grouped GEMMs' algorithmic bytes of a step over `ms_per_step`, as a fraction
of 8 TB/s. `lru_fused_us_per_layer` is the fused LRU kernel (manager + both aligns) alone, the
52 layers' calls replayed as one graph (`lru_fused_eager_us_per_layer`: the same calls
launched eagerly). `prefill_4096` times the prefill kernels on a 4096-token chunk; `cpu_baseline` the
layer step in torch fp32 on the host cores.

    python bench.py [--steps K] [--warmup W] [--only-b4 | --only-b1]
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import platform
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
PKG_NAME = "r9700_lru_expert_cache_amd"

METRIC = "MoE decode ms/step (LRU+align+grouped GEMM) B=1/4; % HBM roofline"
E, S, H, I, TOPK, LAYERS = 512, 257, 2560, 768, 10, 52
EXPERT_BYTES = 2 * I * H + H * I + (2 * I // 128) * (H // 128) * 4 + (H // 128) * (I // 128) * 4
HBM_PEAK_GBS = 8000.0
PCIE_STEPS = 10                 # steps replayed one at a time to count host-link traffic


def load_pkg():
    import importlib.util
    if PKG_NAME in sys.modules:
        return sys.modules[PKG_NAME]
    d = ROOT / "r9700-lru-expert-cache_amd"
    spec = importlib.util.spec_from_file_location(PKG_NAME, d / "__init__.py",
                                                  submodule_search_locations=[str(d)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[PKG_NAME] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---- workload ---------------------------------------------------------------------------------
def make_pool(torch, dev, ops):
    """512 experts, fp8 + block scales, quantized on the GPU (chunks of 32 experts) and stored
    in the fragment order the GEMMs read."""
    def quant(w):
        n, k = w.shape[-2], w.shape[-1]
        b = w.reshape(w.shape[0], n // 128, 128, k // 128, 128)
        ws = (b.abs().amax(dim=(2, 4)).clamp(min=1e-12) / 448.0).float()
        wq = (b / ws[:, :, None, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
        return wq.reshape(w.shape), ws
    g = torch.Generator(device=dev).manual_seed(2)
    out = {}
    for name, (n, k) in (("w13", (2 * I, H)), ("w2", (H, I))):
        wq = torch.empty((E, n, k), dtype=torch.float8_e4m3fn, device=dev)
        ws = torch.empty((E, n // 128, k // 128), dtype=torch.float32, device=dev)
        for e0 in range(0, E, 32):
            q, s = quant(torch.randn(32, n, k, device=dev, generator=g) * 0.02)
            ops.shuffle_fp8_weight(q.contiguous(), out=wq[e0:e0 + 32])
            ws[e0:e0 + 32] = s
        out[name], out[name + "s"] = wq, ws
    return out


def layer_trace(layer, rows, steps, corr=None):
    """The layer's Zipf(1.1) routing; rows correlated at 20 rows by default (corr 0.7: 5-13
    misses per layer per step, about 47 distinct experts), uncorrelated with corr=0 (about 97
    distinct at 20 rows)."""
    trace = load_pkg().traces
    if corr is None:
        corr = 0.7 if rows >= 20 else 0.0
    return trace.zipf_trace(seed=1000 + layer, E=E, rows=rows, k=TOPK, steps=steps, s=1.1,
                            corr=corr)


def build(torch, pkg, rows, steps, dev, pool_dev, host_full, layers_cache=None,
          max_inserts=None, corr=None):
    """Layers (slots shared between batch sizes: the hot set depends only on the layer seed)."""
    trace = pkg.traces
    ids = np.empty((steps, LAYERS, rows, TOPK), np.int32)
    layers = []
    for l in range(LAYERS):
        tr, perm0 = layer_trace(l, rows, steps, corr)
        ids[:, l] = tr.reshape(steps, rows, TOPK)
        hot, rank = trace.warm_hot(perm0, S)
        if layers_cache is not None and l < len(layers_cache):
            slots = layers_cache[l].slots
            if pool_dev is not None:          # refill the shared buffers with this hot set
                idx = torch.tensor(sorted(hot.tolist()), dtype=torch.int64, device=dev)
                for dst, n in zip(slots.tensors(), ("w13", "w13s", "w2", "w2s")):
                    torch.index_select(pool_dev[n], 0, idx, out=dst)
        else:
            idx = torch.tensor(sorted(hot.tolist()), dtype=torch.int64, device=dev)
            slots = pkg.ExpertWeights(*[pool_dev[n].index_select(0, idx).contiguous()
                                        for n in ("w13", "w13s", "w2", "w2s")])
        layers.append(pkg.LruMoELayer(host_full, hot, rank, rows, TOPK, dev, slots=slots,
                                      max_inserts=max_inserts))
    return layers, ids


def capture(torch, layers, ids_static, tw, hbuf, gather, side, overlap=None):
    def step():
        for l, layer in enumerate(layers):
            layer.apply(hbuf[l + 1], hbuf[l], tw, ids_static[l], gather=gather, side=side,
                        overlap=overlap)
    # one eager step first (loads every kernel), then the cache state is put back
    snap = snapshot(torch, layers)
    step()
    torch.cuda.synchronize()
    restore(layers, snap)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    return g


def snapshot(torch, layers):
    return [[t.clone() for t in L.cache.state()] for L in layers]


def restore(layers, snap):
    for L, s in zip(layers, snap):
        for t, v in zip(L.cache.state(), s):
            t.copy_(v)


def run_steps(torch, g, ids_dev, ids_static, t0, k):
    for t in range(t0, t0 + k):
        ids_static.copy_(ids_dev[t])
        g.replay()


def time_steps(torch, g, ids_dev, ids_static, t0, k):
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    a.record()
    run_steps(torch, g, ids_dev, ids_static, t0, k)
    b.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    return a.elapsed_time(b) / k, wall


def distinct_per_layer(ids_step):
    """distinct experts routed per layer for one step [LAYERS, rows, TOPK]."""
    return np.array([len(np.unique(ids_step[l])) for l in range(ids_step.shape[0])])


def algorithmic_bytes(ids_last, rows, fused=False):
    """Bytes one grouped-GEMM launch must move, averaged over the 104 launches of a step: every
    distinct expert's weights and block scales once, the activations and their scales once,
    the output rows once (and the routed weights for the down projection). fused: gate_up
    writes the bf16 activation [mtk, I] and down reads it (in place of gate_up's [mtk, 2I]
    output and the e4m3 q2 with its scales)."""
    mtk = rows * TOPK
    total = 0.0
    d = distinct_per_layer(ids_last)
    for l in range(len(d)):
        e = int(d[l])
        total += (e * (2 * I * H + (2 * I // 128) * (H // 128) * 4)
                  + rows * H + rows * (H // 128) * 4
                  + (mtk * I * 2 if fused else mtk * 2 * I * 2))                 # gate_up
        total += (e * (H * I + (H // 128) * (I // 128) * 4)
                  + (mtk * I * 2 if fused else mtk * I + mtk * (I // 128) * 4)
                  + mtk * H * 2 + mtk * 4)                                      # down
    return total / (2 * len(d)), d


def gemm_launches(layers):
    """Both grouped GEMMs of every layer as the layer step runs them (gate_up with its
    activation and down from it, or the plain pair), eager, on the current stream (inputs as
    the last step left them)."""
    for L in layers:
        if L.fuse_dec:
            L._gate_up_act()
            L._down(L.tw)
            continue
        L._gemm_split(L.ic1, L.qx, L.xs, L.slots.w13, L.slots.s13, 0, None, L.top_k, L.npw1,
                      L.sk1)
        L._gemm_split(L.ic3, L.q2, L.s2, L.slots.w2, L.slots.s2, 2, L.tw, 1, L.npw2, L.sk2)


def load_traffic():
    """HBM bytes per grouped-GEMM launch from the committed counter runs (FETCH_SIZE and
    WRITE_SIZE of `bench.py --pmc-probe`, each scaled by the same counter on a plain copy of
    known size), or None when the file is absent."""
    p = ROOT / "profiles" / "moe_gemm_traffic_b4.json"
    if not p.exists():
        return None
    return json.loads(p.read_text())


def gemm_roofline(torch, pkg, layers, ids_last, rows, reps=3):
    """Average duration of the grouped GEMM launches of one step (both GEMMs of all 52 layers,
    back to back, captured once into a HIP graph so that the host's per-call cost does not pace
    the shorter ones; HIP events around each replay on the replaying stream) and the
    algorithmic bytes each launch moves."""
    fused = layers[0].fuse_dec
    per_launch_bytes, d = algorithmic_bytes(ids_last, rows, fused)
    n = 2 * len(layers)
    gemm_launches(layers)                       # eager once (loads every kernel)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gemm_launches(layers)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    best = 1e30
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        torch.cuda.synchronize()
        best = min(best, a.elapsed_time(b) * 1e3 / n)
    del g
    gbs = per_launch_bytes / (best * 1e-6) / 1e9
    tr = load_traffic()
    return dict(bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                frac=round(gbs / HBM_PEAK_GBS, 4),
                traffic=None if tr is None else tr["hbm_bytes_per_launch"],
                traffic_source=None if tr is None else tr["source"],
                kernel=(f"rlu::moe_gemm_k (gate_up npw {layers[0].npw1} sk {layers[0].sk1}"
                        + (" with the SiLU-mul epilogue" if fused else "")
                        + (", down in 8-wave workgroups, 2 strips per wave, quantizing the "
                           "activation per workgroup" if fused else
                           f", down npw {layers[0].npw2} sk {layers[0].sk2}")
                        + "; hot + cold in one launch)"),
                avg_launch_us=round(best, 2), algorithmic_bytes_per_launch=int(per_launch_bytes),
                distinct_experts_per_layer=round(float(d.mean()), 1))


def lru_us_per_layer(torch, layers, ids_dev, ids_static, t, reps=5):
    """The fused LRU kernel alone for all 52 layers, each call from the same state (restored
    between repetitions, outside the timed region): (eager launches, one graph replay of the
    52 launches) in µs per layer. The graph figure is the one comparable with the reference's
    in-graph manager timing."""
    snap = snapshot(torch, layers)
    ids_static.copy_(ids_dev[t])
    def go():
        for l, L in enumerate(layers):
            L.cache.fused(ids_static[l], out=L.align)
    go()
    torch.cuda.synchronize()
    restore(layers, snap)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        go()
    torch.cuda.synchronize()
    best = {"eager": 1e30, "graph": 1e30}
    for _ in range(reps):
        for kind, fn in (("eager", go), ("graph", g.replay)):
            restore(layers, snap)
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            best[kind] = min(best[kind], a.elapsed_time(b) * 1e3 / len(layers))
    restore(layers, snap)
    del g
    return best["eager"], best["graph"]


def lm_head_fp8(torch, pkg, dev, M=5, reps=20):
    """The fp8 target lm_head GEMV: vocab 151936 x 2560 e4m3 in fragment order with 128x128
    block scales (N(0, 0.02) weights, seed 5), x bf16 N(0, 1) [M, 2560] (seed 4), already
    quantized per token group 128. Two weight copies alternate so that no launch finds its
    389 MB in the 256 MB last-level cache. Bytes per launch: weights + scales + activations +
    logits."""
    N, K = 151936, 2560
    ops = pkg.ops
    g = torch.Generator(device=dev).manual_seed(5)
    W = []
    for _ in range(2):
        w = torch.randn(N, K, device=dev, generator=g) * 0.02
        W.append(ops.pack_fp8_block(w))
        del w
    torch.cuda.empty_cache()
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(dev)
    qx, xs = ops.fp8_quant_group(x)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    nbytes = N * K + (N // 128) * (K // 128) * 4 + M * K + M * (K // 128) * 4 + M * N * 2
    for i in range(2):
        ops.gemm_fp8_block_q(qx, xs, *W[i], out=y)
    torch.cuda.synchronize()
    best = 1e30
    for _ in range(3):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(reps):
            ops.gemm_fp8_block_q(qx, xs, *W[i % 2], out=y)
        b.record()
        torch.cuda.synchronize()
        best = min(best, a.elapsed_time(b) * 1e3 / reps)
    gbs = nbytes / (best * 1e-6) / 1e9
    del W
    torch.cuda.empty_cache()
    return dict(M=M, us=round(best, 2), bytes=nbytes, achieved_gbs=round(gbs, 1),
                frac=round(gbs / HBM_PEAK_GBS, 4))


def lm_head_w4(torch, pkg, dev, Ms=(1, 4, 8), reps=20):
    """The W4 draft lm_head GEMV: vocab 151936 x 2560, int4 group-128 codes with bf16 scale and
    integer zero (N(0, 0.02) weights, seed 5, packed with the clip search), x bf16 [M, 2560].
    Two packed copies alternate (207 MB each, past the 256 MB last-level cache between
    launches). Bytes per launch: codes + scale/zero words + activations + logits."""
    N, K = 151936, 2560
    w4 = pkg.w4
    g = torch.Generator(device=dev).manual_seed(5)
    P = []
    for _ in range(2):
        w = torch.randn(N, K, device=dev, generator=g) * 0.02
        P.append(w4.pack_w4a16(w))
        del w
    torch.cuda.empty_cache()
    out = {}
    for M in Ms:
        x = torch.randn(M, K, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(dev)
        y = torch.empty((M, P[0].n_pad), dtype=torch.bfloat16, device=dev)
        nbytes = P[0].nbytes + M * K * 2 + M * N * 2
        # every M starts from the same power state: back to back, this kernel slows by up to
        # a fifth after a few ms (its dequant work draws enough power to lower the clocks)
        torch.cuda.synchronize()
        time.sleep(0.25)
        for i in range(2):
            w4.gemm_w4a16(x, P[i], out=y)
        torch.cuda.synchronize()
        best = 1e30
        for _ in range(3):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for i in range(reps):
                w4.gemm_w4a16(x, P[i % 2], out=y)
            b.record()
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b) * 1e3 / reps)
        gbs = nbytes / (best * 1e-6) / 1e9
        out[f"M{M}"] = dict(us=round(best, 2), bytes=nbytes, achieved_gbs=round(gbs, 1),
                            frac=round(gbs / HBM_PEAK_GBS, 4))
    del P
    torch.cuda.empty_cache()
    return out


def _fp8_bytes(torch, shape, dev, g):
    """Random e4m3 bytes of magnitude code < 100, never a NaN pattern (0x7f / 0xff)."""
    t = torch.randint(-100, 100, shape, device=dev, generator=g, dtype=torch.int8)
    t[t == -1] = 0
    return t.view(torch.float8_e4m3fn)


def prefill_gemm(torch, pkg, dev, T=4096, reps=3, lru=True, wv=0):
    """The grouped GEMMs in the MFMA regime: a 4096-token prefill chunk, top-10 uniform over
    the 512 experts (seed 0), all experts HBM-resident (w13 / w2 fp8, fragment order), through
    the fused LRU + align (read-through: 512 distinct > 128) and the prefill kernels (wv = 0:
    the streamed kernel at these shapes). Reports each GEMM's time, its dense TFLOP/s (2 mk N K)
    and its weight bytes / time; gate_up with SiLU-mul-quant in its epilogue (what the layer
    runs) beside gate_up followed by the separate SiLU-mul-quant. The align's tile list is
    built once (tile_list_us) and read by every GEMM, as the layer does."""
    ops = pkg.ops
    g = torch.Generator(device=dev).manual_seed(7)
    w13 = _fp8_bytes(torch, (E, 2 * I, H), dev, g)
    w2 = _fp8_bytes(torch, (E, H, I), dev, g)
    w13s = torch.rand(E, 2 * I // 128, H // 128, device=dev, generator=g) * 1e-3
    w2s = torch.rand(E, H // 128, I // 128, device=dev, generator=g) * 1e-3
    rng = np.random.default_rng(0)
    ids = np.stack([rng.choice(E, TOPK, replace=False) for _ in range(T)]).astype(np.int32)
    cache = pkg.LruCache.build(E, range(E), None, dev)
    al = cache.alloc_align(ids.size)
    (sh, eh, nh), _ = cache.fused(torch.from_numpy(ids).to(dev), out=al)
    mtk = ids.size
    x = _fp8_bytes(torch, (T, H), dev, g)
    xs = torch.rand(T, H // 128, device=dev, generator=g)
    x2 = _fp8_bytes(torch, (mtk, I), dev, g)
    s2 = torch.rand(mtk, I // 128, device=dev, generator=g)
    tw = torch.rand(mtk, device=dev, generator=g)
    y1 = torch.empty(mtk, 2 * I, dtype=torch.bfloat16, device=dev)
    y2 = torch.empty(mtk, H, dtype=torch.bfloat16, device=dev)
    tiles = torch.empty(2 * eh.numel() + 1, dtype=torch.int32, device=dev)

    def timed(fn):
        # each timed call starts from an idle GPU: these kernels draw enough power that a few
        # ms of them back to back lower the clocks, which spreads repeated timings by 10-20%.
        # A short spin kernel ahead of the start event keeps the GPU busy while the host
        # enqueues the timed launches, so the events bracket GPU work only (not the Python
        # call's own latency)
        fn()
        torch.cuda.synchronize()
        best = 1e30
        for _ in range(reps):
            time.sleep(0.1)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda._sleep(200_000)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b) * 1e3)
        return best
    # the align's tile list, built once and read by both GEMMs (as the layer does)
    u_tiles = timed(lambda: ops.moe_gemm_tiles(eh, nh, tiles))
    u1 = timed(lambda: ops.moe_gemm_tiled(y1, x, xs, w13, w13s, sh, eh, nh, None, mtk, TOPK,
                                          tiles=tiles, wv=wv, tiles_ready=True))
    u2 = timed(lambda: ops.moe_gemm_tiled(y2, x2, s2, w2, w2s, sh, eh, nh, tw, mtk, 1,
                                          tiles=tiles, wv=wv, tiles_ready=True))
    q2 = torch.empty(mtk, I, dtype=ops.FP8, device=dev)
    sq2 = torch.empty(mtk, I // 128, dtype=torch.float32, device=dev)
    u_act = timed(lambda: ops.silu_mul_quant(y1, out=(q2, sq2)))
    u_fused = None
    if wv == 0 and ops.moe_gemm_tiled_silu_quant_built(H, 2 * I):
        u_fused = timed(lambda: ops.moe_gemm_tiled_silu_quant(q2, sq2, x, xs, w13, w13s, sh, eh,
                                                              nh, mtk, TOPK, tiles=tiles,
                                                              tiles_ready=True))
    # the fused LRU + both aligns (+ the group-128 quant of the chunk's hidden states, as the
    # layer calls it) over the chunk's 40960 (token, k) ids
    ids_d = torch.from_numpy(ids).to(dev).reshape(-1)
    hs = torch.randn(T, H, device=dev, generator=g).to(torch.bfloat16)
    qx = torch.empty(T, H, dtype=torch.uint8, device=dev)
    qs = torch.empty(T, H // 128, dtype=torch.float32, device=dev)
    def timed_avg(fn, n=50):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / n
    res = {}
    if lru:
        res["lru_align_us"] = round(timed_avg(lambda: cache.fused(ids_d, out=al)), 1)
        res["lru_align_quant_us"] = round(timed_avg(lambda: cache.fused_quant(ids_d, al, hs, qx,
                                                                              qs)), 1)
    for name, us, n, k in (("gate_up", u1, 2 * I, H), ("down", u2, H, I)):
        res[name] = dict(us=round(us, 1), tflops=round(2.0 * mtk * n * k / us / 1e6, 1),
                         weight_gbs=round(E * n * k / us / 1e3, 1))
    res["gate_up_plus_down_us"] = round(u1 + u2, 1)
    res["tile_list_us"] = round(u_tiles, 1)
    res["silu_mul_quant_us"] = round(u_act, 1)
    if u_fused is not None:
        res["gate_up_silu_quant_fused_us"] = round(u_fused, 1)
        res["layer_gemms_us"] = round(u_fused + u2, 1)
    wbytes = E * (2 * I * H + H * I)
    res["weight_bytes"] = wbytes
    res["weights_frac_of_hbm_peak"] = round(wbytes / ((u1 + u2) * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
    res["kernel"] = "streamed prefill kernel" if wv == 0 else f"tiled_k, {wv} workgroups/CU"
    res["tokens"], res["rows_per_expert"] = T, round(mtk / E, 1)
    res["tiles"] = int(tiles[-1].item())
    if lru:
        # the whole layer step on this chunk: every expert resident (the slots are the weight
        # tensors themselves), apply() without a gather. Uniform routing over 512 experts is a
        # read-through step (512 distinct > 256), so repeated steps leave the cache as it is.
        full = pkg.ExpertWeights(w13, w13s, w2, w2s)
        layer = pkg.LruMoELayer(full, range(E), None, T, TOPK, dev, slots=full)
        ids_t = torch.from_numpy(ids).to(dev)
        twl = torch.rand(T, TOPK, device=dev, generator=g)
        out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
        res["layer_step_us"] = round(timed(lambda: layer.apply(out, hs, twl, ids_t,
                                                                 gather=False)), 1)
        res["layer_step"] = ("LruMoELayer.apply on the chunk: fused LRU + align + quant, gate_up "
                             "with SiLU-mul-quant, down, moe_sum")
        del layer
        # the same chunk through a layer of 257 slots (the decode workload's cache size): 257
        # experts' rows come from the slots, the other 255 experts' from the full tensor, and
        # each GEMM covers both aligns in one launch
        layer = pkg.LruMoELayer(full, range(257), None, T, TOPK, dev)
        res["layer_step_257_slots_us"] = round(timed(lambda: layer.apply(out, hs, twl, ids_t,
                                                                           gather=False)), 1)
        del layer
    del w13, w2
    torch.cuda.empty_cache()
    return res


def prefill_crossover(torch, pkg, dev, tokens=(64, 128, 256, 512, 640, 768, 896, 1024),
                      reps=5):
    """Where the layer should switch from the decode grouped GEMM to the prefill kernels: the
    whole layer step (LruMoELayer.apply: fused LRU + align + quant, both GEMMs, moe_sum; every
    expert resident, no gather) at each token count, once with the decode kernel
    (prefill_rows past the chunk) and once with the prefill kernels (prefill_rows 0), on the
    same routing: top-10 uniform over the 512 experts, and top-10 Zipf(1.1) (rows drawn
    independently; hot experts then take several 16-row blocks). Each step is captured as a HIP graph
    (as the decode bench runs it, so the host's per-launch cost is out of the figure) and each
    figure is the best of `reps` replays, each started from an idle GPU.
    -> {routing: {tokens: {"rows", "decode_us", "prefill_us"}}}, and the layer's own
    threshold (moe.PREFILL_ROWS_PER_EXPERT x E)."""
    g = torch.Generator(device=dev).manual_seed(17)
    w13 = _fp8_bytes(torch, (E, 2 * I, H), dev, g)
    w2 = _fp8_bytes(torch, (E, H, I), dev, g)
    w13s = torch.rand(E, 2 * I // 128, H // 128, device=dev, generator=g) * 1e-3
    w2s = torch.rand(E, H // 128, I // 128, device=dev, generator=g) * 1e-3
    full = pkg.ExpertWeights(w13, w13s, w2, w2s)

    def best_of(fn):
        fn()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            fn()
        best = 1e30
        for _ in range(reps):
            time.sleep(0.05)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda._sleep(200_000)
            a.record()
            gr.replay()
            b.record()
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b) * 1e3)
        del gr
        return best

    out = {"uniform": {}, "zipf": {}}
    for routing, T in ((r, T) for r in out for T in tokens):
        if routing == "uniform":
            rng = np.random.default_rng(1000 + T)
            ids = np.stack([rng.choice(E, TOPK, replace=False)
                            for _ in range(T)]).astype(np.int32)
        else:
            ids = pkg.traces.zipf_trace(seed=2000 + T, E=E, rows=T, k=TOPK, steps=1,
                                        s=1.1)[0].reshape(T, TOPK)
        ids_t = torch.from_numpy(ids).to(dev)
        hs = torch.randn(T, H, device=dev, generator=g).to(torch.bfloat16)
        tw = torch.rand(T, TOPK, device=dev, generator=g)
        row = {"rows": T * TOPK}
        ys = {}
        for name, pr in (("decode", 1 << 30), ("prefill", 0)):
            layer = pkg.LruMoELayer(full, range(E), None, T, TOPK, dev, slots=full,
                                    prefill_rows=pr)
            y = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
            row[f"{name}_us"] = round(best_of(lambda: layer.apply(y, hs, tw, ids_t,
                                                                  gather=False)), 1)
            ys[name] = y
            del layer
        # the two paths' GEMMs agree bit for bit at sk 1; the decode layer splits gate_up's K
        # over two waves above 8 tokens, so the outputs are compared loosely here (the layer
        # tests pin both paths)
        d = (ys["decode"].float() - ys["prefill"].float()).abs().max().item()
        row["max_abs_diff"] = round(d, 4)
        row["blocks"] = int(sum(-(-c // 16) for c in np.bincount(ids.reshape(-1), minlength=E)))
        out[routing][str(T)] = row
        log(f"crossover {routing} {T} tokens ({T * TOPK} rows, {row['blocks']} blocks): decode "
            f"{row['decode_us']} us, prefill {row['prefill_us']} us")
    del w13, w2, full
    torch.cuda.empty_cache()
    return {"layer_step_us": out, "prefill_rows": pkg.moe.PREFILL_ROWS_PER_EXPERT * E,
            "setup": "512 experts, all resident, no gather; blocks = 16-row blocks of the "
                     "decode kernel"}


def lru_insert_sweep(torch, pkg, dev, reps=50, rounds=5):
    """r4d_lru_fused time vs inserts per step at E=512, S=257 (the insert storm of
    tests/lru/bench_victim.py:43-79): routing with exactly k non-resident experts among mk ids,
    no read-through. Each graph replays (restore state, fused call) reps times; the restore
    alone is timed the same way and subtracted."""
    out = {}
    for mk in (50, 200):
        row = {}
        for k in (0, 1, 2, 4, 8, 13, 14, 32, 64):
            if k > mk - 10:                 # keep some resident experts in the step
                continue
            rng = np.random.default_rng(100 + k)
            hot = np.sort(rng.choice(E, S, replace=False))
            rank = {int(e): i for i, e in enumerate(rng.permutation(hot))}
            cache = pkg.LruCache.build(E, hot, rank, dev)
            cache.max_distinct = E
            ids = torch.from_numpy(pkg.traces.insert_storm_ids(rng, hot, E, mk, k)).to(dev)
            align = cache.alloc_align(mk)
            pristine = [t.clone() for t in cache.state()]

            def restore():
                for t, v in zip(cache.state(), pristine):
                    t.copy_(v)

            def full():
                restore()
                cache.fused(ids, out=align)
            times = {}
            for name, fn in (("full", full), ("restore", restore)):
                side = torch.cuda.Stream()
                side.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(side):
                    fn()
                torch.cuda.current_stream().wait_stream(side)
                torch.cuda.synchronize()
                gr = torch.cuda.CUDAGraph()
                with torch.cuda.graph(gr):
                    for _ in range(reps):
                        fn()
                gr.replay()
                torch.cuda.synchronize()
                best = 1e30
                for _ in range(rounds):
                    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    a.record()
                    gr.replay()
                    b.record()
                    torch.cuda.synchronize()
                    best = min(best, a.elapsed_time(b) * 1e3 / reps)
                times[name] = best
                if name == "full":          # the state the last fused call left
                    nm = int(cache.n_miss.item())
                    assert nm == min(k, 64), (mk, k, nm)
            row[str(k)] = round(times["full"] - times["restore"], 2)
        out[f"mk{mk}"] = row
    return out


def down_sum_probe(torch, pkg, dev, calls=20, M=5):
    """The B=1 folded down + moe_sum kernel from the activation (rlu_moe_down_sum_act) at the
    decode shape, for the counter runs: w2 e4m3 [512, 2560, 768] with 128x128 block scales, 257
    of the experts resident in slots, M tokens of top-10 (each token's ten experts distinct,
    half of them resident), `calls` calls."""
    g = torch.Generator(device=dev).manual_seed(11)
    w2 = _fp8_bytes(torch, (E, H, I), dev, g)
    s2 = torch.rand((E, H // 128, I // 128), device=dev, generator=g) * 1e-3 + 1e-4
    hot = torch.randperm(E, device=dev, generator=g)[:S].sort().values
    table = torch.full((E,), -1, dtype=torch.int32, device=dev)
    table[hot] = torch.arange(S, dtype=torch.int32, device=dev)
    w_hot, s_hot = w2[hot].contiguous(), s2[hot].contiguous()
    ids = torch.stack([torch.randperm(E, device=dev, generator=g)[:TOPK] for _ in range(M)])
    ids = ids.to(torch.int32).contiguous()
    tw = torch.rand((M, TOPK), device=dev, generator=g)
    act = torch.randn((M * TOPK, I), device=dev, generator=g).to(torch.bfloat16)
    out = torch.empty((M, H), dtype=torch.bfloat16, device=dev)
    for _ in range(calls):
        pkg.ops.moe_down_sum_act(act, ids, tw, table, w_hot, s_hot, w2, s2, out)
    torch.cuda.synchronize()
    del w2, w_hot


def counter_probe(torch, pkg, dev, calls=50):
    """The workload of the LDS and MFMA counter runs: the fused LRU kernel in the insert storm
    (E=512, S=257, mk 200 with no read-through; `calls` calls with 0 inserts, then `calls` with
    64, each from the same pristine state, restored by copies between the calls), then the
    prefill grouped GEMMs (gate_up, down, SiLU-mul-quant and the fused gate_up, 4 launches
    each), then the B=1 folded down + moe_sum (20 calls), then the 256 MiB calibration copy."""
    for k in (0, 64):
        rng = np.random.default_rng(100 + k)
        hot = np.sort(rng.choice(E, S, replace=False))
        rank = {int(e): i for i, e in enumerate(rng.permutation(hot))}
        cache = pkg.LruCache.build(E, hot, rank, dev)
        cache.max_distinct = E
        ids = torch.from_numpy(pkg.traces.insert_storm_ids(rng, hot, E, 200, k)).to(dev)
        align = cache.alloc_align(200)
        pristine = [t.clone() for t in cache.state()]
        for _ in range(calls):
            for t, v in zip(cache.state(), pristine):
                t.copy_(v)
            cache.fused(ids, out=align)
        torch.cuda.synchronize()
        assert int(cache.n_miss.item()) == k
    res = prefill_gemm(torch, pkg, dev, reps=3, lru=False)
    down_sum_probe(torch, pkg, dev)
    # the calibration kernel of known size for FETCH_SIZE / WRITE_SIZE: a 256 MiB device copy,
    # the run's last copy dispatch
    a = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
    c = torch.empty_like(a)
    torch.cuda.synchronize()
    c.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"counter_probe": f"lru_k: {calls} calls at 0 inserts, then {calls} at 64 "
                                       "(mk 200); then the prefill kernels (4096 tokens): "
                                       "gate_up, down, SiLU-mul-quant, fused gate_up x4 each; "
                                       "then the B=1 folded down + moe_sum from the activation "
                                       "x20; then one 256 MiB device-to-device copy",
                      "copy_bytes": 256 << 20, "prefill": res}), flush=True)


# ---- host-link traffic and the hot-profile routing ----------------------------------------------
def pcie_per_step(torch, layers, g, ids_dev, ids_static, t0, k):
    """Replays k steps of graph g one at a time and reads every layer's cache state after each:
    bytes over the host link per step = experts inserted (the miss gather copies each one's
    four buffers) + distinct routed experts left cold (read-through or over the insert cap:
    the GEMMs read their weights from pinned host memory), both x the per-expert bytes.
    -> (MB per step, inserted experts per layer per step, cold experts per layer per step)."""
    per = layers[0].full.per_expert_bytes()
    mb, ins, cold = [], [], []
    for t in range(t0, t0 + k):
        ids_static.copy_(ids_dev[t])
        g.replay()
        torch.cuda.synchronize()
        n_in = n_cold = 0
        for l, L in enumerate(layers):
            n_in += int(L.cache.n_miss.item())
            il = ids_static[l].reshape(-1).long()
            n_cold += int(torch.unique(il[L.cache.map_cold[il] >= 0]).numel())
        mb.append((n_in + n_cold) * per / 1e6)
        ins.append(n_in / len(layers))
        cold.append(n_cold / len(layers))
    return (round(float(np.mean(mb)), 1), round(float(np.mean(ins)), 2),
            round(float(np.mean(cold)), 2))


def pcie_drift(torch, pkg, dev, rows=20, steps=400, window=50):
    """Host-link traffic as the routing drifts: the 52 layers' caches alone (no GEMMs; the
    fused LRU kernel decides inserts and cold experts exactly as in the layer step), LRU and
    static arms from the same warm start, over `steps` steps of the layer traces (Zipf(1.1),
    26 of the 512 permutation positions re-shuffled every 8 steps). Bytes per step as in
    pcie_per_step, averaged over the first and the last `window` steps.
    -> {arm: {"mb_first", "mb_last", "cold_first", "cold_last", "ins_first", "ins_last"}}."""
    trace = pkg.traces
    ids = np.empty((steps, LAYERS, rows * TOPK), np.int32)
    warm = []
    for l in range(LAYERS):
        tr, perm0 = layer_trace(l, rows, steps)
        ids[:, l] = tr.reshape(steps, rows * TOPK)
        warm.append(trace.warm_hot(perm0, S))
    ids_dev = torch.from_numpy(ids).to(dev)
    out = {}
    for arm, mi in (("lru", None), ("static", 0)):
        caches = []
        for hot, rank in warm:
            c = (pkg.LruCache.build(E, hot, rank, dev) if mi is None else
                 pkg.LruCache.build(E, hot, rank, dev, max_inserts=mi))
            caches.append((c, c.alloc_align(rows * TOPK)))
        seen = torch.zeros(LAYERS, E, dtype=torch.int32, device=dev)
        ins, cold = [], []
        for t in range(steps):
            seen.zero_()
            n_in = []
            for l, (c, al) in enumerate(caches):
                il = ids_dev[t, l].long()
                c.fused(ids_dev[t, l], out=al)
                n_in.append(c.n_miss[0])
                # distinct routed experts left cold after this step's manager
                seen[l].index_fill_(0, il[c.map_cold[il] >= 0], 1)
            ins.append(float(torch.stack(n_in).sum().item()) / LAYERS)
            cold.append(float(seen.sum().item()) / LAYERS)
        mb = [(a + b) * LAYERS * EXPERT_BYTES / 1e6 for a, b in zip(ins, cold)]
        first, last = slice(0, window), slice(steps - window, steps)
        out[arm] = {"mb_first": round(float(np.mean(mb[first])), 1),
                    "mb_last": round(float(np.mean(mb[last])), 1),
                    "ins_first": round(float(np.mean(ins[first])), 2),
                    "ins_last": round(float(np.mean(ins[last])), 2),
                    "cold_first": round(float(np.mean(cold[first])), 2),
                    "cold_last": round(float(np.mean(cold[last])), 2)}
        del caches
    out["steps"], out["window"] = steps, window
    out["routing"] = ("the headline's layer traces (seed 1000 + layer, rows correlated), "
                      f"{steps} steps; per-layer means over the first and last {window}")
    return out


def b1_leg(torch, pkg, dev, pool, host_full, layers4, hb4, side, g, args):
    """The B=1 (5 tokens) HBM-resident 52-layer step on the B=4 layers' slot buffers, refilled
    with the B=1 warm-start sets (fresh caches): the step's ms and its GEMM roofline."""
    rows1 = 5
    layers1, ids1 = build(torch, pkg, rows1, args.warmup + 3 * args.steps + 2, dev, pool,
                          host_full, layers_cache=layers4)
    tw1 = torch.softmax(torch.randn(rows1, TOPK, generator=g), -1).to(dev)
    hb1 = torch.empty((LAYERS + 1, rows1, H), dtype=torch.bfloat16, device=dev)
    hb1[0] = hb4[0, :rows1]
    ids1_dev = torch.from_numpy(ids1).to(dev)
    ids1_static = torch.empty_like(ids1_dev[0])
    ids1_static.copy_(ids1_dev[0])
    g1 = capture(torch, layers1, ids1_static, tw1, hb1, gather=False, side=side)
    run_steps(torch, g1, ids1_dev, ids1_static, 0, args.warmup)
    ms1, _ = time_steps(torch, g1, ids1_dev, ids1_static, args.warmup, args.steps)
    log(f"B=1 HBM-resident step: {ms1:.3f} ms")
    r1 = gemm_roofline(torch, pkg, layers1, ids1[args.warmup + args.steps - 1], rows1)
    roof = {k: r1[k] for k in ("bound", "achieved", "peak", "unit", "frac", "kernel",
                               "avg_launch_us", "algorithmic_bytes_per_launch",
                               "distinct_experts_per_layer")}
    log(f"B=1 grouped GEMM: {roof['achieved']} GB/s, frac {roof['frac']}")
    del g1
    return {"b1_ms_per_step": round(ms1, 4), "b1_roofline": roof,
            "state": (layers1, ids1, tw1, hb1, ids1_dev, ids1_static)}


def refill_slots(torch, pkg, layers):
    """Every live slot <- the bytes of the expert its cache state names, copied from the pinned
    pool by the library's own gather kernel with a miss list of every (expert, slot) pair. For
    caches that were advanced without their gathers, and after capture(), whose eager step
    gathers into slots and then puts the cache state back."""
    for L in layers:
        se = L.cache.slot_expert
        live = torch.nonzero(se >= 0).flatten()
        miss = torch.stack([se[live], live.to(torch.int32)], 1).contiguous()
        n = torch.full((1,), miss.shape[0], dtype=torch.int32, device=se.device)
        pairs = [(L.slots.w13, L.full.w13, L.full_ptrs[0]), (L.slots.w2, L.full.w2, L.full_ptrs[2]),
                 (L.slots.s13, L.full.s13, L.full_ptrs[1]), (L.slots.s2, L.full.s2, L.full_ptrs[3])]
        pairs += pairs[2:]
        pkg._r4d_lru_gather([d for d, _, _ in pairs], [s_ for _, s_, _ in pairs], miss, n,
                            pkg.lru.LRU_CHUNKS, pkg.lru.LRU_LANES,
                            src_ptrs=[p_ for _, _, p_ in pairs])
    torch.cuda.synchronize()


def drift_e2e(torch, pkg, dev, host_full, slot_bufs, tw, hb, side, rows=20, steps=400,
              window=50):
    """The cache's benefit in time: the whole 52-layer step with the miss gather (overlapped)
    over the last `window` steps of the 400-step drifting traces, LRU against the static arm.
    Each arm's caches start from the layers' warm sets and are advanced through the first
    steps - window steps of routing by the fused LRU kernel alone (the state those steps
    leave is what matters; their gathers would only move bytes that later steps evict), then
    every slot is refilled with its expert's bytes over the host link, and the last `window`
    steps replay the captured step graph: gather, GEMMs over slots and over pinned host memory,
    moe_sum. -> {arm: ms per step}, plus the window's host-link bytes per step."""
    trace = pkg.traces
    ids = np.empty((steps, LAYERS, rows, TOPK), np.int32)
    warm = []
    for l in range(LAYERS):
        tr, perm0 = layer_trace(l, rows, steps)
        ids[:, l] = tr.reshape(steps, rows, TOPK)
        warm.append(trace.warm_hot(perm0, S))
    ids_dev = torch.from_numpy(ids).to(dev)
    ids_static = torch.empty_like(ids_dev[0])
    t0 = steps - window
    out = {}
    for arm, mi in (("lru", None), ("static", 0)):
        layers = build_from(torch, pkg, rows, warm, dev, None, host_full, slot_bufs,
                            max_inserts=mi)
        for t in range(t0):
            for l, L in enumerate(layers):
                L.cache.fused(ids_dev[t, l], out=L.align)
        torch.cuda.synchronize()
        ids_static.copy_(ids_dev[t0])
        g = capture(torch, layers, ids_static, tw, hb, gather=True, side=side)
        refill_slots(torch, pkg, layers)
        ms, _ = time_steps(torch, g, ids_dev, ids_static, t0, window - PCIE_STEPS)
        pc = pcie_per_step(torch, layers, g, ids_dev, ids_static, steps - PCIE_STEPS,
                           PCIE_STEPS)
        out[arm] = {"e2e_with_gather_ms_per_step": round(ms, 3), "pcie_mb_per_step": pc[0],
                    "inserted_per_layer": pc[1], "cold_per_layer": pc[2]}
        log(f"drifted end, {arm} arm: {ms:.3f} ms/step, {pc[0]} MB/step over PCIe")
        del g, layers
        torch.cuda.synchronize()
    out["steps"], out["timed"] = steps, f"steps {t0}..{steps - PCIE_STEPS - 1} timed, " \
        f"{steps - PCIE_STEPS}..{steps - 1} replayed one at a time to count host-link bytes"
    return out


def profile_routing(pkg, rows, steps):
    """Routing that follows the reference's hot profile (tests/golden/hot_profile.json: 48 MoE
    layers of routing counts from real decode and prefill traffic): layer l of the 52 draws
    from profile layer l % 48 (traces.profile_trace, seed 2000 + l), and its warm start is that
    profile layer's S top-ranked experts, stamped by profile rank.
    -> (ids [steps, 52, rows, top_k], [(hot ids, rank)] per layer)."""
    prof = pkg.hot_profile.load(ROOT / "tests" / "golden" / "hot_profile.json")
    keys = sorted(prof.layers)
    ids = np.empty((steps, LAYERS, rows, TOPK), np.int32)
    warm = []
    for l in range(LAYERS):
        pl = keys[l % len(keys)]
        ranked, counts = prof.layers[pl]
        ids[:, l] = pkg.traces.profile_trace(ranked, counts, E, seed=2000 + l, rows=rows, k=TOPK,
                                             steps=steps).reshape(steps, rows, TOPK)
        warm.append((np.sort(ranked[:S]), prof.rank(pl)))
    return ids, warm


def build_from(torch, pkg, rows, warm, dev, pool_dev, host_full, slot_bufs, max_inserts=None):
    """Layers warm-started from explicit (hot, rank) sets; the slot buffers of slot_bufs are
    reused and refilled with the hot experts' bytes from the device pool."""
    layers = []
    for l, (hot, rank) in enumerate(warm):
        sl = slot_bufs[l]
        if pool_dev is not None:
            idx = torch.from_numpy(np.asarray(hot, np.int64)).to(dev)
            for dst, n in zip(sl.tensors(), ("w13", "w13s", "w2", "w2s")):
                torch.index_select(pool_dev[n], 0, idx, out=dst)
        layers.append(pkg.LruMoELayer(host_full, hot, rank, rows, TOPK, dev, slots=sl,
                                      max_inserts=max_inserts))
    return layers


# ---- CPU baseline: one layer step in torch on the host cores -------------------------------------
def _cpu_threads() -> int:
    """Host threads for the CPU baseline: the cores this process may run on, at most 16 (a
    one-GPU box's share of its host)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def _median_ms(fn, runs=20, warm=2, setup=None):
    """Median wall time of fn over `runs` calls after `warm` untimed ones; setup() (untimed)
    runs before every call."""
    for _ in range(warm):
        if setup:
            setup()
        fn()
    ts = []
    for _ in range(runs):
        if setup:
            setup()
        a = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - a)
    return 1e3 * float(np.median(ts))


def cpu_baseline(torch, pool_cpu_w13, pool_cpu_w2, ids, budget_s=10.0, runs=20):
    """The layer step of the B=4 workload on the host: the LRU manager + both aligns (the
    vectorized numpy restatement and the serial C one, oracle/lru_oracle.c; the step counts the
    faster), the miss gather as
    an index copy of the inserted experts' bytes, and the compute in torch fp32 on the CPU --
    group-128 quant, gate_up over each routed expert's rows, SiLU-mul-quant, down with routed
    weights, moe_sum -- with each routed expert's weights dequantized to fp32 once, outside
    the timed pieces. Every piece: 2 warm-up calls, then the median of `runs`. Layers are
    sampled in order until the time budget is spent (at least 2); the step is the mean
    per-layer sum x 52. The two lm_head GEMVs: torch fp32 on a 2048-row slice of the 151936
    vocab rows (dequantized outside the timing), scaled by rows."""
    from oracle import clru, fp8, lru as olru
    threads = _cpu_threads()
    torch.set_num_threads(threads)
    rows = ids.shape[2]
    mtk = rows * TOPK
    rng = np.random.default_rng(1)
    x = torch.from_numpy(fp8.bf16_round(rng.standard_normal((rows, H)).astype(np.float32)))
    tw = torch.from_numpy(rng.random(mtk).astype(np.float32))
    trace = load_pkg().traces
    e4m3 = torch.float8_e4m3fn

    def quant(a, group=128):                       # group-128 e4m3 quant, fp32 in
        r, k = a.shape
        g_ = a.reshape(r, k // group, group)
        s_ = (g_.abs().amax(-1) / 448.0).clamp(min=1.0 / (448.0 * 512.0))
        q = (g_ / s_[..., None]).clamp(-448.0, 448.0).to(e4m3)
        return q.reshape(r, k), s_

    def deq(q, s_, group=128):
        r, k = q.shape
        return (q.to(torch.float32).reshape(r, k // group, group) * s_[..., None]).reshape(r, k)

    def dequant_expert(pair):                      # fragment-order e4m3 + block scales -> fp32
        wq, ws = pair
        w = torch.from_numpy(fp8.unshuffle_weight(np.ascontiguousarray(wq))).view(e4m3)
        n, k = w.shape
        b = w.to(torch.float32).reshape(n // 128, 128, k // 128, 128)
        return (b * torch.from_numpy(np.ascontiguousarray(ws))[:, None, :, None]).reshape(n, k)

    pieces = {k: [] for k in ("lru_fused_align_vectorized", "lru_fused_align_serial_c",
                              "gather_index_copy", "group_quant", "gate_up", "silu_mul_quant",
                              "down", "moe_sum")}
    t0 = time.perf_counter()
    done = 0
    slots_w13 = torch.empty((S,) + tuple(pool_cpu_w13.wq.shape[1:]), dtype=torch.uint8)
    slots_w2 = torch.empty((S,) + tuple(pool_cpu_w2.wq.shape[1:]), dtype=torch.uint8)
    src_w13 = torch.from_numpy(pool_cpu_w13.wq)
    src_w2 = torch.from_numpy(pool_cpu_w2.wq)
    while done < LAYERS and (done < 2 or time.perf_counter() - t0 < budget_s):
        l = done
        _, perm0 = layer_trace(l, rows, 1)
        hot, rank = trace.warm_hot(perm0, S)
        st0 = olru.warm_start(E, S, hot, rank)
        ids_l = ids[0, l].reshape(-1)
        box = {}

        def fresh():
            box["st"] = st0.copy()
        pieces["lru_fused_align_vectorized"].append(
            _median_ms(lambda: olru.fused(box["st"], ids_l, 16), runs, setup=fresh))
        pieces["lru_fused_align_serial_c"].append(
            _median_ms(lambda: clru.fused(box["st"], ids_l, 16), runs, setup=fresh))
        fresh()
        al = olru.fused(box["st"], ids_l, 16)
        st = box["st"]
        miss = st.miss[:int(st.n_miss[0])]
        me = torch.from_numpy(miss[:, 0].astype(np.int64))
        ms_ = torch.from_numpy(miss[:, 1].astype(np.int64))

        def gather():
            slots_w13.index_copy_(0, ms_, src_w13.index_select(0, me))
            slots_w2.index_copy_(0, ms_, src_w2.index_select(0, me))
        pieces["gather_index_copy"].append(_median_ms(gather, runs))
        # expert -> its rows, from the align output (every routed expert, hot or cold)
        used = np.unique(ids_l)
        W13 = {int(e): dequant_expert(pool_cpu_w13[e]) for e in used}
        W2 = {int(e): dequant_expert(pool_cpu_w2[e]) for e in used}
        rows_of = {int(e): torch.from_numpy(np.nonzero(ids_l == e)[0].astype(np.int64))
                   for e in used}
        box2 = {}
        pieces["group_quant"].append(_median_ms(lambda: box2.update(qx=quant(x)), runs))
        qx, xs = box2["qx"]
        xd = deq(qx, xs)

        def gate_up():
            y = torch.empty((mtk, 2 * I))
            for e, r in rows_of.items():
                y[r] = xd[r // TOPK] @ W13[e].T
            box2["y1"] = y.to(torch.bfloat16).to(torch.float32)
        pieces["gate_up"].append(_median_ms(gate_up, runs))

        def act():
            y1 = box2["y1"]
            g_, u_ = y1[:, :I], y1[:, I:]
            sl = (g_ / (1.0 + torch.exp(-g_))).to(torch.bfloat16).to(torch.float32)
            a_ = (sl * u_).to(torch.bfloat16).to(torch.float32)
            box2["q2"] = quant(a_)
        pieces["silu_mul_quant"].append(_median_ms(act, runs))
        a2 = deq(*box2["q2"])

        def down():
            y = torch.empty((mtk, H))
            for e, r in rows_of.items():
                y[r] = (a2[r] @ W2[e].T) * tw[r, None]
            box2["y2"] = y.to(torch.bfloat16)
        pieces["down"].append(_median_ms(down, runs))
        pieces["moe_sum"].append(_median_ms(
            lambda: box2["y2"].to(torch.float32).reshape(rows, TOPK, H).sum(1).to(torch.bfloat16),
            runs))
        del W13, W2
        done += 1
    per_layer = {k: float(np.mean(v)) for k, v in pieces.items()}
    # the step takes the faster of the two CPU managers
    mgr = min(per_layer["lru_fused_align_vectorized"], per_layer["lru_fused_align_serial_c"])
    ms_layer = mgr + sum(v for k, v in per_layer.items() if not k.startswith("lru_"))
    # the lm_head GEMVs on a vocab slice, scaled by rows
    vocab, nsl = 151936, 2048
    gg = torch.Generator().manual_seed(5)
    whead = torch.randn(nsl, H, generator=gg) * 0.02   # fp32: the head already dequantized
    x5 = torch.randn(5, H, generator=gg)
    x1 = x5[:1]
    head_fp8 = _median_ms(lambda: x5 @ whead.T, runs) * vocab / nsl
    head_w4 = _median_ms(lambda: x1 @ whead.T, runs) * vocab / nsl
    return dict(value=round(ms_layer * LAYERS, 2), unit="ms/step", cores=threads,
                kind="port",
                sample=f"{done} of the 52 layers of one B={rows // 5} step (20 tokens), each "
                       f"piece the median of {runs} runs after 2 warm-ups; step = mean layer x "
                       f"52. Pieces: LRU manager + both aligns (vectorized numpy restatement), "
                       f"miss gather (torch index copy of the inserted experts' bytes), then "
                       f"torch fp32 on the CPU: group quant, gate_up, SiLU-mul-quant, down with "
                       f"routed weights, moe_sum, each routed expert dequantized to fp32 once "
                       f"outside the timing. The serial C manager (oracle/lru_oracle.c) is "
                       f"timed beside the vectorized one; the step sums the faster.",
                pieces_ms_per_layer={k: round(v, 4) for k, v in per_layer.items()},
                lm_head_ms={"fp8_M5": round(head_fp8, 2), "w4_M1": round(head_w4, 2),
                            "sample": f"torch fp32 GEMV over {nsl} of the {vocab} vocab rows "
                                      f"(weights already dequantized), scaled by rows"},
                torch_threads=threads, cpu=_cpu_model(), os_cpu_count=os.cpu_count())


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


class _Dict:
    """expert -> (wq, ws) numpy pair, indexed like the [E, ...] arrays the oracle expects."""
    def __init__(self, d, which):
        self.d, self.w = d, which

    def __getitem__(self, e):
        return self.d[int(e)][self.w]

    @property
    def shape(self):
        k = next(iter(self.d))
        return (E,) + self.d[k][self.w].shape


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only-b4", action="store_true",
                    help="only the B=4 HBM-resident step (the profiled command)")
    ap.add_argument("--only-b1", action="store_true",
                    help="only the B=1 HBM-resident step (its profiled command); prints the B=1 "
                         "figures instead of the bench line")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--counter-probe", action="store_true",
                    help="for LDS / MFMA counter runs: the fused LRU kernel in the insert storm "
                         "and the prefill grouped GEMMs, then exit")
    ap.add_argument("--prefill-leg", action="store_true",
                    help="only the prefill leg (4096 tokens: the GEMMs alone, then the layer "
                         "steps with every expert resident and with 257 slots); prints its "
                         "figures")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="for counter runs: one eager B=4 step of the 52 layers, their 104 "
                         "grouped-GEMM launches once more, then a 256 MiB device copy (the "
                         "calibration kernel of known size); prints what was launched")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this path runs on one GPU; --gpus must be 1 (multi-GPU "
                                   "sharding is a design here, not launched)"}))
        sys.exit(2)
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py runs on one GPU only", file=sys.stderr)
        sys.exit(2)
    sys.path.insert(0, str(ROOT))
    import torch
    pkg = load_pkg()
    pkg.lib()                                   # fail loudly without the HIP library
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.counter_probe:
        counter_probe(torch, pkg, dev)
        return
    if args.prefill_leg:
        print(json.dumps({"prefill_4096": prefill_gemm(torch, pkg, dev)}), flush=True)
        return
    t_setup = time.perf_counter()
    log("generating 512 fp8 experts")
    pool = make_pool(torch, dev, pkg.ops)
    host = {n: torch.empty(t.shape, dtype=t.dtype, pin_memory=True) for n, t in pool.items()}
    for n in pool:
        host[n].copy_(pool[n])
    host_full = pkg.ExpertWeights(host["w13"], host["w13s"], host["w2"], host["w2s"])
    T = args.warmup + 3 * args.steps + 2 + 2 * PCIE_STEPS
    rows4 = 20
    log(f"building {LAYERS} layers (B=4, {rows4} tokens)")
    layers4, ids4 = build(torch, pkg, rows4, T, dev, pool, host_full)
    # numpy views of the pinned pool (no copies) for the CPU baseline
    cpu_w13 = _Pair(host["w13"].view(torch.uint8).numpy(), host["w13s"].numpy())
    cpu_w2 = _Pair(host["w2"].view(torch.uint8).numpy(), host["w2s"].numpy())
    g = torch.Generator().manual_seed(3)
    tw4 = torch.softmax(torch.randn(rows4, TOPK, generator=g), -1).to(dev)
    hb4 = torch.empty((LAYERS + 1, rows4, H), dtype=torch.bfloat16, device=dev)
    hb4[0] = torch.randn(rows4, H, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    ids4_dev = torch.from_numpy(ids4).to(dev)
    ids4_static = torch.empty_like(ids4_dev[0])
    side = torch.cuda.Stream()
    ids4_static.copy_(ids4_dev[0])
    if args.pmc_probe:
        for l, L in enumerate(layers4):
            L.apply(hb4[l + 1], hb4[l], tw4, ids4_static[l], gather=False)
        gemm_launches(layers4)
        a = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
        c = torch.empty_like(a)
        torch.cuda.synchronize()
        c.copy_(a)
        torch.cuda.synchronize()
        per, d = algorithmic_bytes(ids4[0], rows4, layers4[0].fuse_dec)
        print(json.dumps({"pmc_probe": "52 eager layer steps, then 104 grouped-GEMM launches, "
                                       "then one 256 MiB device-to-device copy (last copy "
                                       "kernel of the run)",
                          "copy_bytes": 256 << 20, "gemm_launches": 2 * LAYERS,
                          "algorithmic_bytes_per_launch": int(per),
                          "distinct_experts_per_layer": round(float(d.mean()), 2)}), flush=True)
        return
    if args.only_b1:
        b1 = b1_leg(torch, pkg, dev, pool, host_full, layers4, hb4, side, g, args)
        print(json.dumps({"only_b1": True, "b1_ms_per_step": b1["b1_ms_per_step"],
                          "b1_roofline": b1["b1_roofline"]}), flush=True)
        return
    gB = capture(torch, layers4, ids4_static, tw4, hb4, gather=False, side=side)
    log(f"setup {time.perf_counter() - t_setup:.1f}s; warmup {args.warmup} steps")
    run_steps(torch, gB, ids4_dev, ids4_static, 0, args.warmup)
    t = args.warmup
    ms4, wall4 = time_steps(torch, gB, ids4_dev, ids4_static, t, args.steps)
    d4 = float(np.mean([distinct_per_layer(ids4[t_]).mean() for t_ in range(t, t + args.steps)]))
    t += args.steps
    log(f"B=4 HBM-resident step: {ms4:.3f} ms")
    roof = gemm_roofline(torch, pkg, layers4, ids4[t - 1], rows4)
    lru_us, lru_graph_us = lru_us_per_layer(torch, layers4, ids4_dev, ids4_static, t)
    # the whole step against the grouped GEMMs' algorithmic bytes (every distinct expert once
    # per GEMM): what fraction of HBM peak the step as a whole moves
    step_bytes = roof["algorithmic_bytes_per_launch"] * 2 * LAYERS
    out = {"metric": METRIC, "value": round(ms4, 4), "unit": "ms/step", "n_gpus": 1,
           "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms4, 4),
           "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
           "dtype": "fp8e4m3", "data": "synthetic",
           "config": {"workload": f"{LAYERS}-layer MoE decode step, B=4 (20 tokens), top-10 of "
                                  f"E=512, S=257 HBM slots/layer, w13 [1536,2560] + w2 "
                                  f"[2560,768] fp8 e4m3 128x128-block-scaled, Zipf(1.1) routing "
                                  f"with {d4:.1f} distinct experts and 5-13 misses per layer "
                                  f"per step; value = the step with every expert already in "
                                  f"HBM: the miss gather over PCIe is NOT in value (it is "
                                  f"timed separately as e2e_with_gather_ms_per_step)",
                      "layers": LAYERS, "tokens": rows4, "top_k": TOPK, "experts": E,
                      "slots": S, "hidden": H, "moe_intermediate": I,
                      "distinct_experts_per_layer": round(d4, 1)},
           "roofline": roof,
           "step_frac": round(step_bytes / (ms4 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           "step_gemm_bytes": int(step_bytes),
           "lru_fused_us_per_layer": round(lru_graph_us, 2),
           "lru_fused_eager_us_per_layer": round(lru_us, 2),
           "wall_s_timed": round(wall4, 3)}
    if not args.only_b4:
        # the gather overlapped with the resident rows' GEMMs (the default), then the same
        # steps from the same cache state with the gather in front of every GEMM
        del gB
        snap = snapshot(torch, layers4)
        t_e2e = t
        gA = capture(torch, layers4, ids4_static, tw4, hb4, gather=True, side=side)
        run_steps(torch, gA, ids4_dev, ids4_static, t, 1)
        t += 1
        mse, _ = time_steps(torch, gA, ids4_dev, ids4_static, t, args.steps)
        t += args.steps
        out["e2e_with_gather_ms_per_step"] = round(mse, 3)
        # misses per layer in the last step, from the device state
        nm = [int(L.cache.n_miss.item()) for L in layers4]
        out["misses_per_layer_last_step"] = round(float(np.mean(nm)), 2)
        log(f"B=4 with PCIe miss gather: {mse:.3f} ms")
        pz = pcie_per_step(torch, layers4, gA, ids4_dev, ids4_static, t, PCIE_STEPS)
        del gA
        torch.cuda.synchronize()
        restore(layers4, snap)
        gN = capture(torch, layers4, ids4_static, tw4, hb4, gather=True, side=side,
                     overlap=False)
        run_steps(torch, gN, ids4_dev, ids4_static, t_e2e, 1)
        msn, _ = time_steps(torch, gN, ids4_dev, ids4_static, t_e2e + 1, args.steps)
        out["e2e_no_overlap_ms_per_step"] = round(msn, 3)
        log(f"B=4 with PCIe miss gather, not overlapped: {msn:.3f} ms")
        del gN, snap
        torch.cuda.synchronize()
        # A/B control: the static hot/cold arm (inserts disabled: the warm-start set stays
        # resident, every other routed expert is read over PCIe by the GEMMs, every step)
        layersS, _ = build(torch, pkg, rows4, 1, dev, pool, host_full, layers_cache=layers4,
                           max_inserts=0)
        gS = capture(torch, layersS, ids4_static, tw4, hb4, gather=True, side=side)
        run_steps(torch, gS, ids4_dev, ids4_static, 0, 1)
        mss, _ = time_steps(torch, gS, ids4_dev, ids4_static, 1, args.steps)
        out["e2e_static_arm_ms_per_step"] = round(mss, 3)
        log(f"B=4 static hot/cold arm (no inserts): {mss:.3f} ms")
        ps = pcie_per_step(torch, layersS, gS, ids4_dev, ids4_static, 1 + args.steps,
                           PCIE_STEPS)
        out["static_arm_cold_experts_per_layer"] = ps[2]
        out["pcie_mb_per_step"] = {
            "zipf": {"lru": pz[0], "static": ps[0],
                     "lru_inserted_per_layer": pz[1], "lru_cold_per_layer": pz[2],
                     "static_cold_per_layer": ps[2]}}
        del gS, layersS
        torch.cuda.synchronize()
        # B=1: the same slot buffers, refilled with the B=1 warm-start sets; fresh caches
        rows1 = 5
        b1 = b1_leg(torch, pkg, dev, pool, host_full, layers4, hb4, side, g, args)
        layers1, ids1, tw1, hb1, ids1_dev, ids1_static = b1["state"]
        out["b1_ms_per_step"] = b1["b1_ms_per_step"]
        out["b1_roofline"] = b1["b1_roofline"]
        torch.cuda.synchronize()
        # the same B=1 steps with the miss gather (overlapped) in the graph
        t1 = args.warmup + args.steps
        g1e = capture(torch, layers1, ids1_static, tw1, hb1, gather=True, side=side)
        run_steps(torch, g1e, ids1_dev, ids1_static, t1, 1)
        ms1e, _ = time_steps(torch, g1e, ids1_dev, ids1_static, t1 + 1, args.steps)
        out["b1_e2e_with_gather_ms_per_step"] = round(ms1e, 3)
        out["b1_misses_per_layer_last_step"] = round(
            float(np.mean([int(L.cache.n_miss.item()) for L in layers1])), 2)
        log(f"B=1 with PCIe miss gather: {ms1e:.3f} ms")
        del g1e
        torch.cuda.synchronize()
        # the same steps from the same point with the gather in front of the GEMMs, where the
        # layer folds down and moe_sum into one kernel (the fold runs only without the overlap)
        refill_slots(torch, pkg, layers1)
        g1f = capture(torch, layers1, ids1_static, tw1, hb1, gather=True, side=side,
                      overlap=False)
        refill_slots(torch, pkg, layers1)
        ms1f, _ = time_steps(torch, g1f, ids1_dev, ids1_static, t1 + 1 + args.steps, args.steps)
        out["b1_e2e_no_overlap_folded_ms_per_step"] = round(ms1f, 3)
        log(f"B=1 with PCIe miss gather, not overlapped, down + moe_sum folded: {ms1f:.3f} ms")
        del g1f, layers1
        torch.cuda.synchronize()
        # B=4, HBM-resident, on the uncorrelated trace (about twice the distinct experts)
        layersU, idsU = build(torch, pkg, rows4, args.warmup + args.steps + 2, dev, pool,
                              host_full, layers_cache=layers4, corr=0.0)
        idsU_dev = torch.from_numpy(idsU).to(dev)
        idsU_static = torch.empty_like(idsU_dev[0])
        idsU_static.copy_(idsU_dev[0])
        gU = capture(torch, layersU, idsU_static, tw4, hb4, gather=False, side=side)
        run_steps(torch, gU, idsU_dev, idsU_static, 0, args.warmup)
        msU, _ = time_steps(torch, gU, idsU_dev, idsU_static, args.warmup, args.steps)
        rU = gemm_roofline(torch, pkg, layersU, idsU[args.warmup + args.steps - 1], rows4)
        stepU = rU["algorithmic_bytes_per_launch"] * 2 * LAYERS
        out["b4_uncorrelated"] = {
            "routing": "the same Zipf(1.1) layers with uncorrelated rows (corr 0)",
            "ms_per_step": round(msU, 4),
            "distinct_experts_per_layer": rU["distinct_experts_per_layer"],
            "avg_launch_us": rU["avg_launch_us"], "achieved": rU["achieved"],
            "frac": rU["frac"],
            "step_frac": round(stepU / (msU * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        log(f"B=4 uncorrelated routing: {msU:.3f} ms, {rU['distinct_experts_per_layer']} "
            f"distinct, GEMM frac {rU['frac']}")
        del gU, layersU
        torch.cuda.synchronize()
        # B=4 with routing from the reference's hot profile, LRU and static arms, gather on
        TP = args.warmup + 2 * args.steps + 2 + PCIE_STEPS
        idsP, warmP = profile_routing(pkg, rows4, TP)
        idsP_dev = torch.from_numpy(idsP).to(dev)
        idsP_static = torch.empty_like(idsP_dev[0])
        prof = {}
        for arm, mi in (("lru", None), ("static", 0)):
            layersP = build_from(torch, pkg, rows4, warmP, dev, pool, host_full,
                                 [L.slots for L in layers4], max_inserts=mi)
            idsP_static.copy_(idsP_dev[0])
            gP = capture(torch, layersP, idsP_static, tw4, hb4, gather=True, side=side)
            run_steps(torch, gP, idsP_dev, idsP_static, 0, args.warmup)
            msP, _ = time_steps(torch, gP, idsP_dev, idsP_static, args.warmup, args.steps)
            pp = pcie_per_step(torch, layersP, gP, idsP_dev, idsP_static,
                               args.warmup + args.steps, PCIE_STEPS)
            prof[arm] = (msP, pp)
            log(f"B=4 hot-profile routing, {arm} arm: {msP:.3f} ms, {pp[0]} MB/step over PCIe")
            del gP, layersP
            torch.cuda.synchronize()
        dP = float(np.mean([distinct_per_layer(idsP[t_]).mean() for t_ in range(TP)]))
        out["profile_trace"] = {
            "routing": "tests/golden/hot_profile.json (48 layers; layer l uses profile layer "
                       "l % 48), traces.profile_trace seed 2000 + l, warm start = the layer's "
                       "257 top-ranked experts stamped by rank",
            "distinct_experts_per_layer": round(dP, 1),
            "lru_e2e_with_gather_ms_per_step": round(prof["lru"][0], 3),
            "static_e2e_ms_per_step": round(prof["static"][0], 3)}
        out["pcie_mb_per_step"]["profile"] = {
            "lru": prof["lru"][1][0], "static": prof["static"][1][0],
            "lru_inserted_per_layer": prof["lru"][1][1], "lru_cold_per_layer": prof["lru"][1][2],
            "static_cold_per_layer": prof["static"][1][2]}
        out["pcie_mb_per_step"]["expert_mb"] = round(EXPERT_BYTES / 1e6, 3)
        out["pcie_mb_per_step"]["steps_counted"] = PCIE_STEPS
        del pool
        torch.cuda.empty_cache()
        out["pcie_drift"] = pcie_drift(torch, pkg, dev)
        log(f"drift: LRU {out['pcie_drift']['lru']['mb_first']} -> "
            f"{out['pcie_drift']['lru']['mb_last']} MB/step, static "
            f"{out['pcie_drift']['static']['mb_first']} -> "
            f"{out['pcie_drift']['static']['mb_last']}")
        out["drift_e2e"] = drift_e2e(torch, pkg, dev, host_full, [L.slots for L in layers4],
                                     tw4, hb4, side)
        out["lm_head_fp8"] = lm_head_fp8(torch, pkg, dev)
        log(f"fp8 lm_head M=5: {out['lm_head_fp8']['us']} us")
        out["lm_head_w4"] = lm_head_w4(torch, pkg, dev)
        log(f"W4 lm_head: {out['lm_head_w4']}")
        out["prefill_4096"] = prefill_gemm(torch, pkg, dev)
        log(f"prefill 4096 tokens: {out['prefill_4096']}")
        out["prefill_crossover"] = prefill_crossover(torch, pkg, dev)
        out["lru_insert_sweep_us"] = lru_insert_sweep(torch, pkg, dev)
        log(f"LRU insert sweep: {out['lru_insert_sweep_us']}")
        out["cpu_baseline"] = cpu_baseline(torch, cpu_w13, cpu_w2, ids4, args.cpu_seconds)
        log(f"CPU baseline: {out['cpu_baseline']['value']} ms/step")
    print(json.dumps(out), flush=True)


class _Pair:
    """expert -> (e4m3 bytes, block scales) from the [E, ...] pool arrays."""
    def __init__(self, wq, ws):
        self.wq, self.ws = wq, ws

    def __getitem__(self, e):
        return self.wq[int(e)], self.ws[int(e)]


if __name__ == "__main__":
    main()
