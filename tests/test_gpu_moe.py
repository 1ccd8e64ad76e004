"""GPU parity of the quant, SiLU-quant, moe_sum and fp8 GEMM kernels through the C-ABI.

* quant / SiLU-quant / moe_sum: bit-exact (activations, scales, e4m3 bytes) against the oracle,
  over the shapes and magnitude regimes of tests/k4/probe_silu_quant.py:22-53 plus the zero row;
* grouped GEMM: within 1e-2 of max|ref| (the path's fp8 tolerance is 2e-2) against the float64
  dequant reference, at the MoE layer's real expert shapes (w13 [1536, 2560], w2 [2560, 768]),
  for every tile width; the reference kernel's row contract (tests/k1/moe_ref_harness.py:282-321):
  only live rows written (output poisoned with NaN), expert -1 skips its block, num_post_pad
  read on the device; partition invariance (hot call + cold call == one call, bit-identical,
  tests/lru/test_numerics_lru.py:183-198); HIP-graph replay == eager;
* fp8 lm_head GEMM at 151936 x 2560: within tolerance and argmax equal to the fp32-dequant
  reference's;
* the fragment-order weight shuffle: bit-exact against the oracle's; the kernels read shuffled
  weights, the oracle the row-major ones, so every GEMM test also checks the layout end to end.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import check_argmax, gpu_case
from oracle import fp8, gemm as ogemm
from oracle import lru as olru

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-2


def bf16_from_np(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).to(DEV)


def np_from_bf16(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


def u8(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.uint8).cpu().numpy()


@pytest.fixture(scope="module")
def ops(pkg):
    from importlib import import_module
    return import_module(pkg.__name__ + ".ops")


# ---- quantizers ------------------------------------------------------------------------------
SILU_CASES = [(r, d, s, g) for r in (1, 10, 50, 80, 2048) for d in (320, 640, 768)
              for s in (1.0, 1e-3, 60.0) for g in (0, 128) if not (g == 128 and d % 128)]
# past the group-128 kernel's grid cap (16 workgroups per CU x 16 units): its grid-stride loop
SILU_CASES += [(12000, 768, 1.0, 128)]


@pytest.mark.parametrize("rows,d,scale_in,group", SILU_CASES)
def test_silu_mul_quant_bitexact(ops, rows, d, scale_in, group):
    rng = np.random.default_rng(rows * 7 + d)
    x = fp8.bf16_round(rng.standard_normal((rows, 2 * d)).astype(np.float32) * scale_in)
    if rows >= 10:
        x[3] = 0.0                                         # the zero row: scale floor
    act_w, q_w, s_w = fp8.silu_mul_quant(x, group)
    xt = bf16_from_np(x)
    gpu_case(f"silu_mul_quant rows={rows} d={d} group={group}")
    act, q, s = ops.silu_mul_quant(xt, write_act=True, group=group)
    torch.cuda.synchronize()
    assert np.array_equal(np_from_bf16(act), act_w)
    assert np.array_equal(s.cpu().numpy(), s_w)
    assert np.array_equal(u8(q), q_w)


@pytest.mark.parametrize("rows", [1, 5, 20, 2048])
@pytest.mark.parametrize("K", [128, 768, 2560])
@pytest.mark.parametrize("group", [0, 128])
def test_group_quant_bitexact(ops, rows, K, group):
    rng = np.random.default_rng(rows + K)
    x = fp8.bf16_round(rng.standard_normal((rows, K)).astype(np.float32) *
                       rng.choice([1e-3, 1.0, 60.0]))
    q_w, s_w = fp8.group_quant(x, group)
    gpu_case(f"group_quant rows={rows} K={K} group={group}")
    q, s = ops.fp8_quant_group(bf16_from_np(x), group)
    torch.cuda.synchronize()
    assert np.array_equal(s.cpu().numpy(), s_w)
    assert np.array_equal(u8(q), q_w)


# H 7168: 14 one-wave workgroups per row; H 8 and 64: one partly idle wave; top_k 12: the
# ten-row batch and then the tail rows one at a time; 4096 x 10 x 2560: a prefill chunk's
# moe_sum
@pytest.mark.parametrize("M,top_k,H", [(5, 10, 2560), (20, 10, 2560), (1, 1, 64), (3, 7, 1024),
                                       (7, 10, 7168), (2, 3, 8), (9, 12, 2560),
                                       (1024, 10, 2560), (4096, 10, 2560)])
def test_moe_sum_bitexact(ops, M, top_k, H):
    rng = np.random.default_rng(M * top_k)
    ic3 = fp8.bf16_round(rng.standard_normal((M * top_k, H)).astype(np.float32))
    want = ogemm.moe_sum(ic3, M, top_k)
    out = torch.empty((M, H), dtype=torch.bfloat16, device=DEV)
    gpu_case(f"moe_sum M={M} top_k={top_k} H={H}")
    ops.moe_sum(bf16_from_np(ic3).view(M, top_k, H), out)
    torch.cuda.synchronize()
    assert np.array_equal(np_from_bf16(out), want)


# ---- grouped GEMM ----------------------------------------------------------------------------
def make_experts(E, N, K, seed):
    """e4m3 weights with 128x128 block scales, quantized on the GPU by the block recipe of
    kernels/fp8_target_lmhead.py:57-64 (checked against the oracle recipe in
    test_gpu_block_quant_matches_oracle)."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randn(E, N, K, device=DEV, generator=g) * 0.02
    return block_quant_gpu(w)


def block_quant_gpu(w):
    shp = w.shape
    N, K = shp[-2], shp[-1]
    b = w.reshape(-1, N // 128, 128, K // 128, 128)
    amax = b.abs().amax(dim=(2, 4)).clamp(min=1e-12)
    ws = (amax / 448.0).float()
    wq = (b / ws[:, :, None, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    return wq.reshape(shp).contiguous(), ws.reshape(*shp[:-2], N // 128, K // 128).contiguous()


def test_gpu_block_quant_matches_oracle():
    """The GPU data generator follows the oracle's block recipe. torch's GPU division may differ
    from the IEEE quotient by an ulp, so scales agree to 1 ulp and codes to one e4m3 step in a
    few places; the recipe itself is pinned bit-exactly on the CPU (test_oracle_quant)."""
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((256, 384)) * 0.02).astype(np.float32)
    wq, ws = block_quant_gpu(torch.from_numpy(w).to(DEV))
    owq, ows = fp8.block_quant_weight(w)
    g = ws.cpu().numpy()
    assert (np.abs(g - ows) <= np.spacing(ows)).all()
    t = fp8.e4m3_table()
    diff = t[u8(wq)] != t[owq]
    assert diff.mean() < 1e-3
    step = np.abs(t[u8(wq)][diff] - t[owq][diff]) / np.maximum(np.abs(t[owq][diff]), 2 ** -9)
    assert (step <= 0.25).all()


def routing(M, top_k, E, seed):
    rng = np.random.default_rng(seed)
    return np.stack([rng.choice(E, top_k, replace=False) for _ in range(M)]).astype(np.int32)


def align_all(ids, E, hot=None, bs=16):
    """moe_align over all experts (table = identity), or a hot/cold split: `hot` maps
    expert -> slot for resident experts."""
    mk = ids.size
    L, NB = olru.align_sizes(mk, E, bs)
    if hot is None:
        table = np.arange(E, dtype=np.int32)
        return olru.align(ids.reshape(-1), E, E, table, bs, L, NB)[:3]
    table = np.full(E, -1, np.int32)
    for e, s in hot.items():
        table[e] = s
    return olru.align(ids.reshape(-1), E, len(hot), table, bs, L, NB)


def to_dev_i32(*arrs):
    return [torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(DEV) for a in arrs]


@pytest.fixture(scope="module")
def layer(ops):
    """One MoE layer at the real expert shapes, 40 experts: row-major weights for the oracle
    (w13q, w2q) and their fragment-order shuffles for the kernels (w13t, w2t)."""
    E, H, I = 40, 2560, 768
    w13q, w13s = make_experts(E, 2 * I, H, 2)
    w2q, w2s = make_experts(E, H, I, 3)
    return dict(E=E, H=H, I=I, w13q=w13q, w13s=w13s, w2q=w2q, w2s=w2s,
                w13t=ops.shuffle_fp8_weight(w13q), w2t=ops.shuffle_fp8_weight(w2q))


@pytest.mark.parametrize("shape", [(1, 16, 128), (3, 48, 384), (40, 1536, 2560)])
def test_shuffle_kernel_matches_oracle(ops, shape):
    g = torch.Generator(device=DEV).manual_seed(sum(shape))
    w = torch.randint(0, 256, shape, dtype=torch.uint8, device=DEV, generator=g)
    w = w.view(torch.float8_e4m3fn)
    gpu_case(f"shuffle {shape}")
    got = u8(ops.shuffle_fp8_weight(w))
    assert np.array_equal(got, fp8.shuffle_weight(u8(w)))
    assert np.array_equal(fp8.unshuffle_weight(got), u8(w))


def test_shuffle_return_codes(pkg):
    P = ctypes.c_void_p
    x = torch.empty(4096, dtype=torch.uint8, device=DEV)
    o = torch.empty_like(x)
    s = P(torch.cuda.current_stream().cuda_stream)
    assert pkg.lib().rlu_shuffle_fp8_weight(P(x.data_ptr()), P(o.data_ptr()), 0, 128, s) == -1
    assert pkg.lib().rlu_shuffle_fp8_weight(P(x.data_ptr()), P(o.data_ptr()), 8, 128, s) == -2
    assert pkg.lib().rlu_shuffle_fp8_weight(P(x.data_ptr()), P(o.data_ptr()), 16, 64, s) == -2


def ref_from(dev_wq, dev_ws, experts):
    """numpy copies of the weights of the experts used (the oracle reads these)."""
    wq = {e: u8(dev_wq[e]) for e in experts}
    ws = {e: dev_ws[e].cpu().numpy() for e in experts}
    return wq, ws


class _Lazy:
    def __init__(self, d):
        self.d = d

    def __getitem__(self, e):
        return self.d[e]

    @property
    def shape(self):
        k = next(iter(self.d))
        return (max(self.d) + 1,) + self.d[k].shape


def run_gemm(ops, y, qx, xs, wq, ws, align, tw, mtk, top_k, npw=4, wv=0, sk=0):
    s, e, n = align
    ops._r4d_fp8_moe_gemm_into(y, qx, xs, wq, ws, None, s, e, n, tw, mtk, top_k, wv, sk, npw)


@pytest.mark.parametrize("sk", [0, 1, 2, 4])
@pytest.mark.parametrize("npw", [1, 2, 4, 8])
@pytest.mark.parametrize("M", [1, 5, 20])
def test_moe_gemm1_vs_oracle(ops, layer, npw, M, sk):
    E, H, I = layer["E"], layer["H"], layer["I"]
    top_k = 10
    ids = routing(M, top_k, E, seed=M)
    mtk = ids.size
    al = align_all(ids, E)
    rng = np.random.default_rng(M + 100)
    x = fp8.bf16_round(rng.standard_normal((M, H)).astype(np.float32))
    qx, xs = fp8.group_quant(x, 128)
    used = sorted(set(ids.reshape(-1).tolist()))
    wq, ws = ref_from(layer["w13q"], layer["w13s"], used)
    want = ogemm.moe_gemm(qx, xs, _Lazy(wq), _Lazy(ws), *al, mtk, top_k)
    y = torch.full((mtk, 2 * I), float("nan"), dtype=torch.bfloat16, device=DEV)
    qx_t = torch.from_numpy(qx).to(DEV).view(torch.float8_e4m3fn)
    xs_t = torch.from_numpy(xs).to(DEV)
    gpu_case(f"moe gemm1 M={M} npw={npw} sk={sk}")
    run_gemm(ops, y, qx_t, xs_t, layer["w13t"], layer["w13s"], to_dev_i32(*al), None, mtk,
             top_k, npw=npw, sk=sk)
    torch.cuda.synchronize()
    got = np_from_bf16(y)
    assert not np.isnan(got).any()
    err = ogemm.rel_err(got, want)
    assert err <= TOL, f"rel err {err:.3e}"


@pytest.mark.parametrize("sk", [0, 1, 2])
@pytest.mark.parametrize("npw", [1, 4])
@pytest.mark.parametrize("M", [1, 5, 20])
def test_moe_gemm2_routed_weight_vs_oracle(ops, layer, npw, M, sk):
    E, H, I = layer["E"], layer["H"], layer["I"]
    top_k = 10
    ids = routing(M, top_k, E, seed=M + 7)
    mtk = ids.size
    al = align_all(ids, E)
    rng = np.random.default_rng(M + 200)
    a = fp8.bf16_round(rng.standard_normal((mtk, I)).astype(np.float32))
    q2, s2 = fp8.group_quant(a, 128)
    tw = rng.random(mtk).astype(np.float32)
    used = sorted(set(ids.reshape(-1).tolist()))
    wq, ws = ref_from(layer["w2q"], layer["w2s"], used)
    want = ogemm.moe_gemm(q2, s2, _Lazy(wq), _Lazy(ws), *al, mtk, 1, tw=tw)
    y = torch.full((mtk, H), float("nan"), dtype=torch.bfloat16, device=DEV)
    gpu_case(f"moe gemm2 M={M} npw={npw} sk={sk}")
    run_gemm(ops, y, torch.from_numpy(q2).to(DEV).view(torch.float8_e4m3fn),
             torch.from_numpy(s2).to(DEV), layer["w2t"], layer["w2s"], to_dev_i32(*al),
             torch.from_numpy(tw).to(DEV), mtk, 1, npw=npw, sk=sk)
    torch.cuda.synchronize()
    err = ogemm.rel_err(np_from_bf16(y), want)
    assert err <= TOL, f"rel err {err:.3e}"


@pytest.mark.parametrize("sk", [0, 1])
def test_moe_gemm_row_contract(ops, layer, sk):
    """tests/k1/moe_ref_harness.py:282-321: only live rows written; expert -1 skips its block;
    num_post_pad is honoured on the device; sk = 0 (auto split) and sk = 1."""
    E, H, I = layer["E"], layer["H"], layer["I"]
    M, top_k = 8, 10
    ids = routing(M, top_k, E, seed=11)
    mtk = ids.size
    s, e, n = align_all(ids, E)
    x = fp8.bf16_round(np.random.default_rng(1).standard_normal((M, H)).astype(np.float32))
    qx, xs = fp8.group_quant(x, 128)
    qx_t = torch.from_numpy(qx).to(DEV).view(torch.float8_e4m3fn)
    xs_t = torch.from_numpy(xs).to(DEV)

    def written(s_, e_, n_):
        y = torch.full((mtk, 2 * I), float("nan"), dtype=torch.bfloat16, device=DEV)
        run_gemm(ops, y, qx_t, xs_t, layer["w13t"], layer["w13s"], to_dev_i32(s_, e_, n_), None,
                 mtk, top_k, sk=sk)
        torch.cuda.synchronize()
        return ~torch.isnan(y).any(dim=1).cpu().numpy(), y

    gpu_case(f"moe gemm row contract sk={sk}")
    w0, y0 = written(s, e, n)
    live = np.zeros(mtk, bool)
    live[s[:n[0]][s[:n[0]] < mtk]] = True
    assert np.array_equal(w0, live)
    e2 = e.copy()
    e2[0] = -1
    w2, y2 = written(s, e2, n)
    b0 = s[:16][s[:16] < mtk]
    assert not w2[b0].any()
    others = live.copy()
    others[b0] = False
    assert torch.equal(y2[torch.from_numpy(others).to(DEV)], y0[torch.from_numpy(others).to(DEV)])
    w3, _ = written(s, e, np.array([16], np.int32))
    assert np.array_equal(np.nonzero(w3)[0], np.sort(b0))


def test_moe_gemm_partition_invariance(ops, layer):
    """hot call (slot buffers) + cold call (full tensor) into one y == one all-cold call,
    bit for bit (tests/lru/test_numerics_lru.py:183-198), output poisoned with NaN first."""
    E, H, I = layer["E"], layer["H"], layer["I"]
    M, top_k = 5, 10
    ids = routing(M, top_k, E, seed=21)
    mtk = ids.size
    hot_experts = sorted(set(ids.reshape(-1).tolist()))[::2]
    hot = {ex: i for i, ex in enumerate(hot_experts)}
    sh, eh, nh, sc, ec, nc = align_all(ids, E, hot)
    slots_q = layer["w13t"][torch.tensor(hot_experts, device=DEV)].contiguous()
    slots_s = layer["w13s"][torch.tensor(hot_experts, device=DEV)].contiguous()
    x = fp8.bf16_round(np.random.default_rng(2).standard_normal((M, H)).astype(np.float32))
    qx, xs = fp8.group_quant(x, 128)
    qx_t = torch.from_numpy(qx).to(DEV).view(torch.float8_e4m3fn)
    xs_t = torch.from_numpy(xs).to(DEV)
    y = torch.full((mtk, 2 * I), float("nan"), dtype=torch.bfloat16, device=DEV)
    gpu_case("moe gemm partition invariance")
    run_gemm(ops, y, qx_t, xs_t, slots_q, slots_s, to_dev_i32(sh, eh, nh), None, mtk, top_k)
    run_gemm(ops, y, qx_t, xs_t, layer["w13t"], layer["w13s"], to_dev_i32(sc, ec, nc), None,
             mtk, top_k)
    y1 = torch.full_like(y, float("nan"))
    run_gemm(ops, y1, qx_t, xs_t, layer["w13t"], layer["w13s"], to_dev_i32(*align_all(ids, E)),
             None, mtk, top_k)
    torch.cuda.synchronize()
    assert not torch.isnan(y).any()
    assert torch.equal(y.view(torch.int16), y1.view(torch.int16))


def test_moe_gemm_graph_replay(ops, layer):
    E, H, I = layer["E"], layer["H"], layer["I"]
    M, top_k = 5, 10
    ids = routing(M, top_k, E, seed=31)
    mtk = ids.size
    al = to_dev_i32(*align_all(ids, E))
    qx_t = torch.zeros((M, H), dtype=torch.float8_e4m3fn, device=DEV)
    xs_t = torch.ones((M, H // 128), dtype=torch.float32, device=DEV)
    y = torch.empty((mtk, 2 * I), dtype=torch.bfloat16, device=DEV)
    rng = np.random.default_rng(3)
    inputs = []
    for _ in range(3):
        x = fp8.bf16_round(rng.standard_normal((M, H)).astype(np.float32))
        q, s_ = fp8.group_quant(x, 128)
        inputs.append((torch.from_numpy(q).to(DEV).view(torch.float8_e4m3fn),
                       torch.from_numpy(s_).to(DEV)))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run_gemm(ops, y, qx_t, xs_t, layer["w13t"], layer["w13s"], al, None, mtk, top_k)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    gpu_case("moe gemm graph capture")
    with torch.cuda.graph(g):
        run_gemm(ops, y, qx_t, xs_t, layer["w13t"], layer["w13s"], al, None, mtk, top_k)
    for q, s_ in inputs:
        qx_t.copy_(q)
        xs_t.copy_(s_)
        g.replay()
        torch.cuda.synchronize()
        ye = torch.empty_like(y)
        run_gemm(ops, ye, q, s_, layer["w13t"], layer["w13s"], al, None, mtk, top_k)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ye.view(torch.int16))


def test_moe_gemm_return_codes(ops, layer):
    y = torch.empty((10, 1536), dtype=torch.bfloat16, device=DEV)
    q = torch.zeros((1, 2560), dtype=torch.float8_e4m3fn, device=DEV)
    s = torch.zeros((1, 20), dtype=torch.float32, device=DEV)
    al = to_dev_i32(np.zeros(16), np.zeros(1), np.zeros(1))
    # sk 3 does not divide K/128 = 20, sk 5 is not a supported split
    for wv, sk, npw, want in ((0, 3, 4, -4), (0, 5, 4, -4), (0, 1, 3, -6), (17, 1, 4, -5)):
        with pytest.raises(RuntimeError, match=f"rc={want}"):
            ops._r4d_fp8_moe_gemm_into(y, q, s, layer["w13t"], layer["w13s"], None, *al, None,
                                       10, 10, wv, sk, npw)


def test_entry_points_refuse_null_operands(pkg):
    """With valid sizes and NULL operands every compute entry point returns -1 before it
    launches anything (a NULL would otherwise fault on the device)."""
    P = ctypes.c_void_p
    lib = pkg.lib()
    s = P(torch.cuda.current_stream().cuda_stream)
    z = P(0)
    assert lib.rlu_quant_fp8_group(z, 4, 256, 256, 128, z, z, s) == -1
    assert lib.rlu_silu_mul_quant(z, 4, 256, 512, 128, z, z, z, s) == -1
    assert lib.rlu_moe_sum(z, 4, 10, 2560, z, s) == -1
    assert lib.r4d_gemm_moe_fp8blk_nt_b16(*([z] * 10), 16, 20, 10, 2560, 1536, 0, 0, 2, s) == -1
    assert lib.rlu_moe_gemm_split(*([z] * 14), 16, 20, 10, 2560, 1536, 0, 0, 2, s) == -1
    assert lib.rlu_gemm_fp8blk_m16(*([z] * 5), 1, 1536, 2560, 0, 2, s) == -1
    assert lib.rlu_gemm_w4_m16(z, 1, 2560, z, z, z, 1536, 0, s) == -1
    assert lib.rlu_lru_split_fresh(z, 4, z, z, 64, 257, z, z, s) == -1
    torch.cuda.synchronize()


# ---- fp8 lm_head -----------------------------------------------------------------------------
@pytest.fixture(scope="module")
def lm_head(ops):
    N, K = 151936, 2560
    g = torch.Generator(device=DEV).manual_seed(5)
    w = torch.randn(N, K, device=DEV, generator=g) * 0.02
    wq, ws = block_quant_gpu(w)
    wt, ws2 = ops.pack_fp8_block(w)
    del w
    # pack_fp8_block is the same recipe as block_quant_gpu, then the shuffle
    assert torch.equal(ws2, ws)
    assert torch.equal(wt.view(torch.uint8), ops.shuffle_fp8_weight(wq).view(torch.uint8))
    return wq, ws, wt


@pytest.mark.parametrize("M", [1, 5, 8, 16])
def test_fp8_lmhead_vs_dequant_reference(ops, lm_head, M):
    wq, ws, wt = lm_head
    N, K = wq.shape
    rng = np.random.default_rng(M + 4)
    x = fp8.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    xt = bf16_from_np(x)
    gpu_case(f"fp8 lm_head M={M}")
    y = ops.gemm_fp8_block(xt, wt, ws)
    torch.cuda.synchronize()
    qx, xs = fp8.group_quant(x, 128)
    a = torch.from_numpy(fp8.dequant_act(qx, xs)).to(DEV).double()
    wd = (wq.float() * ws.repeat_interleave(128, 0).repeat_interleave(128, 1)).double()
    ref = a @ wd.T
    del wd
    err = ((y.double() - ref).abs().max() / ref.abs().max()).item()
    assert err <= TOL, f"rel err {err:.3e}"
    check_argmax(y.float().cpu().numpy(), ref.cpu().numpy(), f"fp8 lm_head M={M}")


def test_moe_gemm_split_one_launch_equals_two_calls(pkg, ops, layer):
    """rlu_moe_gemm_split (hot slots + full tensor in one launch) == the two reference-style
    calls, bit for bit, with the full tensor in pinned host memory read over PCIe."""
    E, H, I = layer["E"], layer["H"], layer["I"]
    M, top_k = 5, 10
    ids = routing(M, top_k, E, seed=41)
    mtk = ids.size
    hot_experts = sorted(set(ids.reshape(-1).tolist()))[1::2]
    hot = {ex: i for i, ex in enumerate(hot_experts)}
    al = to_dev_i32(*align_all(ids, E, hot))
    idx = torch.tensor(hot_experts, device=DEV)
    sq, ss = layer["w13t"][idx].contiguous(), layer["w13s"][idx].contiguous()
    hq = torch.empty(layer["w13t"].shape, dtype=layer["w13t"].dtype, pin_memory=True)
    hs = torch.empty(layer["w13s"].shape, dtype=torch.float32, pin_memory=True)
    hq.copy_(layer["w13t"])
    hs.copy_(layer["w13s"])
    from importlib import import_module
    moe = import_module(pkg.__name__ + ".moe")
    hqp, hsp = moe.device_ptr_of_pinned(hq), moe.device_ptr_of_pinned(hs)
    x = fp8.bf16_round(np.random.default_rng(3).standard_normal((M, H)).astype(np.float32))
    qx, xs = fp8.group_quant(x, 128)
    qx_t = torch.from_numpy(qx).to(DEV).view(torch.float8_e4m3fn)
    xs_t = torch.from_numpy(xs).to(DEV)
    y2 = torch.full((mtk, 2 * I), float("nan"), dtype=torch.bfloat16, device=DEV)
    gpu_case("split gemm: two calls")
    run_gemm(ops, y2, qx_t, xs_t, sq, ss, al[0:3], None, mtk, top_k)
    run_gemm(ops, y2, qx_t, xs_t, layer["w13t"], layer["w13s"], al[3:6], None, mtk, top_k)
    y1 = torch.full_like(y2, float("nan"))
    P = ctypes.c_void_p
    gpu_case("split gemm: one launch, cold side from pinned host memory")
    rc = pkg.lib().rlu_moe_gemm_split(
        P(qx_t.data_ptr()), P(xs_t.data_ptr()), P(sq.data_ptr()), P(ss.data_ptr()),
        P(al[0].data_ptr()), P(al[1].data_ptr()), P(al[2].data_ptr()), P(hqp), P(hsp),
        P(al[3].data_ptr()), P(al[4].data_ptr()), P(al[5].data_ptr()), P(0), P(y1.data_ptr()),
        al[0].numel(), mtk, top_k, H, 2 * I, 0, 0, 4,
        P(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    torch.cuda.synchronize()
    assert not torch.isnan(y1).any()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))


# ---- gate_up with its activation, down from the activation (decode) -------------------------
@pytest.mark.parametrize("M,sk,pinned,holes", [(1, 1, False, False), (5, 1, True, False),
                                               (20, 2, False, False), (20, 2, True, True),
                                               (20, 4, False, False), (64, 2, False, False)])
def test_moe_gemm_split_act_and_qin_equal_the_unfused_path(pkg, ops, layer, M, sk, pinned,
                                                            holes):
    """gate_up with SiLU-mul in its epilogue (rlu_moe_gemm_split_act) equals the split gate_up
    GEMM followed by silu_mul_quant's activation, and the down GEMM that quantizes that
    activation per workgroup (rlu_moe_gemm_split_qin) equals the split down GEMM on
    silu_mul_quant's q2 / s2, bit for bit: hot slots + cold full tensor (device or pinned host
    memory), and with holes (every other hot block's expert id set to -1, as the gather
    overlap's resident bucket has them) then the hot list alone over the other blocks. At 64
    tokens (640 rows over 40 experts) down has more 8-wave workgroups than a GPU holds at once."""
    E, H, I = layer["E"], layer["H"], layer["I"]
    top_k = 10
    ids = routing(M, top_k, E, seed=M + 61)
    mtk = ids.size
    hot_experts = sorted(set(ids.reshape(-1).tolist()))[::2]
    hot = {ex: i for i, ex in enumerate(hot_experts)}
    al = to_dev_i32(*align_all(ids, E, hot))
    idx = torch.tensor(hot_experts, device=DEV)
    slots = {n: layer[n][idx].contiguous() for n in ("w13t", "w13s", "w2t", "w2s")}
    full = {n: layer[n] for n in ("w13t", "w13s", "w2t", "w2s")}
    if pinned:
        for n, t in list(full.items()):
            h = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
            h.copy_(t)
            full[n] = h
    rng = np.random.default_rng(M + 62)
    x = fp8.bf16_round(rng.standard_normal((M, H)).astype(np.float32))
    qx, xs = fp8.group_quant(x, 128)
    qx_t = torch.from_numpy(qx).to(DEV).view(torch.float8_e4m3fn)
    xs_t = torch.from_numpy(xs).to(DEV)
    tw = torch.from_numpy(rng.random(mtk).astype(np.float32)).to(DEV)
    hot_al, cold_al = al[0:3], al[3:6]
    passes = [(hot_al, True)]
    if holes:                      # two hot passes over complementary block sets
        e = hot_al[1].clone()
        e_odd = e.clone()
        e_odd[1::2] = -1
        e_even = e.clone()
        e_even[0::2] = -1
        passes = [((hot_al[0], e_odd, hot_al[2]), True), ((hot_al[0], e_even, hot_al[2]), False)]
    # the unfused path
    ic1 = torch.full((mtk, 2 * I), float("nan"), dtype=torch.bfloat16, device=DEV)
    ic3 = torch.full((mtk, H), float("nan"), dtype=torch.bfloat16, device=DEV)
    P = ctypes.c_void_p
    st = P(torch.cuda.current_stream().cuda_stream)
    def split(y, a, a_s, w, ws, wc, wsc, alh, cold, t, tk, npw, sk_):
        if not cold:               # the hot list alone: the single-set GEMM
            run_gemm(ops, y, a, a_s, w, ws, alh, t, mtk, tk, npw=npw, sk=sk_)
            return
        rc = pkg.lib().rlu_moe_gemm_split(
            P(a.data_ptr()), P(a_s.data_ptr()), P(w.data_ptr()), P(ws.data_ptr()),
            P(alh[0].data_ptr()), P(alh[1].data_ptr()), P(alh[2].data_ptr()),
            P(pkg._lib.device_ptr(wc)), P(pkg._lib.device_ptr(wsc)),
            P(cold_al[0].data_ptr()), P(cold_al[1].data_ptr()), P(cold_al[2].data_ptr()),
            P(0 if t is None else t.data_ptr()), P(y.data_ptr()), alh[0].numel(), mtk, tk,
            a.shape[1], w.shape[1], 0, sk_, npw, st)
        assert rc == 0
    gpu_case(f"split act/qin M={M} sk={sk} pinned={pinned} holes={holes}: unfused")
    for alh, cold in passes:
        split(ic1, qx_t, xs_t, slots["w13t"], slots["w13s"], full["w13t"], full["w13s"], alh,
              cold, None, top_k, 2, sk)
    act_ref, q2, s2 = ops.silu_mul_quant(ic1, write_act=True)
    for alh, cold in passes:
        split(ic3, q2, s2, slots["w2t"], slots["w2s"], full["w2t"], full["w2s"], alh, cold, tw,
              1, 4, 1)
    # the fused pair
    act = torch.full((mtk, I), float("nan"), dtype=torch.bfloat16, device=DEV)
    y = torch.full((mtk, H), float("nan"), dtype=torch.bfloat16, device=DEV)
    gpu_case(f"split act/qin M={M} sk={sk} pinned={pinned} holes={holes}: fused")
    for alh, cold in passes:
        ops.moe_gemm_split_act(act, qx_t, xs_t, slots["w13t"], slots["w13s"], alh, mtk, top_k,
                               *((full["w13t"], full["w13s"], cold_al) if cold else ()), sk=sk)
    for alh, cold in passes:
        ops.moe_gemm_split_qin(y, act, slots["w2t"], slots["w2s"], alh, tw, mtk,
                               *((full["w2t"], full["w2s"], cold_al) if cold else ()))
    torch.cuda.synchronize()
    assert not torch.isnan(act).any() and not torch.isnan(y).any()
    assert torch.equal(act.view(torch.int16), act_ref.view(torch.int16))
    assert torch.equal(y.view(torch.int16), ic3.view(torch.int16))


@pytest.mark.parametrize("I", [128, 256, 640])
def test_moe_gemm_split_act_qin_short_k(pkg, ops, I):
    """The decode pair at intermediates whose K steps do not fill the register ring (down's K =
    I: 1, 2 and 5 steps against a ring of 3, so the ring is padded with scale-0 steps): gate_up
    with its activation and down quantizing it equal the unfused split GEMMs around
    silu_mul_quant bit for bit, hot slots + cold tensor, and no output is NaN. A padded step
    once read its LDS A operand past the row's bytes."""
    E, H, M, top_k = 24, 512, 20, 10
    w13, s13 = make_experts(E, 2 * I, H, 300 + I)
    w2, s2w = make_experts(E, H, I, 400 + I)
    w13t, w2t = ops.shuffle_fp8_weight(w13), ops.shuffle_fp8_weight(w2)
    ids = routing(M, top_k, E, seed=I)
    mtk = ids.size
    hot_experts = sorted(set(ids.reshape(-1).tolist()))[::2]
    hot = {ex: i for i, ex in enumerate(hot_experts)}
    al = to_dev_i32(*align_all(ids, E, hot))
    idx = torch.tensor(hot_experts, device=DEV)
    rng = np.random.default_rng(I + 1)
    x = fp8.bf16_round(rng.standard_normal((M, H)).astype(np.float32))
    qx, xs = fp8.group_quant(x, 128)
    qx_t = torch.from_numpy(qx).to(DEV).view(torch.float8_e4m3fn)
    xs_t = torch.from_numpy(xs).to(DEV)
    tw = torch.from_numpy(rng.random(mtk).astype(np.float32)).to(DEV)
    P = ctypes.c_void_p
    st = P(torch.cuda.current_stream().cuda_stream)

    hs = [t[idx].contiguous() for t in (w13t, s13, w2t, s2w)]     # the hot slots

    def split(y, a, a_s, hw, hws, wt, ws, t, tk, npw, sk):
        rc = pkg.lib().rlu_moe_gemm_split(
            P(a.data_ptr()), P(a_s.data_ptr()), P(hw.data_ptr()), P(hws.data_ptr()),
            P(al[0].data_ptr()), P(al[1].data_ptr()), P(al[2].data_ptr()), P(wt.data_ptr()),
            P(ws.data_ptr()), P(al[3].data_ptr()), P(al[4].data_ptr()), P(al[5].data_ptr()),
            P(0 if t is None else t.data_ptr()), P(y.data_ptr()), al[0].numel(), mtk, tk,
            a.shape[1], wt.shape[1], 0, sk, npw, st)
        assert rc == 0
    gpu_case(f"short-K pair I={I}: unfused")
    ic1 = torch.full((mtk, 2 * I), float("nan"), dtype=torch.bfloat16, device=DEV)
    split(ic1, qx_t, xs_t, hs[0], hs[1], w13t, s13, None, top_k, 2, 2)
    act_ref, q2, sq2 = ops.silu_mul_quant(ic1, write_act=True)
    ic3 = torch.full((mtk, H), float("nan"), dtype=torch.bfloat16, device=DEV)
    split(ic3, q2, sq2, hs[2], hs[3], w2t, s2w, tw, 1, 4, 1)
    gpu_case(f"short-K pair I={I}: fused")
    act = torch.full((mtk, I), float("nan"), dtype=torch.bfloat16, device=DEV)
    y = torch.full((mtk, H), float("nan"), dtype=torch.bfloat16, device=DEV)
    ops.moe_gemm_split_act(act, qx_t, xs_t, hs[0], hs[1], al[0:3], mtk, top_k, w13t, s13,
                           al[3:6], sk=2)
    ops.moe_gemm_split_qin(y, act, hs[2], hs[3], al[0:3], tw, mtk, w2t, s2w, al[3:6])
    torch.cuda.synchronize()
    assert not torch.isnan(y).any() and not torch.isnan(act).any()
    assert torch.equal(act.view(torch.int16), act_ref.view(torch.int16))
    assert torch.equal(y.view(torch.int16), ic3.view(torch.int16))


def test_moe_gemm_split_act_qin_return_codes(pkg):
    """Size checks return before anything is launched (null operands included)."""
    P = ctypes.c_void_p
    st = P(torch.cuda.current_stream().cuda_stream)
    buf = torch.zeros(4096, dtype=torch.int32, device=DEV)
    b = P(buf.data_ptr())
    act = pkg.lib().rlu_moe_gemm_split_act
    qin = pkg.lib().rlu_moe_gemm_split_qin
    # N not a multiple of 256 / K not a multiple of 128 / K past 1024 / null operands
    assert act(*([b] * 7), P(0), *([P(0)] * 4), b, 16, 10, 10, 2560, 1408, 0, 0, st) == -2
    assert act(*([b] * 7), P(0), *([P(0)] * 4), b, 16, 10, 10, 2500, 1536, 0, 0, st) == -2
    assert act(*([b] * 6), P(0), P(0), *([P(0)] * 4), b, 16, 10, 10, 2560, 1536, 0, 0, st) == -1
    assert qin(*([b] * 6), P(0), *([P(0)] * 5), b, 16, 10, 1152, 2560, st) == -2
    assert qin(*([b] * 6), P(0), *([P(0)] * 5), b, 16, 10, 896, 2560, st) == -2   # K > 768
    assert qin(*([b] * 6), P(0), *([P(0)] * 5), b, 16, 10, 768, 2432, st) == -2
    assert qin(P(0), *([b] * 5), P(0), *([P(0)] * 5), b, 16, 10, 768, 2560, st) == -1
    # a cold weight tensor without its align
    assert qin(*([b] * 6), b, P(0), *([P(0)] * 4), b, 16, 10, 768, 2560, st) == -1


# ---- down + moe_sum folded (decode) ----------------------------------------------------------
@pytest.mark.parametrize("M,pinned", [(1, False), (5, False), (20, False), (20, True)])
def test_moe_down_sum_equals_split_gemm_and_moe_sum(pkg, ops, layer, M, pinned):
    """The token-major down + moe_sum equals the split down GEMM (hot slots + cold full
    tensor, sk = 1) into ic3 followed by moe_sum, bit for bit; the cold experts come from the
    full tensor in device or pinned host memory."""
    E, H, I = layer["E"], layer["H"], layer["I"]
    top_k = 10
    ids = routing(M, top_k, E, seed=M + 91)
    mtk = ids.size
    hot_experts = sorted(set(ids.reshape(-1).tolist()))[1::2]
    hot = {ex: i for i, ex in enumerate(hot_experts)}
    sh, eh, nh, sc, ec, nc = align_all(ids, E, hot)
    table = np.full(E, -1, np.int32)
    for ex, sl in hot.items():
        table[ex] = sl
    sq = layer["w2t"][torch.tensor(hot_experts, device=DEV)].contiguous()
    ss = layer["w2s"][torch.tensor(hot_experts, device=DEV)].contiguous()
    if pinned:
        fq = torch.empty(layer["w2t"].shape, dtype=layer["w2t"].dtype, pin_memory=True)
        fq.copy_(layer["w2t"])
        fs = torch.empty(layer["w2s"].shape, dtype=torch.float32, pin_memory=True)
        fs.copy_(layer["w2s"])
    else:
        fq, fs = layer["w2t"], layer["w2s"]
    rng = np.random.default_rng(M + 91)
    a = fp8.bf16_round(rng.standard_normal((mtk, I)).astype(np.float32))
    q2, s2 = fp8.group_quant(a, 128)
    q2_t = torch.from_numpy(q2).to(DEV).view(torch.float8_e4m3fn)
    s2_t = torch.from_numpy(s2).to(DEV)
    tw = torch.from_numpy(rng.random((M, top_k)).astype(np.float32)).to(DEV)
    al = to_dev_i32(sh, eh, nh, sc, ec, nc)
    from importlib import import_module
    moe = import_module(pkg.__name__ + ".moe")
    P = ctypes.c_void_p
    fqp = moe.device_ptr_of_pinned(fq) if pinned else fq.data_ptr()
    fsp = moe.device_ptr_of_pinned(fs) if pinned else fs.data_ptr()
    ic3 = torch.full((mtk, H), float("nan"), dtype=torch.bfloat16, device=DEV)
    gpu_case(f"down + moe_sum unfused M={M} pinned={pinned}")
    rc = pkg.lib().rlu_moe_gemm_split(
        P(q2_t.data_ptr()), P(s2_t.data_ptr()), P(sq.data_ptr()), P(ss.data_ptr()),
        P(al[0].data_ptr()), P(al[1].data_ptr()), P(al[2].data_ptr()), P(fqp), P(fsp),
        P(al[3].data_ptr()), P(al[4].data_ptr()), P(al[5].data_ptr()), P(tw.data_ptr()),
        P(ic3.data_ptr()), al[0].numel(), mtk, 1, I, H, 0, 1, 4,
        P(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    want = torch.empty((M, H), dtype=torch.bfloat16, device=DEV)
    ops.moe_sum(ic3.view(M, top_k, H), want)
    got = torch.full((M, H), float("nan"), dtype=torch.bfloat16, device=DEV)
    gpu_case(f"down + moe_sum folded M={M} pinned={pinned}")
    ops.moe_down_sum(q2_t, s2_t, torch.from_numpy(ids.astype(np.int32)).to(DEV), tw,
                     torch.from_numpy(table).to(DEV), sq, ss, fq, fs, got)
    torch.cuda.synchronize()
    assert not torch.isnan(ic3).any()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_moe_down_sum_return_codes(pkg):
    """Argument errors return before anything is launched."""
    P = ctypes.c_void_p
    f = pkg.lib().rlu_moe_down_sum
    x = torch.empty(1 << 16, dtype=torch.uint8, device=DEV)
    p = P(x.data_ptr())
    s = P(torch.cuda.current_stream().cuda_stream)
    assert f(p, p, p, p, p, p, p, p, p, p, 4, 10, 1024, 2560, 64, s) == -6
    assert f(p, p, p, p, p, p, p, p, p, p, 4, 8, 768, 2560, 64, s) == -6
    assert f(p, p, p, p, p, p, p, p, p, p, 4, 17, 768, 2560, 64, s) == -1
    assert f(p, p, p, p, p, p, p, p, p, p, 4, 10, 768, 2500, 64, s) == -2
    assert f(P(0), p, p, p, p, p, p, p, p, p, 4, 10, 768, 2560, 64, s) == -1
    assert f(p, p, p, p, p, P(0), p, p, p, p, 4, 10, 768, 2560, 64, s) == -1     # w_hot
    assert f(p, p, p, p, p, p, P(0), p, p, p, 4, 10, 768, 2560, 64, s) == -1     # s_hot
    assert f(p, p, p, p, p, p, p, p, p, p, 4, 10, 768, 2624, 64, s) == -2      # N % 128


@pytest.mark.parametrize("M,pinned", [(1, False), (5, False), (5, True), (8, False)])
def test_moe_down_sum_act_equals_down_sum_on_silu_quant(pkg, ops, layer, M, pinned):
    """The folded down + moe_sum from the bf16 SiLU-mul activation (each workgroup quantizes
    its token's rows) equals the folded kernel on silu_mul_quant's q2 / s2 of the same gate_up
    output, bit for bit: hot slots + cold full tensor in device or pinned host memory, with an
    all-zero token (its scales fall to the floor 1 / (448 * 512)) and one of large values."""
    E, H, I = layer["E"], layer["H"], layer["I"]
    top_k = 10
    ids = routing(M, top_k, E, seed=M + 93)
    mtk = ids.size
    hot_experts = sorted(set(ids.reshape(-1).tolist()))[::2]
    table = np.full(E, -1, np.int32)
    for sl, ex in enumerate(hot_experts):
        table[ex] = sl
    idx = torch.tensor(hot_experts, device=DEV)
    sq, ss = layer["w2t"][idx].contiguous(), layer["w2s"][idx].contiguous()
    fq, fs = layer["w2t"], layer["w2s"]
    if pinned:
        fq = torch.empty(fq.shape, dtype=fq.dtype, pin_memory=True); fq.copy_(layer["w2t"])
        fs = torch.empty(fs.shape, dtype=fs.dtype, pin_memory=True); fs.copy_(layer["w2s"])
    rng = np.random.default_rng(M + 94)
    ic1 = rng.standard_normal((mtk, 2 * I)).astype(np.float32)
    ic1[:top_k] = 0.0                                      # token 0: a zero activation
    if M > 1:
        ic1[top_k:2 * top_k] *= 300.0                      # token 1: large values
    ic1_t = torch.from_numpy(ic1).to(torch.bfloat16).to(DEV)
    act, q2, s2 = ops.silu_mul_quant(ic1_t, write_act=True)
    tw = torch.from_numpy(rng.random((M, top_k)).astype(np.float32)).to(DEV)
    ids_t = torch.from_numpy(ids.astype(np.int32)).to(DEV)
    table_t = torch.from_numpy(table).to(DEV)
    want = torch.full((M, H), float("nan"), dtype=torch.bfloat16, device=DEV)
    got = torch.full_like(want, float("nan"))
    gpu_case(f"down + moe_sum folded on q2 M={M} pinned={pinned}")
    ops.moe_down_sum(q2, s2, ids_t, tw, table_t, sq, ss, fq, fs, want)
    gpu_case(f"down + moe_sum folded on act M={M} pinned={pinned}")
    ops.moe_down_sum_act(act, ids_t, tw, table_t, sq, ss, fq, fs, got)
    torch.cuda.synchronize()
    assert not torch.isnan(want).any()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_moe_down_sum_act_return_codes(pkg):
    """Argument errors of the activation form return before anything is launched."""
    P = ctypes.c_void_p
    f = pkg.lib().rlu_moe_down_sum_act
    x = torch.empty(1 << 16, dtype=torch.uint8, device=DEV)
    p = P(x.data_ptr())
    s = P(torch.cuda.current_stream().cuda_stream)
    assert f(p, p, p, p, p, p, p, p, p, 4, 10, 1024, 2560, 64, s) == -6
    assert f(p, p, p, p, p, p, p, p, p, 4, 8, 768, 2560, 64, s) == -6
    assert f(p, p, p, p, p, p, p, p, p, 4, 17, 768, 2560, 64, s) == -1
    assert f(p, p, p, p, p, p, p, p, p, 4, 10, 768, 2500, 64, s) == -2
    assert f(P(0), p, p, p, p, p, p, p, p, 4, 10, 768, 2560, 64, s) == -1
    assert f(p, p, p, p, P(0), p, p, p, p, 4, 10, 768, 2560, 64, s) == -1        # w_hot
    assert f(p, p, p, p, p, P(0), p, p, p, 4, 10, 768, 2560, 64, s) == -1        # s_hot
    assert f(p, p, p, p, p, p, p, p, p, 4, 10, 768, 2624, 64, s) == -2         # N % 128


# ---- a tensor-parallel rank's shapes ----------------------------------------------------------
@pytest.mark.parametrize("which", ["gate_up", "down"])
def test_moe_gemm_tp2_shapes(ops, which):
    """One rank of tensor parallel 2 (intermediate 768 / 2 = 384): gate_up [768, 2560] and
    down [2560, 384] on the decode kernel (every sk it takes at that K) within 1e-2 of the
    float64 oracle, and on the prefill kernel (gate_up: the streamed kernel at N = 768; down:
    no streamed configuration at K = 384, so the general tiled kernel) bit-identical to the
    decode kernel at sk = 1. gate_up's SiLU-mul-quant epilogue (N = 768 is a multiple of 256)
    equals silu_mul_quant of that output bit for bit."""
    E, top_k = 24, 10
    N, K = (768, 2560) if which == "gate_up" else (2560, 384)
    wq, ws = make_experts(E, N, K, 11 if which == "gate_up" else 12)
    wt = ops.shuffle_fp8_weight(wq)
    for M in (5, 96):
        ids = routing(M, top_k, E, seed=M + 41)
        mtk = ids.size
        al = align_all(ids, E)
        rows = M if which == "gate_up" else mtk
        tk = top_k if which == "gate_up" else 1
        rng = np.random.default_rng(M + 41)
        x = fp8.bf16_round(rng.standard_normal((rows, K)).astype(np.float32))
        qx, xs = fp8.group_quant(x, 128)
        qx_t = torch.from_numpy(qx).to(DEV).view(torch.float8_e4m3fn)
        xs_t = torch.from_numpy(xs).to(DEV)
        tw = None if which == "gate_up" else rng.random(mtk).astype(np.float32)
        tw_t = None if tw is None else torch.from_numpy(tw).to(DEV)
        used = sorted(set(ids.reshape(-1).tolist()))
        wr, wsr = ref_from(wq, ws, used)
        want = ogemm.moe_gemm(qx, xs, _Lazy(wr), _Lazy(wsr), *al, mtk, tk, tw=tw)
        al_t = to_dev_i32(*al)
        outs = {}
        for sk in (1,) if K == 384 else (1, 2, 4):
            y = torch.full((mtk, N), float("nan"), dtype=torch.bfloat16, device=DEV)
            gpu_case(f"tp2 {which} M={M} decode sk={sk}")
            run_gemm(ops, y, qx_t, xs_t, wt, ws, al_t, tw_t, mtk, tk, npw=2, sk=sk)
            torch.cuda.synchronize()
            err = ogemm.rel_err(np_from_bf16(y), want)
            assert err <= TOL, f"{which} M={M} sk={sk}: rel err {err:.3e}"
            outs[sk] = y
        yt = torch.full((mtk, N), float("nan"), dtype=torch.bfloat16, device=DEV)
        gpu_case(f"tp2 {which} M={M} prefill kernel")
        ops.moe_gemm_tiled(yt, qx_t, xs_t, wt, ws, *al_t, tw_t, mtk, tk)
        torch.cuda.synchronize()
        assert torch.equal(yt.view(torch.int16), outs[1].view(torch.int16))
        if which == "gate_up":
            assert ops.moe_gemm_tiled_silu_quant_built(K, N)
            _, q_ref, s_ref = ops.silu_mul_quant(yt)
            q = torch.full((mtk, N // 2), 0x7F, dtype=torch.uint8, device=DEV).view(ops.FP8)
            sc = torch.full((mtk, N // 256), float("nan"), device=DEV)
            gpu_case(f"tp2 gate_up M={M} prefill kernel + silu-mul-quant")
            ops.moe_gemm_tiled_silu_quant(q, sc, qx_t, xs_t, wt, ws, *al_t, mtk, tk)
            torch.cuda.synchronize()
            assert torch.equal(q.view(torch.uint8), q_ref.view(torch.uint8))
            assert torch.equal(sc.view(torch.int32), s_ref.view(torch.int32))


# ---- the tiled (prefill) grouped GEMM ---------------------------------------------------------
def tiles_ref(eids, npad, tmb=8):
    """The tile list by walking the align output: each run of one expert's blocks cut into
    tiles of at most tmb blocks; expert -1 blocks make none."""
    nb = int(npad) // 16
    out = []
    b = 0
    while b < nb:
        e = eids[b]
        r = b
        while r < nb and eids[r] == e:
            r += 1
        if e >= 0:
            for s in range(b, r, tmb):
                out.append((s, min(tmb, r - s)))
        b = r
    return out


# 4096 x 512: more blocks than threads (three per thread); 4096 x 10 and 12000 x 12: runs of
# 256-750 blocks that cross many threads' segments and waves, the last one near the builder's
# 8192-block limit
@pytest.mark.parametrize("M,E_used", [(256, 40), (600, 40), (37, 12), (4096, 512), (4096, 10),
                                      (12000, 12)])
def test_moe_gemm_tile_list(ops, M, E_used):
    ids = routing(M, 10, E_used, seed=M)
    s, e, n = align_all(ids, E_used)
    e2 = e.copy()
    if len(e2) > 3:
        e2[2] = -1                                   # a skipped block
    tl = ops.moe_gemm_tiles(*to_dev_i32(e2, n)[0:2])
    torch.cuda.synchronize()
    got = tl.cpu().numpy()
    nt = int(got[-1])
    want = tiles_ref(e2, n[0])
    assert nt == len(want)
    assert [tuple(x) for x in got[:2 * nt].reshape(-1, 2)] == want


@pytest.mark.parametrize("wv", [0, 2])
@pytest.mark.parametrize("M", [256, 600])
def test_moe_gemm_tiled_equals_decode_kernel(ops, layer, M, wv):
    """Prefill-sized routing (64 / 150 rows per expert): the tiled kernels and the decode kernel
    with sk = 1 run the same per-step fma sequence, so their outputs are bit-identical.
    wv = 0 takes the streamed kernel (K = 2560 and 768 have one), wv = 2 the general tiled
    kernel at two workgroups per CU."""
    E, H, I = layer["E"], layer["H"], layer["I"]
    top_k = 10
    ids = routing(M, top_k, E, seed=M + 1)
    mtk = ids.size
    al = to_dev_i32(*align_all(ids, E))
    rng = np.random.default_rng(M)
    x = fp8.bf16_round(rng.standard_normal((M, H)).astype(np.float32))
    qx, xs = fp8.group_quant(x, 128)
    qx_t = torch.from_numpy(qx).to(DEV).view(torch.float8_e4m3fn)
    xs_t = torch.from_numpy(xs).to(DEV)
    yt = torch.full((mtk, 2 * I), float("nan"), dtype=torch.bfloat16, device=DEV)
    yd = torch.full_like(yt, float("nan"))
    gpu_case(f"tiled gemm1 M={M} wv={wv}")
    ops.moe_gemm_tiled(yt, qx_t, xs_t, layer["w13t"], layer["w13s"], *al, None, mtk, top_k,
                       wv=wv)
    run_gemm(ops, yd, qx_t, xs_t, layer["w13t"], layer["w13s"], al, None, mtk, top_k, npw=2, sk=1)
    torch.cuda.synchronize()
    assert not torch.isnan(yt).any()
    assert torch.equal(yt.view(torch.int16), yd.view(torch.int16))
    # down projection with routed weights
    a = fp8.bf16_round(rng.standard_normal((mtk, I)).astype(np.float32))
    q2, s2 = fp8.group_quant(a, 128)
    q2_t = torch.from_numpy(q2).to(DEV).view(torch.float8_e4m3fn)
    s2_t = torch.from_numpy(s2).to(DEV)
    tw = torch.from_numpy(rng.random(mtk).astype(np.float32)).to(DEV)
    zt = torch.full((mtk, H), float("nan"), dtype=torch.bfloat16, device=DEV)
    zd = torch.full_like(zt, float("nan"))
    gpu_case(f"tiled gemm2 M={M} wv={wv}")
    # the align's tile list built once and handed over ready, as the layer shares it
    tiles = ops.moe_gemm_tiles(al[1], al[2])
    ops.moe_gemm_tiled(zt, q2_t, s2_t, layer["w2t"], layer["w2s"], *al, tw, mtk, 1, wv=wv,
                       tiles=tiles, tiles_ready=True)
    run_gemm(ops, zd, q2_t, s2_t, layer["w2t"], layer["w2s"], al, tw, mtk, 1, npw=2, sk=1)
    torch.cuda.synchronize()
    assert not torch.isnan(zt).any()
    assert torch.equal(zt.view(torch.int16), zd.view(torch.int16))
    if M == 256:
        used = sorted(set(ids.reshape(-1).tolist()))
        wq, ws = ref_from(layer["w13q"], layer["w13s"], used)
        want = ogemm.moe_gemm(qx, xs, _Lazy(wq), _Lazy(ws), *align_all(ids, E), mtk, top_k)
        assert ogemm.rel_err(np_from_bf16(yt), want) <= TOL


@pytest.mark.parametrize("M", [256, 600])
def test_moe_gemm_tiled_silu_quant_fused(ops, layer, M):
    """gate_up with SiLU-mul-quant in the streamed kernel's epilogue: q2 / s2 equal
    silu_mul_quant of the tiled gate_up output bit for bit on every row the align names; rows
    it does not name (a block set to expert -1) keep their contents. Built for K = 2560 only:
    the down shape (K = 768) reports no kernel and the call raises."""
    E, H, I = layer["E"], layer["H"], layer["I"]
    top_k = 10
    assert ops.moe_gemm_tiled_silu_quant_built(H, 2 * I)
    assert not ops.moe_gemm_tiled_silu_quant_built(I, H)
    ids = routing(M, top_k, E, seed=M + 7)
    mtk = ids.size
    s, e, n = align_all(ids, E)
    e2 = e.copy()
    e2[1] = -1
    al = to_dev_i32(s, e2, n)
    x = fp8.bf16_round(np.random.default_rng(M + 7).standard_normal((M, H)).astype(np.float32))
    qx, xs = fp8.group_quant(x, 128)
    qx_t = torch.from_numpy(qx).to(DEV).view(torch.float8_e4m3fn)
    xs_t = torch.from_numpy(xs).to(DEV)
    y = torch.zeros((mtk, 2 * I), dtype=torch.bfloat16, device=DEV)
    ops.moe_gemm_tiled(y, qx_t, xs_t, layer["w13t"], layer["w13s"], *al, None, mtk, top_k)
    _, q_ref, s_ref = ops.silu_mul_quant(y)
    q = torch.full((mtk, I), 0x7F, dtype=torch.uint8, device=DEV).view(ops.FP8)
    sc = torch.full((mtk, I // 128), float("nan"), device=DEV)
    gpu_case(f"tiled gate_up + silu-mul-quant M={M}")
    ops.moe_gemm_tiled_silu_quant(q, sc, qx_t, xs_t, layer["w13t"], layer["w13s"], *al, mtk,
                                  top_k)
    torch.cuda.synchronize()
    live = np.zeros(mtk, bool)
    live[s[:n[0]][s[:n[0]] < mtk]] = True
    live[s[16:32][s[16:32] < mtk]] = False
    lv = torch.from_numpy(live).to(DEV)
    qb = q.view(torch.uint8)
    assert torch.equal(qb[lv], q_ref.view(torch.uint8)[lv])
    assert torch.equal(sc[lv].view(torch.int32), s_ref[lv].view(torch.int32))
    assert bool((qb[~lv] == 0x7F).all()) and bool(torch.isnan(sc[~lv]).all())
    a2 = torch.zeros((mtk, I), dtype=ops.FP8, device=DEV)          # down-shaped operands
    with pytest.raises(RuntimeError, match="rc=-6"):
        ops.moe_gemm_tiled_silu_quant(
            torch.empty((mtk, H // 2), dtype=ops.FP8, device=DEV),
            torch.empty((mtk, H // 256), device=DEV), a2, torch.ones((mtk, I // 128), device=DEV),
            layer["w2t"], layer["w2s"], *al, mtk, 1)


# ---- the prefill GEMMs over a layer's two aligns in one launch -------------------------------
def split_case(layer, M, hot_share, seed):
    """A hot / cold split of prefill routing over the layer's 40 experts: every hot_share-th
    routed expert resident in a slot (0: only an expert no row routes to, so the hot align is
    empty; -1: every routed expert, so the cold align is empty). Returns the routing, the two
    aligns (host arrays) and the slot tensors' expert order."""
    E = layer["E"]
    ids = routing(M, 10, E - 1 if hot_share == 0 else E, seed=seed)   # 0: expert E - 1 unused
    used = sorted(set(ids.reshape(-1).tolist()))
    if hot_share > 0:
        hot_experts = used[::hot_share]
    elif hot_share == 0:
        hot_experts = [E - 1]
    else:
        hot_experts = used
    al = align_all(ids, E, {e: i for i, e in enumerate(hot_experts)})
    return ids, al, hot_experts


@pytest.mark.parametrize("M,hot_share", [(256, 2), (600, 3), (37, 2), (256, 0), (256, -1)])
def test_moe_gemm_tile_list_split(ops, layer, M, hot_share):
    """The tile list of two aligns: the hot align's tiles, then the cold align's with bit 16
    of the block count set, then the count -- each list as tiles_ref walks it."""
    _, al, _ = split_case(layer, M, hot_share, seed=M + 11)
    sh, eh, nh, sc, ec, nc = al
    e_h, n_h, e_c, n_c = to_dev_i32(eh, nh, ec, nc)
    gpu_case(f"split tile list M={M} hot_share={hot_share}")
    tl = ops.moe_gemm_tiles_split((e_h, n_h), (e_c, n_c))
    torch.cuda.synchronize()
    got = tl.cpu().numpy()
    want = tiles_ref(eh, nh[0]) + [(b, n | 1 << 16) for b, n in tiles_ref(ec, nc[0])]
    nt = int(got[-1])
    assert nt == len(want)
    assert [tuple(x) for x in got[:2 * nt].reshape(-1, 2)] == want
    assert len(got) == 2 * (len(eh) + len(ec)) + 1


@pytest.mark.parametrize("M,hot_share,pinned", [(256, 2, False), (600, 3, True), (37, 2, False),
                                                (256, 0, False), (256, -1, True)])
def test_moe_gemm_tiled_split_equals_two_calls(ops, layer, M, hot_share, pinned):
    """moe_gemm_tiled_split over a hot align (slot weights) and a cold align (the full tensor,
    in device or pinned host memory) in one launch equals moe_gemm_tiled on each align bit
    for bit: gate_up, down with routed weights, and gate_up with SiLU-mul-quant."""
    E, H, I = layer["E"], layer["H"], layer["I"]
    ids, al, hot_experts = split_case(layer, M, hot_share, seed=M + 13)
    mtk = ids.size
    sh, eh, nh, sc, ec, nc = to_dev_i32(*al)
    hot, cold = (sh, eh, nh), (sc, ec, nc)
    idx = torch.tensor(hot_experts, device=DEV)

    def full(t):
        if not pinned:
            return t
        h = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
        h.copy_(t)
        return h
    rng = np.random.default_rng(M + 17)
    x = fp8.bf16_round(rng.standard_normal((M, H)).astype(np.float32))
    qx, xs = fp8.group_quant(x, 128)
    qx_t = torch.from_numpy(qx).to(DEV).view(torch.float8_e4m3fn)
    xs_t = torch.from_numpy(xs).to(DEV)
    a = fp8.bf16_round(rng.standard_normal((mtk, I)).astype(np.float32))
    q2, s2 = fp8.group_quant(a, 128)
    q2_t = torch.from_numpy(q2).to(DEV).view(torch.float8_e4m3fn)
    s2_t = torch.from_numpy(s2).to(DEV)
    tw = torch.from_numpy(rng.random(mtk).astype(np.float32)).to(DEV)
    for name, w, s, xq, xsc, twt, tk, N in (
            ("gate_up", layer["w13t"], layer["w13s"], qx_t, xs_t, None, 10, 2 * I),
            ("down", layer["w2t"], layer["w2s"], q2_t, s2_t, tw, 1, H)):
        sw, ss = w[idx].contiguous(), s[idx].contiguous()
        fw, fs = full(w), full(s)
        y2 = torch.full((mtk, N), float("nan"), dtype=torch.bfloat16, device=DEV)
        gpu_case(f"split tiled {name} M={M} hot_share={hot_share} pinned={pinned}: two calls")
        ops.moe_gemm_tiled(y2, xq, xsc, sw, ss, *hot, twt, mtk, tk)
        ops.moe_gemm_tiled(y2, xq, xsc, fw, fs, *cold, twt, mtk, tk)
        y1 = torch.full_like(y2, float("nan"))
        gpu_case(f"split tiled {name} M={M} hot_share={hot_share} pinned={pinned}: one launch")
        ops.moe_gemm_tiled_split(y1, xq, xsc, sw, ss, hot, fw, fs, cold, twt, mtk, tk)
        torch.cuda.synchronize()
        assert not torch.isnan(y1).any()
        assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
        if name == "gate_up":
            qa = torch.full((mtk, I), 0x7F, dtype=torch.uint8, device=DEV).view(ops.FP8)
            sa = torch.full((mtk, I // 128), float("nan"), device=DEV)
            qb = torch.full_like(qa.view(torch.uint8), 0x7F).view(ops.FP8)
            sb = torch.full_like(sa, 1.0)
            gpu_case(f"split tiled gate_up + silu-mul-quant M={M} hot_share={hot_share}")
            ops.moe_gemm_tiled_silu_quant(qa, sa, xq, xsc, sw, ss, *hot, mtk, tk)
            ops.moe_gemm_tiled_silu_quant(qa, sa, xq, xsc, fw, fs, *cold, mtk, tk)
            ops.moe_gemm_tiled_split_silu_quant(qb, sb, xq, xsc, sw, ss, hot, fw, fs, cold, mtk,
                                                tk)
            torch.cuda.synchronize()
            assert not torch.isnan(sa).any()
            assert torch.equal(qa.view(torch.uint8), qb.view(torch.uint8))
            assert torch.equal(sa.view(torch.int32), sb.view(torch.int32))


def test_moe_gemm_tiled_split_return_codes(pkg, ops):
    """Built for the streamed kernel's shapes only (-6 otherwise, before any other check);
    null pointers -1; the tile builder's limits."""
    assert ops.moe_gemm_tiled_split_built(2560, 1536) and ops.moe_gemm_tiled_split_built(768, 2560)
    assert not ops.moe_gemm_tiled_split_built(1024, 1536)
    assert not ops.moe_gemm_tiled_split_built(2560, 1536 + 128)
    P = ctypes.c_void_p
    lib = pkg.lib()
    s = P(torch.cuda.current_stream().cuda_stream)
    z = [P(0)] * 12
    assert lib.rlu_moe_gemm_fp8blk_tiled_split_silu_quant(*z, 1, P(0), P(0), 0, 1, 768, 2560,
                                                          s) == -6
    assert lib.rlu_moe_gemm_fp8blk_tiled_split(*z, 1, P(0), P(0), 20, 10, 2560, 1536, s) == -1
    assert lib.rlu_moe_gemm_fp8blk_tiled_split_silu_quant(*z, 1, P(0), P(0), 20, 10, 2560, 1536,
                                                          s) == -1
    assert lib.rlu_moe_gemm_fp8blk_tiled_split(*z, 0, P(0), P(0), 20, 10, 2560, 1536, s) == -1
    # the one-align entries: a NULL operand is -1 before anything is launched (mtk > 0)
    z8 = [P(0)] * 8
    assert lib.rlu_moe_gemm_fp8blk_tiled(*z8, 1, P(0), P(0), 20, 10, 2560, 1536, 0, s) == -1
    assert lib.rlu_moe_gemm_fp8blk_tiled_silu_quant(*z8, 1, P(0), P(0), 20, 10, 2560, 1536,
                                                    s) == -1
    assert lib.rlu_moe_gemm_fp8blk_tiled_noalloc(*([P(0)] * 5), P(1), P(1), 1, P(0), P(0), 20,
                                                 10, 2560, 1536, 0, s) == -1
    t = torch.zeros(64, dtype=torch.int32, device=DEV)
    p = P(t.data_ptr())
    assert lib.rlu_moe_gemm_tiles_split(p, p, 4, p, p, 8193, p, p, s) == -1
    assert lib.rlu_moe_gemm_tiles_split(p, p, 0, p, p, 4, p, p, s) == -1
    assert lib.rlu_moe_gemm_tiles_split(p, p, 4, P(0), p, 4, p, p, s) == -1


def test_moe_gemm_tiled_row_contract_and_graph(ops, layer):
    """A block of expert -1 is skipped (its rows stay NaN); graph replay equals eager."""
    E, H, I = layer["E"], layer["H"], layer["I"]
    M, top_k = 128, 10
    ids = routing(M, top_k, E, seed=5)
    mtk = ids.size
    s, e, n = align_all(ids, E)
    e2 = e.copy()
    e2[1] = -1
    al = to_dev_i32(s, e2, n)
    x = fp8.bf16_round(np.random.default_rng(6).standard_normal((M, H)).astype(np.float32))
    qx, xs = fp8.group_quant(x, 128)
    qx_t = torch.from_numpy(qx).to(DEV).view(torch.float8_e4m3fn)
    xs_t = torch.from_numpy(xs).to(DEV)
    y = torch.full((mtk, 2 * I), float("nan"), dtype=torch.bfloat16, device=DEV)
    tiles = torch.empty(2 * e2.size + 1, dtype=torch.int32, device=DEV)
    gpu_case("tiled gemm row contract")
    ops.moe_gemm_tiled(y, qx_t, xs_t, layer["w13t"], layer["w13s"], *al, None, mtk, top_k,
                       tiles=tiles)
    torch.cuda.synchronize()
    skipped = s[16:32][s[16:32] < mtk]
    written = ~torch.isnan(y).any(dim=1).cpu().numpy()
    live = np.zeros(mtk, bool)
    live[s[:n[0]][s[:n[0]] < mtk]] = True
    live[skipped] = False
    assert np.array_equal(written, live)
    g = torch.cuda.CUDAGraph()
    y2 = torch.full_like(y, float("nan"))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.moe_gemm_tiled(y2, qx_t, xs_t, layer["w13t"], layer["w13s"], *al, None, mtk, top_k,
                           tiles=tiles)
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(g):
        ops.moe_gemm_tiled(y2, qx_t, xs_t, layer["w13t"], layer["w13s"], *al, None, mtk, top_k,
                           tiles=tiles)
    for _ in range(3):
        y2.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y2.view(torch.int16), y.view(torch.int16))


class _OrigHead:
    """Stand-in for the lm_head's original quant method: records calls, returns a marker."""

    def __init__(self):
        self.calls = []
        self.tag = "orig-attr"

    def apply(self, layer, x, bias=None):
        self.calls.append((tuple(x.shape), x.dtype, bias is not None))
        return "orig"


def test_fp8_target_head(ops, lm_head):
    """Fp8TargetHead (kernels/fp8_target_lmhead.py:77-93): batched bf16 input of up to 64 rows
    goes through gemm_fp8_block in 16-row launches (rows of a full slice equal a direct 16-row
    call bit for bit; all rows within 1e-2 of the float64 dequant reference); more rows, a
    bias or another dtype go to the original method; other attributes pass through."""
    wq, ws, wt = lm_head
    N, K = wq.shape
    head = ops.Fp8TargetHead.__new__(ops.Fp8TargetHead)
    head.orig, head.wq, head.ws, head.n_fp8 = _OrigHead(), wt, ws, 0
    rng = np.random.default_rng(40)
    x = fp8.bf16_round(rng.standard_normal((2, 20, K)).astype(np.float32))
    xt = bf16_from_np(x.reshape(40, K)).reshape(2, 20, K)
    gpu_case("fp8 target head M=40")
    y = head.apply(None, xt)
    y16 = ops.gemm_fp8_block(xt.reshape(40, K)[16:32], wt, ws)
    torch.cuda.synchronize()
    assert y.shape == (2, 20, N) and head.n_fp8 == 1 and not head.orig.calls
    assert torch.equal(y.reshape(40, N)[16:32].view(torch.int16), y16.view(torch.int16))
    qx, xs = fp8.group_quant(x.reshape(40, K), 128)
    a = torch.from_numpy(fp8.dequant_act(qx, xs)).to(DEV).double()
    wd = (wq.float() * ws.repeat_interleave(128, 0).repeat_interleave(128, 1)).double()
    ref = a @ wd.T
    del wd
    err = ((y.reshape(40, N).double() - ref).abs().max() / ref.abs().max()).item()
    assert err <= TOL, f"rel err {err:.3e}"
    # routed to the original method
    big = torch.zeros((65, K), dtype=torch.bfloat16, device=DEV)
    assert head.apply(None, big) == "orig"
    assert head.apply(None, xt, bias=torch.zeros(N, device=DEV)) == "orig"
    assert head.apply(None, xt.float()) == "orig"
    assert [c[0] for c in head.orig.calls] == [(65, K), (2, 20, K), (2, 20, K)]
    assert head.n_fp8 == 1 and head.tag == "orig-attr"


def test_fp8_target_head_packs_its_weight(ops):
    """The constructor packs the weight exactly as pack_fp8_block does."""
    g = torch.Generator(device=DEV).manual_seed(3)
    w = (torch.randn(256, 384, device=DEV, generator=g) * 0.05).to(torch.bfloat16)
    gpu_case("fp8 target head pack")
    head = ops.Fp8TargetHead(_OrigHead(), w)
    wt, ws = ops.pack_fp8_block(w)
    torch.cuda.synchronize()
    assert torch.equal(head.wq.view(torch.uint8), wt.view(torch.uint8))
    assert torch.equal(head.ws, ws)


# ---- the grouped-GEMM torch ops at the reference's names ---------------------------------------
def _c_gemm(pkg, y, qx, xs, wq_ptr, ws_ptr, al, tw, mtk, top_k, npw=4, sk=0):
    """The C-ABI call itself (r4d_gemm_moe_fp8blk_nt_b16), no Python op in between."""
    P = ctypes.c_void_p
    rc = pkg.lib().r4d_gemm_moe_fp8blk_nt_b16(
        P(qx.data_ptr()), P(xs.data_ptr()), P(wq_ptr), P(ws_ptr), P(0), P(y.data_ptr()),
        P(al[0].data_ptr()), P(al[1].data_ptr()), P(al[2].data_ptr()),
        P(0 if tw is None else tw.data_ptr()), al[0].numel(), mtk, top_k, qx.shape[1],
        y.shape[1], 0, sk, npw, P(torch.cuda.current_stream().cuda_stream))
    assert rc == 0


def test_moe_gemm_ops_equal_c_abi(pkg, ops, layer):
    """torch.ops.<ns>.r4d_mxfp4_moe_gemm_into (patches/.../r4d_mxfp4_moe.py.lru.diff:363-423,
    mutates y) over the hot slots and then the full expert tensor in pinned host memory, and
    the allocating r4d_mxfp4_moe_gemm (:625,635) over one all-expert align, equal the C-ABI
    calls bit for bit -- eagerly, and replayed three times from a captured graph with new
    activations and routed weights."""
    ns = getattr(torch.ops, pkg.lru.OPS_NAMESPACE)
    E, H, I = layer["E"], layer["H"], layer["I"]
    M, top_k = 5, 10
    ids = routing(M, top_k, E, seed=51)
    mtk = ids.size
    hot_experts = sorted(set(ids.reshape(-1).tolist()))[::3]
    hot = {ex: i for i, ex in enumerate(hot_experts)}
    al = to_dev_i32(*align_all(ids, E, hot))
    al_all = to_dev_i32(*align_all(ids, E))
    idx = torch.tensor(hot_experts, device=DEV)
    sq, ss = layer["w2t"][idx].contiguous(), layer["w2s"][idx].contiguous()
    hq = torch.empty(layer["w2t"].shape, dtype=layer["w2t"].dtype, pin_memory=True)
    hs = torch.empty(layer["w2s"].shape, dtype=torch.float32, pin_memory=True)
    hq.copy_(layer["w2t"])
    hs.copy_(layer["w2s"])
    hqp, hsp = pkg._lib.device_ptr_of_pinned(hq), pkg._lib.device_ptr_of_pinned(hs)
    rng = np.random.default_rng(5)

    def inputs():
        x = fp8.bf16_round(rng.standard_normal((mtk, I)).astype(np.float32))
        q, s_ = fp8.group_quant(x, 128)
        return (torch.from_numpy(q).to(DEV).view(torch.float8_e4m3fn),
                torch.from_numpy(s_).to(DEV),
                torch.from_numpy(rng.random(mtk).astype(np.float32)).to(DEV))

    def expected(q, s_, tw):
        yc = torch.full((mtk, H), float("nan"), dtype=torch.bfloat16, device=DEV)
        _c_gemm(pkg, yc, q, s_, sq.data_ptr(), ss.data_ptr(), al[0:3], tw, mtk, 1)
        _c_gemm(pkg, yc, q, s_, hqp, hsp, al[3:6], tw, mtk, 1)
        ya = torch.full((mtk, H), float("nan"), dtype=torch.bfloat16, device=DEV)
        _c_gemm(pkg, ya, q, s_, layer["w2t"].data_ptr(), layer["w2s"].data_ptr(), al_all, tw,
                mtk, 1)
        return yc, ya

    q, s_, tw = inputs()
    y = torch.full((mtk, H), float("nan"), dtype=torch.bfloat16, device=DEV)
    gpu_case("gemm ops eager")
    ns.r4d_mxfp4_moe_gemm_into(y, q, s_, sq, ss, None, *al[0:3], tw, mtk, 1, 0, 0, 4)
    ns.r4d_mxfp4_moe_gemm_into(y, q, s_, hq, hs, None, *al[3:6], tw, mtk, 1, 0, 0, 4)
    ya = ns.r4d_mxfp4_moe_gemm(q, s_, layer["w2t"], layer["w2s"], None, *al_all, tw, mtk, 1,
                               0, 0, 4)
    yc, yac = expected(q, s_, tw)
    torch.cuda.synchronize()
    assert not torch.isnan(y).any() and ya.shape == (mtk, H)
    assert torch.equal(y.view(torch.int16), yc.view(torch.int16))
    assert torch.equal(ya.view(torch.int16), yac.view(torch.int16))
    assert torch.equal(y.view(torch.int16), ya.view(torch.int16))    # partition invariance

    qg, sg, twg = q.clone(), s_.clone(), tw.clone()
    yg = torch.empty_like(y)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ns.r4d_mxfp4_moe_gemm_into(yg, qg, sg, sq, ss, None, *al[0:3], twg, mtk, 1, 0, 0, 4)
    torch.cuda.current_stream().wait_stream(side)
    gr = torch.cuda.CUDAGraph()
    gpu_case("gemm ops graph capture")
    with torch.cuda.graph(gr):
        ns.r4d_mxfp4_moe_gemm_into(yg, qg, sg, sq, ss, None, *al[0:3], twg, mtk, 1, 0, 0, 4)
        ns.r4d_mxfp4_moe_gemm_into(yg, qg, sg, hq, hs, None, *al[3:6], twg, mtk, 1, 0, 0, 4)
        yag = ns.r4d_mxfp4_moe_gemm(qg, sg, layer["w2t"], layer["w2s"], None, *al_all, twg,
                                    mtk, 1, 0, 0, 4)
    for _ in range(3):
        q, s_, tw = inputs()
        qg.copy_(q)
        sg.copy_(s_)
        twg.copy_(tw)
        gr.replay()
        torch.cuda.synchronize()
        yc, yac = expected(q, s_, tw)
        torch.cuda.synchronize()
        assert torch.equal(yg.view(torch.int16), yc.view(torch.int16))
        assert torch.equal(yag.view(torch.int16), yac.view(torch.int16))
