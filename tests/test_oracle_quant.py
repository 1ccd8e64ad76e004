"""CPU: pin the fp8 / quant / GEMM oracle before trusting it.

* e4m3 table and encoder against torch's float8_e4m3fn cast (every code, every rounding midpoint);
* the float32 exp against math.exp (<= 2 ulp);
* quantizer closed forms: the zero row lands on 1/(448*512) (docs/PATCHES.md:916-921); every
  code is the nearest e4m3 to x/scale (brute force over all 256 codes); the scale is the group
  amax / 448; dequantized error within half an e4m3 step;
* block weight quant against its closed form (kernels/fp8_target_lmhead.py:57-64);
* the grouped-GEMM reference against a pure-Python triple loop on tiny shapes, including the
  row contract (padding rows, expert -1, num_post_pad);
* moe_sum against a float64 sum within one bf16 rounding;
* the fragment-order weight shuffle against a byte-by-byte walk of its address formula.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import fp8, gemm

torch = pytest.importorskip("torch")


def test_e4m3_table_matches_torch():
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    t = fp8.e4m3_table()
    assert np.array_equal(np.isnan(ref), np.isnan(t))
    assert np.array_equal(ref[~np.isnan(ref)], t[~np.isnan(t)])
    assert t[0x7E] == 448.0 and t[0x01] == 2.0 ** -9


def test_e4m3_encoder_matches_torch_on_midpoints():
    vals = np.unique(fp8.e4m3_table()[~np.isnan(fp8.e4m3_table())])
    mids = ((vals[:-1].astype(np.float64) + vals[1:]) / 2).astype(np.float32)
    up = np.nextafter(mids, np.float32(np.inf)).astype(np.float32)
    dn = np.nextafter(mids, np.float32(-np.inf)).astype(np.float32)
    rng = np.random.default_rng(0)
    x = np.concatenate([vals, mids, up, dn, rng.standard_normal(200_000).astype(np.float32) * 30,
                        rng.standard_normal(50_000).astype(np.float32) * 1e-3,
                        np.array([0, -0.0, 1e-12, -1e-12, 447.9, 448, -448], np.float32)])
    x = x.astype(np.float32)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(fp8.f32_to_e4m3(x), ref)


def test_exp_within_two_ulp():
    x = np.linspace(-87, 88, 400_001, dtype=np.float32)
    got = fp8.exp_f32(x).astype(np.float64)
    want = np.array([math.exp(float(v)) for v in x[::97]])
    g = got[::97]
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    assert (np.abs(g - want) / ulp).max() <= 2.0
    assert fp8.exp_f32(np.array([89.0], np.float32))[0] == np.inf
    assert fp8.exp_f32(np.array([-104.0], np.float32))[0] == 0.0


def test_silu_zero_row_lands_on_scale_floor():
    _, q, s = fp8.silu_mul_quant(np.zeros((2, 640), np.float32), group=0)
    assert np.allclose(s, 1.0 / (448.0 * 512.0)) and abs(s[0, 0] - 4.35965e-06) < 1e-10
    assert not q.any()


@pytest.mark.parametrize("group", [0, 128])
def test_quant_codes_are_nearest(group):
    rng = np.random.default_rng(1)
    x = fp8.bf16_round(rng.standard_normal((3, 512)).astype(np.float32) * 3)
    q, s = fp8.group_quant(x, group)
    gs = 512 if group == 0 else group
    amax = np.abs(x).reshape(3, -1, gs).max(-1)
    assert np.array_equal(s, np.maximum(np.float32(amax / np.float32(448)),
                                        np.float32(1 / (448 * 512))))
    v = np.float32(x / np.repeat(s, gs, 1))
    table = fp8.e4m3_table()
    finite = np.nonzero(~np.isnan(table))[0]
    d = np.abs(v.reshape(-1, 1).astype(np.float64) - table[finite][None, :])
    best = d.min(1)
    got = np.abs(v.reshape(-1).astype(np.float64) - table[q.reshape(-1)])
    assert np.array_equal(best, got)                       # nearest (ties: either code)
    # max code is hit in every group: amax maps to 448
    assert (np.abs(table[q]).reshape(3, -1, gs).max(-1) == 448.0).all()


def test_silu_matches_definition():
    rng = np.random.default_rng(2)
    x = fp8.bf16_round(rng.standard_normal((4, 256)).astype(np.float32) * 4)
    act, q, s = fp8.silu_mul_quant(x, group=128)
    g, u = x[:, :128].astype(np.float64), x[:, 128:].astype(np.float64)
    silu = g / (1 + np.exp(-g))
    want = silu * u
    assert np.abs(act - want).max() <= 2 ** -7 * np.abs(want).max() + 1e-30
    deq = fp8.dequant_act(q, s)
    assert np.abs(deq - act).max() <= np.abs(act).max() / 16 + 1e-12   # e4m3: 3 mantissa bits


def test_block_quant_weight_closed_form():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((256, 384)) * 0.02).astype(np.float32)
    wq, ws = fp8.block_quant_weight(w)
    amax = np.abs(w.reshape(2, 128, 3, 128)).max(axis=(1, 3))
    assert np.array_equal(ws, np.float32(np.maximum(amax, np.float32(1e-12)) / np.float32(448)))
    t = fp8.e4m3_table()
    assert (np.abs(t[wq]).reshape(2, 128, 3, 128).max(axis=(1, 3)) == 448.0).all()
    deq = fp8.dequant_weight(wq, ws)
    assert np.abs(deq - w).max() <= np.repeat(np.repeat(ws, 128, 0), 128, 1).max() * 16
    torch_q = torch.from_numpy(np.clip(w.reshape(2, 128, 3, 128) / ws[:, None, :, None],
                                       -448, 448).astype(np.float32)).to(torch.float8_e4m3fn)
    assert np.array_equal(torch_q.view(torch.uint8).numpy().reshape(256, 384), wq)


def test_moe_gemm_reference_against_loops():
    rng = np.random.default_rng(4)
    E, N, K, M, top_k = 3, 128, 256, 3, 2
    mtk = M * top_k
    w = (rng.standard_normal((E, N, K)) * 0.05).astype(np.float32)
    wq = np.empty((E, N, K), np.uint8)
    ws = np.empty((E, N // 128, K // 128), np.float32)
    for e in range(E):
        wq[e], ws[e] = fp8.block_quant_weight(w[e])
    x = fp8.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    qx, xs = fp8.group_quant(x, 128)
    sorted_ids = np.array([0, 3, mtk] + [mtk] * 13 + [1, 2, 4] + [mtk] * 13 + [5] + [mtk] * 15,
                          np.int32)
    expert_ids = np.array([2, 0, -1], np.int32)
    tw = rng.random(mtk).astype(np.float32)
    y = gemm.moe_gemm(qx, xs, wq, ws, sorted_ids, expert_ids, [48], mtk, top_k, tw=tw)
    A = fp8.dequant_act(qx, xs)
    for row, e in ((0, 2), (3, 2), (1, 0), (2, 0), (4, 0)):
        W = fp8.dequant_weight(wq[e], ws[e])
        for n in range(0, N, 37):
            acc = 0.0
            for k in range(K):
                acc += float(A[row // top_k, k]) * float(W[n, k])
            assert abs(y[row, n] - acc * float(tw[row])) <= 1e-9 * max(1.0, abs(acc))
    assert np.isnan(y[5]).all()                   # block of expert -1 is skipped
    y2 = gemm.moe_gemm(qx, xs, wq, ws, sorted_ids, expert_ids, [16], mtk, top_k)
    assert np.isnan(y2[[1, 2, 4, 5]]).all() and not np.isnan(y2[[0, 3]]).any()


def test_moe_sum_reference():
    rng = np.random.default_rng(5)
    x = fp8.bf16_round(rng.standard_normal((5 * 10, 64)).astype(np.float32))
    out = gemm.moe_sum(x, 5, 10)
    want = x.astype(np.float64).reshape(5, 10, 64).sum(1)
    assert np.abs(out - want).max() <= np.abs(want).max() * 2 ** -7
    assert np.array_equal(out, fp8.bf16_round(out))


def test_shuffle_layout_formula():
    """Every byte (n, k) of a [2, 64, 384] stack lands where the fragment-order formula says
    (the gfx950 counterpart of tests/k3/test_layout.py), and unshuffle inverts it."""
    E, N, K = 2, 64, 384
    w = (np.arange(E * N * K, dtype=np.int64) % 251).astype(np.uint8).reshape(E, N, K)
    s = fp8.shuffle_weight(w)
    flat = s.reshape(E, -1)
    KB = K // 128
    for e in range(E):
        for n in range(N):
            nt, r = divmod(n, 16)
            for k in range(K):
                kb, rem = divmod(k, 128)
                h, rem = divmod(rem, 64)
                c, j = divmod(rem, 16)
                off = ((nt * KB + kb) * 2 + h) * 1024 + (16 * c + r) * 16 + j
                assert flat[e, off] == w[e, n, k], (e, n, k)
    assert np.array_equal(fp8.unshuffle_weight(s), w)
    # the lane view: lane l = 16 c + r reads 16 contiguous bytes = row r, k in [16c, 16c + 16)
    lane_bytes = s[0].reshape(-1)[:1024].reshape(64, 16)
    for l in range(64):
        assert np.array_equal(lane_bytes[l], w[0, l % 16, 16 * (l // 16):16 * (l // 16) + 16])
