"""fp32-dequant references of the GEMMs on the path (test infrastructure only).

  moe_gemm()   the grouped expert GEMM contract of r4d_mxfp4_moe_gemm_into
               (patches/.../r4d_mxfp4_moe.py.lru.diff:363-395) as probed by
               tests/k1/moe_ref_harness.py:199-207,282-321: block b of sorted_ids (16 rows) uses
               expert expert_ids[b] (-1 skips it); row id `so` < mtk reads activation row
               so // top_k and writes output row so; rows past num_post_pad and sentinel rows
               are never written; y[so] *= tw[so] when tw is given. Dequantized operands,
               float64 accumulation. Pinned by a pure-Python triple loop on tiny shapes.
  moe_sum()    out[m] = bf16(sum_k in[m * top_k + k]) in float32, k ascending (the contract of
               vLLM's moe_sum as used at r4d_mxfp4_moe.py.lru.diff:696; its own accumulation
               order is parity unpinned -- vLLM is absent -- this is the build's convention).
"""
from __future__ import annotations

import numpy as np

from . import fp8


def moe_gemm(qx, xs, wq, ws, sorted_ids, expert_ids, npad, mtk, top_k, tw=None, y=None,
             cache=None):
    """-> y float64 [mtk, N]; rows not named by the align output keep their value in `y`
    (NaN when y is None)."""
    sorted_ids = np.asarray(sorted_ids)
    expert_ids = np.asarray(expert_ids)
    npad = int(np.asarray(npad).reshape(-1)[0])
    N = wq.shape[1]
    if y is None:
        y = np.full((mtk, N), np.nan)
    A = fp8.dequant_act(qx, xs).astype(np.float64)
    cache = {} if cache is None else cache
    for b in range(npad // 16):
        e = int(expert_ids[b])
        if e < 0:
            continue
        rows = sorted_ids[b * 16:(b + 1) * 16]
        rows = rows[rows < mtk].astype(np.int64)
        if rows.size == 0:
            continue
        if e not in cache:
            cache[e] = fp8.dequant_weight(wq[e], ws[e]).astype(np.float64)
        out = A[rows // top_k] @ cache[e].T
        if tw is not None:
            out = out * np.asarray(tw, np.float64)[rows, None]
        y[rows] = out
    return y


def moe_sum(ic3: np.ndarray, M: int, top_k: int) -> np.ndarray:
    """ic3 float32 holding bf16 values [M * top_k, H] -> bf16-as-float32 [M, H]."""
    x = np.asarray(ic3, np.float32).reshape(M, top_k, -1)
    acc = np.zeros((M, x.shape[2]), np.float32)
    for k in range(top_k):
        acc = np.float32(acc + x[:, k])
    return fp8.bf16_round(acc)


def rel_err(got, want) -> float:
    """max |got - want| / max |want| over the finite entries of want (the metric of
    tests/k1/moe_ref_harness.py:352-357)."""
    want = np.asarray(want, np.float64)
    got = np.asarray(got, np.float64)
    m = np.isfinite(want)
    denom = max(np.abs(want[m]).max(), 1e-30)
    return float(np.abs(got[m] - want[m]).max() / denom)
