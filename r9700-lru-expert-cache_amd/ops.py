"""Host side of the quant, SiLU-quant, moe_sum and fp8 GEMM kernels of librlu.so.

Mirrors the reference's Python entry points for these stages:
  silu_mul_quant / supported      kernels/fused_silu_mul_quant.py:60-101
  fp8_quant_group                 the activation quant of r4dhip.py.diff:22-34 and of
                                  kernels/fp8_target_lmhead.py:72-73 (per token group 128)
  moe_sum                         vLLM ops.moe_sum (r4d_mxfp4_moe.py.lru.diff:696)
  _r4d_fp8_moe_gemm_into          the op r4d_mxfp4_moe_gemm_into (r4d_mxfp4_moe.py.lru.diff:
                                  363-423), same argument list; ws_t = [E, N/128, K/128] fp32
                                  block scales, x_scale = [rows, K/128]; wref unused
  gemm_fp8_block                  kernels/fp8_target_lmhead.py:70-74
  Fp8TargetHead                   kernels/fp8_target_lmhead.py:77-93
  shuffle_fp8_weight              shuffle_weight_gfx1201 (kernels/fp8_target_lmhead.py:47,64),
                                  here the gfx950 MFMA fragment order every GEMM reads
  pack_fp8_block                  kernels/fp8_target_lmhead.py:44-66
  moe_gemm_tiled                  the grouped GEMM for prefill-sized inputs (no counterpart:
                                  the reference ran one closed kernel at every M)
Errors from the C-ABI raise RuntimeError; there is no fallback implementation (Fp8TargetHead
hands the calls its kernel does not take to the caller's own lm_head method, as the
reference's does).
"""
from __future__ import annotations

import ctypes
import os

import torch

from ._lib import check, device_ptr, lib, stream_ptr

_P = ctypes.c_void_p
FP8 = torch.float8_e4m3fn
GROUP = 128
MAX_ROW_PER_TOKEN = 256 * 8 * 4     # per-token SiLU-quant row limit (one workgroup)


def _p(t: torch.Tensor | None) -> _P:
    return _P(0 if t is None else t.data_ptr())


def supported(x: torch.Tensor) -> bool:
    """Whether `x` is a [rows, 2*d] gated-activation input the fused kernel handles
    (kernels/fused_silu_mul_quant.py:60-72, with this kernel's own limits)."""
    return (x.is_cuda and x.ndim == 2 and x.dtype == torch.bfloat16 and x.shape[1] % 16 == 0
            and x.stride(1) == 1 and x.stride(0) % 8 == 0 and x.shape[1] // 2 <= MAX_ROW_PER_TOKEN)


def silu_mul_quant(x: torch.Tensor, fp8_dtype: torch.dtype = FP8, write_act: bool = False,
                   group: int = GROUP, out: tuple | None = None):
    """silu(x[:, :d]) * x[:, d:] and its e4m3 quant in one launch -> (act|None, q, scale).
    group=128: scale [rows, d/128]; group=0: the reference's per-token scale [rows, 1]."""
    assert fp8_dtype == FP8, "e4m3fn only"
    assert supported(x), "silu_mul_quant: unsupported input"
    rows, d = x.shape[0], x.shape[1] // 2
    if out is None:
        q = torch.empty((rows, d), dtype=FP8, device=x.device)
        scale = torch.empty((rows, d // group if group else 1), dtype=torch.float32,
                            device=x.device)
    else:
        q, scale = out
    act = torch.empty((rows, d), dtype=x.dtype, device=x.device) if write_act else None
    rc = lib().rlu_silu_mul_quant(_p(x), rows, d, x.stride(0), group, _p(q), _p(scale), _p(act),
                                  _P(stream_ptr()))
    check(rc, "rlu_silu_mul_quant")
    return act, q, scale


def fp8_quant_group(x: torch.Tensor, group: int = GROUP, out: tuple | None = None):
    """bf16 [rows, K] -> (e4m3 [rows, K], fp32 scale [rows, K/group] or [rows, 1])."""
    assert x.dtype == torch.bfloat16 and x.ndim == 2 and x.stride(1) == 1
    rows, K = x.shape
    if out is None:
        q = torch.empty((rows, K), dtype=FP8, device=x.device)
        scale = torch.empty((rows, K // group if group else 1), dtype=torch.float32,
                            device=x.device)
    else:
        q, scale = out
    rc = lib().rlu_quant_fp8_group(_p(x), rows, K, x.stride(0), group, _p(q), _p(scale),
                                   _P(stream_ptr()))
    check(rc, "rlu_quant_fp8_group")
    return q, scale


def moe_sum(ic3: torch.Tensor, output: torch.Tensor) -> None:
    """output[m] = sum_k ic3[m, k] for ic3 [M, top_k, H] bf16 (vLLM ops.moe_sum signature)."""
    M, top_k, H = ic3.shape
    assert ic3.is_contiguous() and output.is_contiguous() and output.shape == (M, H)
    rc = lib().rlu_moe_sum(_p(ic3), M, top_k, H, _p(output), _P(stream_ptr()))
    check(rc, "rlu_moe_sum")


def moe_down_sum(q2: torch.Tensor, s2: torch.Tensor, topk_ids: torch.Tensor,
                 topk_weights: torch.Tensor, table: torch.Tensor, w_hot: torch.Tensor,
                 s_hot: torch.Tensor, w_full: torch.Tensor, s_full: torch.Tensor,
                 out: torch.Tensor) -> None:
    """The decode down projection with moe_sum folded in: out [M, N] bf16 = moe_sum of the
    down GEMM's routed-weight rows, bit for bit, without the [M top_k, N] intermediate. Expert
    e comes from slot table[e] of (w_hot, s_hot) when resident, else from (w_full, s_full)
    (device or pinned host memory). topk_ids int32 [M, top_k] with every id in [0, E)."""
    M, top_k = topk_ids.shape
    N, K = w_full.shape[1], w_full.shape[2]
    assert topk_ids.dtype == torch.int32 and topk_ids.is_contiguous()
    assert topk_weights.dtype == torch.float32 and topk_weights.is_contiguous()
    assert topk_weights.shape == (M, top_k) and q2.shape == (M * top_k, K)
    assert out.shape == (M, N) and out.dtype == torch.bfloat16 and out.is_contiguous()
    rc = lib().rlu_moe_down_sum(
        _p(q2), _p(s2), _p(topk_ids), _p(topk_weights), _p(table), _p(w_hot), _p(s_hot),
        _P(device_ptr(w_full)), _P(device_ptr(s_full)), _p(out), M, top_k, K, N,
        w_full.shape[0], _P(stream_ptr()))
    check(rc, "rlu_moe_down_sum")


def moe_down_sum_act(act: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
                     table: torch.Tensor, w_hot: torch.Tensor, s_hot: torch.Tensor,
                     w_full: torch.Tensor, s_full: torch.Tensor, out: torch.Tensor) -> None:
    """moe_down_sum from the bf16 SiLU-mul activation act [M top_k, K] (what
    moe_gemm_split_act writes) in place of silu_mul_quant's q2 / s2: the kernel quantizes each
    token's rows per 128-column group as silu_mul_quant does, so out is the same bit for bit
    and the activation needs no quant launch of its own."""
    M, top_k = topk_ids.shape
    N, K = w_full.shape[1], w_full.shape[2]
    assert topk_ids.dtype == torch.int32 and topk_ids.is_contiguous()
    assert topk_weights.dtype == torch.float32 and topk_weights.is_contiguous()
    assert topk_weights.shape == (M, top_k) and act.shape == (M * top_k, K)
    assert act.dtype == torch.bfloat16 and act.is_contiguous()
    assert out.shape == (M, N) and out.dtype == torch.bfloat16 and out.is_contiguous()
    rc = lib().rlu_moe_down_sum_act(
        _p(act), _p(topk_ids), _p(topk_weights), _p(table), _p(w_hot), _p(s_hot),
        _P(device_ptr(w_full)), _P(device_ptr(s_full)), _p(out), M, top_k, K, N,
        w_full.shape[0], _P(stream_ptr()))
    check(rc, "rlu_moe_down_sum_act")


def _r4d_fp8_moe_gemm_into(y: torch.Tensor, qx: torch.Tensor, x_scale: torch.Tensor,
                           wq: torch.Tensor, ws_t: torch.Tensor, wref: torch.Tensor | None,
                           sorted_ids: torch.Tensor, expert_ids: torch.Tensor,
                           num_post_pad: torch.Tensor, topk_weights: torch.Tensor | None,
                           mtk: int, top_k: int, wv: int, sk: int, npw: int) -> None:
    """The grouped GEMM writing into caller-owned y: only rows named in sorted_ids are
    touched, so hot and cold subsets fill one buffer. wq / ws_t may be device memory (the
    slots) or pinned host memory (the full expert tensor, read over the host link)."""
    K = qx.shape[1]
    N = wq.shape[1]
    assert y.shape == (mtk, N) and y.dtype == torch.bfloat16 and y.is_contiguous()
    assert qx.dtype == FP8 and wq.dtype == FP8 and wq.shape[2] == K
    assert x_scale.dtype == torch.float32 and ws_t.dtype == torch.float32
    assert sorted_ids.dtype == torch.int32 and expert_ids.dtype == torch.int32
    em = sorted_ids.numel()
    rc = lib().r4d_gemm_moe_fp8blk_nt_b16(
        _p(qx), _p(x_scale), _P(device_ptr(wq)), _P(device_ptr(ws_t)), _p(wref), _p(y),
        _p(sorted_ids), _p(expert_ids), _p(num_post_pad), _p(topk_weights), em, mtk, top_k, K,
        N, wv, sk, npw, _P(stream_ptr()))
    check(rc, "r4d_gemm_moe_fp8blk_nt_b16")


def _r4d_fp8_moe_gemm(qx: torch.Tensor, x_scale: torch.Tensor, wq: torch.Tensor,
                      ws_t: torch.Tensor, wref: torch.Tensor | None, sorted_ids: torch.Tensor,
                      expert_ids: torch.Tensor, num_post_pad: torch.Tensor,
                      topk_weights: torch.Tensor | None, mtk: int, top_k: int, wv: int,
                      sk: int, npw: int) -> torch.Tensor:
    """The allocating form the reference's single-call path uses (r4d_mxfp4_moe.py.lru.diff:
    625,635): a new y [mtk, N] bf16. Rows no block of sorted_ids names are left as allocated
    (torch.empty); with one align over every expert, every valid (token, k) row is named."""
    y = torch.empty((mtk, wq.shape[1]), dtype=torch.bfloat16, device=qx.device)
    _r4d_fp8_moe_gemm_into(y, qx, x_scale, wq, ws_t, wref, sorted_ids, expert_ids,
                           num_post_pad, topk_weights, mtk, top_k, wv, sk, npw)
    return y


def moe_gemm_split_act(act: torch.Tensor, qx: torch.Tensor, x_scale: torch.Tensor,
                       w_hot: torch.Tensor, s_hot: torch.Tensor, align_hot, mtk: int, top_k: int,
                       w_cold: torch.Tensor | None = None, s_cold: torch.Tensor | None = None,
                       align_cold=None, wv: int = 0, sk: int = 0) -> None:
    """gate_up of the split GEMM (npw 2) with the SiLU-mul in its epilogue: act [mtk, N/2]
    bf16 equals silu_mul_quant's activation of the [mtk, N] gate_up output, bit for bit, on
    every row the aligns name. align_* = (sorted_ids, expert_ids, num_post_pad); without a
    cold set the hot list runs alone. w_cold / s_cold may be pinned host tensors."""
    N, K = w_hot.shape[1], w_hot.shape[2]
    assert act.shape == (mtk, N // 2) and act.dtype == torch.bfloat16 and act.is_contiguous()
    assert qx.dtype == FP8 and w_hot.dtype == FP8 and qx.shape[1] == K
    sh, eh, nh = align_hot
    sc, ec, nc = align_cold if align_cold is not None else (None, None, None)
    rc = lib().rlu_moe_gemm_split_act(
        _p(qx), _p(x_scale), _p(w_hot), _p(s_hot), _p(sh), _p(eh), _p(nh),
        _P(device_ptr(w_cold)) if w_cold is not None else _P(0),
        _P(device_ptr(s_cold)) if s_cold is not None else _P(0), _p(sc), _p(ec), _p(nc),
        _p(act), sh.numel(), mtk, top_k, K, N, wv, sk, _P(stream_ptr()))
    check(rc, "rlu_moe_gemm_split_act")


def moe_gemm_split_qin(y: torch.Tensor, act: torch.Tensor, w_hot: torch.Tensor,
                       s_hot: torch.Tensor, align_hot, topk_weights: torch.Tensor | None,
                       mtk: int, w_cold: torch.Tensor | None = None,
                       s_cold: torch.Tensor | None = None, align_cold=None) -> None:
    """down of the split GEMM (sk 1) from the bf16 activation [mtk, K]: each workgroup (8
    waves, 256 columns of one block) quantizes its block's rows as silu_mul_quant (group 128)
    does, so y [mtk, N] equals the split GEMM on that kernel's q2 / s2, bit for bit."""
    N, K = w_hot.shape[1], w_hot.shape[2]
    assert y.shape == (mtk, N) and y.dtype == torch.bfloat16 and y.is_contiguous()
    assert act.shape == (mtk, K) and act.dtype == torch.bfloat16 and act.is_contiguous()
    sh, eh, nh = align_hot
    sc, ec, nc = align_cold if align_cold is not None else (None, None, None)
    rc = lib().rlu_moe_gemm_split_qin(
        _p(act), _p(w_hot), _p(s_hot), _p(sh), _p(eh), _p(nh),
        _P(device_ptr(w_cold)) if w_cold is not None else _P(0),
        _P(device_ptr(s_cold)) if s_cold is not None else _P(0), _p(sc), _p(ec), _p(nc),
        _p(topk_weights), _p(y), sh.numel(), mtk, K, N, _P(stream_ptr()))
    check(rc, "rlu_moe_gemm_split_qin")


def gemm_fp8_block_q(qx: torch.Tensor, xs: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor,
                     out: torch.Tensor | None = None, wv: int = 0, npw: int = 0) -> torch.Tensor:
    """e4m3 [M, K] (xs [M, K/128]) x e4m3 [N, K] in fragment order (ws [N/128, K/128])^T ->
    bf16 [M, N], one launch per 16 rows. npw = 0 picks the tile width measured fastest at
    vocab 151936 x 2560: two 16-column tiles per item up to 8 rows, four above."""
    M, K = qx.shape
    N = wq.shape[0]
    assert qx.is_contiguous() and xs.is_contiguous() and xs.shape == (M, K // GROUP)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=qx.device) if out is None else out
    assert y.shape == (M, N) and y.is_contiguous()
    for r0 in range(0, M, 16):
        m = min(M, r0 + 16) - r0
        p = npw if npw else (2 if m <= 8 else 4)
        rc = lib().rlu_gemm_fp8blk_m16(_P(qx[r0].data_ptr()), _P(xs[r0].data_ptr()), _p(wq),
                                       _p(ws), _P(y[r0].data_ptr()), m, N, K, wv, p,
                                       _P(stream_ptr()))
        check(rc, "rlu_gemm_fp8blk_m16")
    return y


def gemm_fp8_block(x: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor) -> torch.Tensor:
    """bf16 [M, K] @ dequant(W)^T -> bf16 [M, N]: group-128 activation quant, then the GEMM
    (kernels/fp8_target_lmhead.py:70-74), 16 rows per launch."""
    qx, xs = fp8_quant_group(x.contiguous(), GROUP)
    return gemm_fp8_block_q(qx, xs, wq, ws)


# decode rows the fp8 head takes; larger batches go to the original method
# (kernels/fp8_target_lmhead.py:31)
FP8_LMHEAD_MAX_M = int(os.environ.get("VLLM_TARGET_FP8_LMHEAD_MAX_M", "64"))


class Fp8TargetHead:
    """Drop-in replacement for the lm_head's quant_method at decode M
    (kernels/fp8_target_lmhead.py:77-93). The weight is packed once (pack_fp8_block). apply()
    runs gemm_fp8_block for bf16 inputs of at most FP8_LMHEAD_MAX_M rows and no bias, and
    hands every other call, and every other attribute, to the original method."""

    def __init__(self, orig_method, weight: torch.Tensor):
        self.orig = orig_method
        self.wq, self.ws = pack_fp8_block(weight)
        self.n_fp8 = 0                              # calls served by the fp8 kernel

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        flat = x.reshape(-1, x.shape[-1])
        if flat.shape[0] > FP8_LMHEAD_MAX_M or bias is not None or x.dtype != torch.bfloat16:
            return self.orig.apply(layer, x, bias=bias)
        y = gemm_fp8_block(flat, self.wq, self.ws)
        self.n_fp8 += 1
        return y.reshape(*x.shape[:-1], y.shape[-1])

    def __getattr__(self, name):
        if name == "orig":                          # not set yet (copy / unpickle)
            raise AttributeError(name)
        return getattr(self.orig, name)


def shuffle_fp8_weight(w: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Row-major e4m3 [..., N, K] -> the same shape in gfx950 fragment order (a permutation
    inside each 16-row strip; stacked experts shuffle as one [E*N, K] matrix)."""
    assert w.dtype == FP8 and w.is_cuda and w.is_contiguous() and w.ndim >= 2
    K = w.shape[-1]
    rows = w.numel() // K
    o = torch.empty_like(w) if out is None else out
    assert o.shape == w.shape and o.dtype == FP8 and o.is_contiguous()
    assert o.data_ptr() != w.data_ptr(), "shuffle is out of place"
    rc = lib().rlu_shuffle_fp8_weight(_p(w), _p(o), rows, K, _P(stream_ptr()))
    check(rc, "rlu_shuffle_fp8_weight")
    return o


@torch.no_grad()
def pack_fp8_block(w: torch.Tensor, rows: int = 4096) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16/fp32 [N, K] -> (e4m3 [N, K] in fragment order, fp32 block scales [N/128, K/128]):
    per 128x128 block scale = max(amax, 1e-12) / 448, q = e4m3(clamp(w / scale, +-448))
    (kernels/fp8_target_lmhead.py:44-66), quantized in row chunks so the fp32 temporaries stay
    small. Each chunk is shuffled straight into the output (the permutation stays inside 16-row
    strips and chunks are whole strips), so the peak is one fp8 weight plus one chunk, not two
    full-size fp8 copies."""
    N, K = w.shape
    assert N % 128 == 0 and K % 128 == 0, (N, K)
    rows = max(128, rows // 128 * 128)
    out = torch.empty((N, K), dtype=FP8, device=w.device)
    ws = torch.empty((N // 128, K // 128), dtype=torch.float32, device=w.device)
    for r0 in range(0, N, rows):
        r1 = min(N, r0 + rows)
        wf = w[r0:r1].float().view((r1 - r0) // 128, 128, K // 128, 128)
        scale = wf.abs().amax(dim=(1, 3), keepdim=True).clamp(min=1e-12) / 448.0
        q = (wf / scale).clamp(-448.0, 448.0).to(FP8).view(r1 - r0, K)
        shuffle_fp8_weight(q, out=out[r0:r1])
        ws[r0 // 128:r1 // 128] = scale.view((r1 - r0) // 128, K // 128)
        del wf, q
    return out, ws


def moe_gemm_tiles(expert_ids: torch.Tensor, num_post_pad: torch.Tensor,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """The tile list of an align output: int32 [2 * nb + 1] = (first block, block count) per
    tile, then the tile count at the end."""
    nb = expert_ids.numel()
    ws = torch.empty(2 * nb + 1, dtype=torch.int32, device=expert_ids.device) if out is None else out
    rc = lib().rlu_moe_gemm_tiles(_p(expert_ids), _p(num_post_pad), nb, _p(ws),
                                  _P(ws.data_ptr() + 8 * nb), _P(stream_ptr()))
    check(rc, "rlu_moe_gemm_tiles")
    return ws


def _tile_list(expert_ids, num_post_pad, tiles, ready):
    if ready:
        assert tiles is not None and tiles.numel() == 2 * expert_ids.numel() + 1 \
            and tiles.dtype == torch.int32, "tiles_ready needs the align's tile list"
        return tiles
    return moe_gemm_tiles(expert_ids, num_post_pad, tiles)


def moe_gemm_tiled(y: torch.Tensor, qx: torch.Tensor, x_scale: torch.Tensor, wq: torch.Tensor,
                   ws_t: torch.Tensor, sorted_ids: torch.Tensor, expert_ids: torch.Tensor,
                   num_post_pad: torch.Tensor, topk_weights: torch.Tensor | None, mtk: int,
                   top_k: int, tiles: torch.Tensor | None = None, wv: int = 0,
                   tiles_ready: bool = False) -> None:
    """_r4d_fp8_moe_gemm_into for prefill-sized inputs: same operands and row contract, one
    workgroup per 128-row x 256-column tile of one expert (bit-identical to the decode kernel
    with sk = 1); N % 256 == 0. `tiles` is an int32 workspace of 2 * expert_ids.numel() + 1
    entries; with tiles_ready it already holds moe_gemm_tiles of this align (computed once and
    shared by the align's GEMMs) and is not rebuilt. wq / ws_t may be pinned host tensors
    (read over the bus, as the cold call's full tensor is)."""
    K = qx.shape[1]
    N = wq.shape[1]
    nb = expert_ids.numel()
    assert y.shape == (mtk, N) and y.dtype == torch.bfloat16 and y.is_contiguous()
    assert qx.dtype == FP8 and wq.dtype == FP8 and wq.shape[2] == K
    tiles = _tile_list(expert_ids, num_post_pad, tiles, tiles_ready)
    rc = lib().rlu_moe_gemm_fp8blk_tiled(
        _p(qx), _p(x_scale), _P(device_ptr(wq)), _P(device_ptr(ws_t)), _p(sorted_ids),
        _p(expert_ids), _p(tiles),
        _P(tiles.data_ptr() + 8 * nb), nb, _p(topk_weights), _p(y), mtk, top_k, K, N, wv,
        _P(stream_ptr()))
    check(rc, "rlu_moe_gemm_fp8blk_tiled")


def moe_gemm_tiled_silu_quant_built(K: int, N: int) -> bool:
    """Whether moe_gemm_tiled_silu_quant has a kernel for gate_up weights [*, N, K] (a
    zero-row call: nothing is launched)."""
    rc = lib().rlu_moe_gemm_fp8blk_tiled_silu_quant(
        *([_P(0)] * 8), 1, _P(0), _P(0), 0, 1, K, N, _P(0))
    return rc == 0


def moe_gemm_tiled_silu_quant(q2: torch.Tensor, s2: torch.Tensor, qx: torch.Tensor,
                              x_scale: torch.Tensor, wq: torch.Tensor, ws_t: torch.Tensor,
                              sorted_ids: torch.Tensor, expert_ids: torch.Tensor,
                              num_post_pad: torch.Tensor, mtk: int, top_k: int,
                              tiles: torch.Tensor | None = None,
                              tiles_ready: bool = False) -> None:
    """moe_gemm_tiled of gate_up followed by silu_mul_quant (group 128) in one kernel: q2
    [mtk, N/2] e4m3 and s2 [mtk, N/256] f32 equal silu_mul_quant(moe_gemm_tiled(...)) bit for
    bit, rows the align does not name untouched. Raises for shapes without a kernel
    (moe_gemm_tiled_silu_quant_built). tiles / tiles_ready as for moe_gemm_tiled."""
    K = qx.shape[1]
    N = wq.shape[1]
    nb = expert_ids.numel()
    assert q2.shape == (mtk, N // 2) and q2.dtype == FP8 and q2.is_contiguous()
    assert s2.shape == (mtk, N // 256) and s2.dtype == torch.float32 and s2.is_contiguous()
    assert qx.dtype == FP8 and wq.dtype == FP8 and wq.shape[2] == K
    tiles = _tile_list(expert_ids, num_post_pad, tiles, tiles_ready)
    rc = lib().rlu_moe_gemm_fp8blk_tiled_silu_quant(
        _p(qx), _p(x_scale), _P(device_ptr(wq)), _P(device_ptr(ws_t)), _p(sorted_ids),
        _p(expert_ids), _p(tiles), _P(tiles.data_ptr() + 8 * nb), nb, _p(q2), _p(s2), mtk,
        top_k, K, N, _P(stream_ptr()))
    check(rc, "rlu_moe_gemm_fp8blk_tiled_silu_quant")


# ---- two aligns in one launch: a layer's resident slots (align 0) and its full tensor --------
def moe_gemm_tiles_split(al0, al1, out: torch.Tensor | None = None) -> torch.Tensor:
    """The tile list of two aligns, al = (expert_ids, num_post_pad): int32 [2 (nb0 + nb1) + 1]
    = align 0's tiles (first block, block count), then align 1's with bit 16 of the block
    count set, then the tile count at the end."""
    (e0, n0), (e1, n1) = al0, al1
    nb = e0.numel() + e1.numel()
    ws = torch.empty(2 * nb + 1, dtype=torch.int32, device=e0.device) if out is None else out
    assert ws.numel() == 2 * nb + 1 and ws.dtype == torch.int32
    rc = lib().rlu_moe_gemm_tiles_split(_p(e0), _p(n0), e0.numel(), _p(e1), _p(n1), e1.numel(),
                                        _p(ws), _P(ws.data_ptr() + 8 * nb), _P(stream_ptr()))
    check(rc, "rlu_moe_gemm_tiles_split")
    return ws


def _split_tiles(al0, al1, tiles, ready):
    nb = al0[1].numel() + al1[1].numel()
    if ready:
        assert tiles is not None and tiles.numel() == 2 * nb + 1 and tiles.dtype == torch.int32, \
            "tiles_ready needs the aligns' split tile list"
        return tiles, nb
    return moe_gemm_tiles_split(al0[1:], al1[1:], tiles), nb


def moe_gemm_tiled_split_built(K: int, N: int) -> bool:
    """Whether moe_gemm_tiled_split has a kernel for weights [*, N, K] (a zero-row call:
    nothing is launched)."""
    rc = lib().rlu_moe_gemm_fp8blk_tiled_split(*([_P(0)] * 12), 1, _P(0), _P(0), 0, 1, K, N,
                                               _P(0))
    return rc == 0


def moe_gemm_tiled_split(y: torch.Tensor, qx: torch.Tensor, x_scale: torch.Tensor,
                         w0: torch.Tensor, s0: torch.Tensor, al0, w1: torch.Tensor,
                         s1: torch.Tensor, al1, topk_weights: torch.Tensor | None, mtk: int,
                         top_k: int, tiles: torch.Tensor | None = None,
                         tiles_ready: bool = False) -> None:
    """moe_gemm_tiled over two aligns in one launch of the streamed kernel: al0 = (sorted_ids,
    expert_ids, num_post_pad) over weights w0 / s0 (a layer's resident slots) and al1 over w1 /
    s1 (its full tensor, device or pinned host memory), both indexing the rows of qx and
    writing y. Equals moe_gemm_tiled on each align bit for bit. Raises for shapes without a
    kernel (moe_gemm_tiled_split_built). tiles: int32 workspace of 2 (nb0 + nb1) + 1 entries;
    with tiles_ready it holds moe_gemm_tiles_split of these aligns and is not rebuilt."""
    K = qx.shape[1]
    N = w0.shape[1]
    assert y.shape == (mtk, N) and y.dtype == torch.bfloat16 and y.is_contiguous()
    assert qx.dtype == FP8 and w0.dtype == FP8 and w1.dtype == FP8
    assert w0.shape[1:] == (N, K) and w1.shape[1:] == (N, K)
    tiles, nb = _split_tiles(al0, al1, tiles, tiles_ready)
    rc = lib().rlu_moe_gemm_fp8blk_tiled_split(
        _p(qx), _p(x_scale), _P(device_ptr(w0)), _P(device_ptr(s0)), _p(al0[0]), _p(al0[1]),
        _P(device_ptr(w1)), _P(device_ptr(s1)), _p(al1[0]), _p(al1[1]), _p(tiles),
        _P(tiles.data_ptr() + 8 * nb), nb, _p(topk_weights), _p(y), mtk, top_k, K, N,
        _P(stream_ptr()))
    check(rc, "rlu_moe_gemm_fp8blk_tiled_split")


def moe_gemm_tiled_split_silu_quant(q2: torch.Tensor, s2: torch.Tensor, qx: torch.Tensor,
                                    x_scale: torch.Tensor, w0: torch.Tensor, s0: torch.Tensor,
                                    al0, w1: torch.Tensor, s1: torch.Tensor, al1, mtk: int,
                                    top_k: int, tiles: torch.Tensor | None = None,
                                    tiles_ready: bool = False) -> None:
    """moe_gemm_tiled_silu_quant over two aligns in one launch, as moe_gemm_tiled_split:
    equals moe_gemm_tiled_silu_quant on each align bit for bit."""
    K = qx.shape[1]
    N = w0.shape[1]
    assert q2.shape == (mtk, N // 2) and q2.dtype == FP8 and q2.is_contiguous()
    assert s2.shape == (mtk, N // 256) and s2.dtype == torch.float32 and s2.is_contiguous()
    assert qx.dtype == FP8 and w0.dtype == FP8 and w1.dtype == FP8
    assert w0.shape[1:] == (N, K) and w1.shape[1:] == (N, K)
    tiles, nb = _split_tiles(al0, al1, tiles, tiles_ready)
    rc = lib().rlu_moe_gemm_fp8blk_tiled_split_silu_quant(
        _p(qx), _p(x_scale), _P(device_ptr(w0)), _P(device_ptr(s0)), _p(al0[0]), _p(al0[1]),
        _P(device_ptr(w1)), _P(device_ptr(s1)), _p(al1[0]), _p(al1[1]), _p(tiles),
        _P(tiles.data_ptr() + 8 * nb), nb, _p(q2), _p(s2), mtk, top_k, K, N, _P(stream_ptr()))
    check(rc, "rlu_moe_gemm_fp8blk_tiled_split_silu_quant")


NOALLOC_MAX_BLOCKS = 8192      # the scratch tile list's capacity (131072 sorted ids)


def moe_gemm_tiled_noalloc(y: torch.Tensor, qx: torch.Tensor, x_scale: torch.Tensor,
                           wq: torch.Tensor, ws_t: torch.Tensor, sorted_ids: torch.Tensor,
                           expert_ids: torch.Tensor, num_post_pad: torch.Tensor,
                           topk_weights: torch.Tensor | None, mtk: int, top_k: int,
                           wv: int = 0) -> None:
    """moe_gemm_tiled with no workspace and no allocation: the tile list lives in the
    library's per-device scratch array. Calls that overlap on one GPU race on it."""
    K = qx.shape[1]
    N = wq.shape[1]
    nb = expert_ids.numel()
    assert y.shape == (mtk, N) and y.dtype == torch.bfloat16 and y.is_contiguous()
    assert qx.dtype == FP8 and wq.dtype == FP8 and wq.shape[2] == K
    if nb > NOALLOC_MAX_BLOCKS:
        raise ValueError(f"moe_gemm_tiled_noalloc: {nb} blocks exceed the scratch tile list "
                         f"({NOALLOC_MAX_BLOCKS} blocks)")
    rc = lib().rlu_moe_gemm_fp8blk_tiled_noalloc(
        _p(qx), _p(x_scale), _P(device_ptr(wq)), _P(device_ptr(ws_t)), _p(sorted_ids),
        _p(expert_ids), _p(num_post_pad), nb, _p(topk_weights), _p(y), mtk, top_k, K, N, wv,
        _P(stream_ptr()))
    check(rc, "rlu_moe_gemm_fp8blk_tiled_noalloc")


# ---- torch custom ops at the reference's names and schemas ----------------------------------
# r4d_mxfp4_moe_gemm_into / r4d_mxfp4_moe_gemm: patches/.../r4d_mxfp4_moe.py.lru.diff:363-423
# (mutates_args=["y"], a fake impl) and the allocating call sites :625,635. Registered in the
# namespace the LRU ops use ("vllm" when vLLM is importable, else "rlu").
def _register():
    from .lru import OPS_NAMESPACE
    lib_ = torch.library.Library(OPS_NAMESPACE, "FRAGMENT")
    args = ("Tensor qx, Tensor x_scale, Tensor wq, Tensor ws_t, Tensor? wref, "
            "Tensor sorted_ids, Tensor expert_ids, Tensor num_post_pad, "
            "Tensor? topk_weights, int mtk, int top_k, int wv, int sk, int npw")
    lib_.define(f"r4d_mxfp4_moe_gemm_into(Tensor(a!) y, {args}) -> ()")
    lib_.define(f"r4d_mxfp4_moe_gemm({args}) -> Tensor")
    lib_.impl("r4d_mxfp4_moe_gemm_into", _r4d_fp8_moe_gemm_into, "CUDA")
    lib_.impl("r4d_mxfp4_moe_gemm", _r4d_fp8_moe_gemm, "CUDA")
    lib_.impl("r4d_mxfp4_moe_gemm_into", lambda *a, **k: None, "Meta")
    lib_.impl("r4d_mxfp4_moe_gemm",
              lambda qx, xs, wq, *a: torch.empty((a[6], wq.shape[1]), dtype=torch.bfloat16,
                                                  device=qx.device), "Meta")
    return lib_


_OPS_LIB = _register()
