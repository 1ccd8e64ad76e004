"""W4 (int4 group-128, asymmetric) quantizer, layout and GEMV reference (test infrastructure).

Functions and what pins them (tests/test_oracle_w4.py):
  quantize_w4()  kernels/draft_w4_lmhead.py:154-198 restated in numpy float32, with the scale
                 rounded to bf16 (this build's format) where the reference rounds to f16: per
                 (row, group) and clip fraction c of the reference grid (:151), scale =
                 bf16((hi_c - lo_c) / 15), a constant nonzero group gets bf16(|lo| / 7) and zero
                 8, zero = round(-lo_c / scale) clamped to +-1024, q = clamp(round(w / scale +
                 zero), 0, 15), the least squared error wins. Pinned by closed forms: every
                 code is the nearest grid point of its (scale, zero) unless clamped; the chosen
                 clip has the least error of the grid (brute force in float64); plain min/max
                 on Gaussian weights lands at the textbook ~0.104 sigma RMS error the reference
                 quotes (:143-150). The reference's exact codes (f16 scale) are parity unpinned:
                 its module imports vLLM, which is absent.
  pack_codes() / unpack_codes() / pack_sz()  this build's layout: [N/16][K/128][64 lanes][16 B],
                 lane 16 c + r = row r, dword i = 32-deep step i, k = 128 g + 32 i + 8 c + j,
                 nibble t of the low half = j 2t, nibble t of the high half = j 2t + 1; sz =
                 bf16 scale bits | int16 zero << 16. Pinned by a byte-by-byte walk of the formula.
  gemv()         float64 x . (scale (q - zero))^T, pinned against pure-Python loops.
"""
from __future__ import annotations

import numpy as np

from . import fp8

CLIP_GRID = (1.0, 0.95, 0.9, 0.85, 0.8, 0.75, 0.7, 0.65, 0.6)
GROUP = 128


def quantize_w4(w: np.ndarray, group: int = GROUP, clip_grid=None):
    """[N, K] -> (q uint8 [N, K], scale float32 (bf16 values) [N, G], zero int16 [N, G])."""
    w = np.asarray(w, np.float32)
    n, k = w.shape
    wf = w.reshape(n, k // group, group)
    lo, hi = wf.min(-1), wf.max(-1)
    f = np.float32
    mid, half = (hi + lo) / f(2), (hi - lo) / f(2)
    best_err = np.full(lo.shape, np.inf, np.float32)
    best_scale = np.zeros(lo.shape, np.float32)
    best_zero = np.zeros(lo.shape, np.float32)
    for c in (clip_grid if clip_grid is not None else CLIP_GRID):
        c = f(c)
        lo_c, hi_c = mid - c * half, mid + c * half
        scale = fp8.bf16_round(np.maximum((hi_c - lo_c) / f(15.0), f(0.0)))
        flat = (scale == 0) & (lo != 0)
        scale = np.where(flat, fp8.bf16_round(np.abs(lo) / f(7.0)), scale).astype(np.float32)
        with np.errstate(divide="ignore"):
            inv = np.where(scale > 0, f(1.0) / np.maximum(scale, f(1e-30)), f(0.0)).astype(np.float32)
        zero = np.clip(np.where(flat, f(8.0), np.round(-lo_c * inv)), -1024, 1024).astype(np.float32)
        q = np.clip(np.round(wf * inv[..., None] + zero[..., None]), 0, 15).astype(np.float32)
        err = np.square((q - zero[..., None]) * scale[..., None] - wf).sum(-1, dtype=np.float32)
        take = err < best_err
        best_err = np.where(take, err, best_err)
        best_scale = np.where(take, scale, best_scale)
        best_zero = np.where(take, zero, best_zero)
    with np.errstate(divide="ignore"):
        inv = np.where(best_scale > 0, f(1.0) / np.maximum(best_scale, f(1e-30)), f(0.0)).astype(np.float32)
    q = np.clip(np.round(wf * inv[..., None] + best_zero[..., None]), 0, 15)
    return q.astype(np.uint8).reshape(n, k), best_scale, best_zero.astype(np.int16)


def dequant(q: np.ndarray, scale: np.ndarray, zero: np.ndarray, group: int = GROUP) -> np.ndarray:
    n, k = q.shape
    v = (q.reshape(n, k // group, group).astype(np.float64) - zero[..., None].astype(np.float64))
    return (v * scale[..., None].astype(np.float64)).reshape(n, k)


def pack_codes(q: np.ndarray) -> np.ndarray:
    """[N, K] codes -> uint8 [N/16, K/128, 64, 16], by walking the layout formula."""
    n, k = q.shape
    out = np.zeros((n // 16, k // 128, 64, 16), np.uint8)
    lo_j, hi_j = (0, 4, 1, 5), (2, 6, 3, 7)
    for c in range(4):
        for r in range(16):
            for i in range(4):
                for b in range(4):
                    kl = np.arange(k // 128) * 128 + 32 * i + 8 * c
                    rows = np.arange(n // 16) * 16 + r
                    lo = q[rows[:, None], (kl + lo_j[b])[None, :]]
                    hi = q[rows[:, None], (kl + hi_j[b])[None, :]]
                    out[:, :, 16 * c + r, 4 * i + b] = lo | (hi << 4)
    return out


def pack_sz(scale: np.ndarray, zero: np.ndarray) -> np.ndarray:
    n, g = scale.shape
    sb = fp8.bf16_bits(scale).astype(np.uint32)
    zb = (zero.astype(np.int32).astype(np.uint32) & 0xFFFF) << 16
    return (sb | zb).view(np.int32).reshape(n // 16, 16, g).transpose(0, 2, 1).copy()


def unpack(wq: np.ndarray, sz: np.ndarray, n: int, k: int) -> tuple[np.ndarray, ...]:
    """Packed bytes -> (q [N_pad, K], scale [N_pad, G] float32, zero [N_pad, G] int16)."""
    nt, g = wq.shape[0], wq.shape[1]
    q = np.zeros((nt * 16, g * 128), np.uint8)
    lo_j, hi_j = (0, 4, 1, 5), (2, 6, 3, 7)
    for c in range(4):
        for r in range(16):
            for i in range(4):
                for b in range(4):
                    byte = wq[:, :, 16 * c + r, 4 * i + b]
                    kl = np.arange(g) * 128 + 32 * i + 8 * c
                    rows = np.arange(nt) * 16 + r
                    q[rows[:, None], (kl + lo_j[b])[None, :]] = byte & 0xF
                    q[rows[:, None], (kl + hi_j[b])[None, :]] = byte >> 4
    d = sz.transpose(0, 2, 1).reshape(nt * 16, g).view(np.uint32)
    scale = fp8.bits_to_f32((d & 0xFFFF).astype(np.uint16))
    zero = (d >> 16).astype(np.uint16).view(np.int16)
    return q, scale, zero


def gemv(x: np.ndarray, q: np.ndarray, scale: np.ndarray, zero: np.ndarray) -> np.ndarray:
    """float64 x [M, K] . dequant [N, K]^T -> [M, N]."""
    return np.asarray(x, np.float64) @ dequant(q, scale, zero).T
