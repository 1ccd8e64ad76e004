"""W4 (int4 group-128, asymmetric) quantizer, layout and GEMV reference (test infrastructure).

This build's W4 format stores w ~ scale * (q - zero) per (row, 128-column group) with a bf16
scale and an integer zero, where the reference stored an f16 scale (kernels/draft_w4_lmhead.py:
31-50, quantize_w4 :154-198). The quantizer is this build's own: the reference's codes are not
reachable with a bf16 scale, and its module imports vLLM (absent), so the reference's exact
codes stay parity unpinned; the format and the kernel are pinned against this restatement.

Functions and what pins them (tests/test_oracle_w4.py):
  quantize_w4()  per (row, group) with range width = hi - lo and centre mid = (lo + hi) / 2:
                 for each fraction f of FRACTIONS (1.0 down to 0.55), scale s = bf16(f * width
                 / 15), centred zero z0 = rint(7.5 - mid / s), and each zero z of z0, z0 - 1,
                 z0 + 1 (clamped to +-1024): codes q = clamp(rint(w / s) + z, 0, 15), error =
                 sum of ((q - z) s - w)^2 summed in ERR_ORDER; the first candidate with the
                 least error wins. A constant group (width 0) stores s = bf16(|v|), z = 1 for a
                 negative v and 0 otherwise (an all-zero group: s = 0, z = 0, codes 0). Every
                 operation is one float32 rounding, as the packing kernel computes it.
                 Pinned by closed forms (each code is the nearest grid point of its (s, z) unless
                 clamped; each constant group decodes to bf16(v)), by brute force (the chosen
                 candidate has the least float64 error of all 30, up to float32 rounding), and
                 by the error level on Gaussian weights: plain min/max at the textbook ~0.104
                 sigma RMS of a 16-level grid over the ~5.4 sigma range of 128 samples, the
                 search below it.
  ERR_ORDER      lane l = 16 c + r of the tile's wave holds row r's 32 values k = 32 i + 8 c + j
                 (i, j ascending, the order they sit in its packed dwords); each lane sums its 32
                 squared errors in that order, then the four lanes of a row combine as
                 (p_0 + p_1) + (p_2 + p_3) -- every lane of the row gets the same float.
  pack_codes() / unpack_codes() / pack_sz()  this build's layout: [N/16][K/128][64 lanes][16 B],
                 lane 16 c + r = row r, dword i = 32-deep step i, k = 128 g + 32 i + 8 c + j,
                 nibble t of the low half = j 2t, nibble t of the high half = j 2t + 1; sz =
                 bf16 scale bits | int16 zero << 16. Pinned by a byte-by-byte walk of the formula.
  gemv()         float64 x . (scale (q - zero))^T, pinned against pure-Python loops.
"""
from __future__ import annotations

import numpy as np

from . import fp8

GROUP = 128
# clip fractions of the group's range, by their float32 bits (1.0, 0.95, ..., 0.55)
FRACTION_BITS = (0x3F800000, 0x3F733333, 0x3F666666, 0x3F59999A, 0x3F4CCCCD,
                 0x3F400000, 0x3F333333, 0x3F266666, 0x3F19999A, 0x3F0CCCCD)
FRACTIONS = tuple(np.uint32(b).view(np.float32) for b in FRACTION_BITS)
ZERO_SHIFTS = (0, -1, 1)
ZMAX = 1024


def _lanes(w: np.ndarray, group: int) -> np.ndarray:
    """[N, K] -> [N, G, 4 (c), 32 (i, j)]: the values each lane of a tile's wave holds."""
    n, k = w.shape
    return w.reshape(n, k // group, 4, 4, 8).transpose(0, 1, 3, 2, 4).reshape(n, k // group, 4, 32)


def _unlanes(t: np.ndarray) -> np.ndarray:
    n, g = t.shape[:2]
    return t.reshape(n, g, 4, 4, 8).transpose(0, 1, 3, 2, 4).reshape(n, g * 128)


def lane_error(d2: np.ndarray) -> np.ndarray:
    """Sum [.., 4, 32] float32 squared errors in ERR_ORDER -> [..] float32."""
    p = d2[..., 0].copy()
    for m in range(1, 32):
        p = p + d2[..., m]
    return (p[..., 0] + p[..., 1]) + (p[..., 2] + p[..., 3])


def quantize_w4(w: np.ndarray, group: int = GROUP, fractions=None, shifts=None):
    """[N, K] -> (q uint8 [N, K], scale float32 (bf16 values) [N, G], zero int16 [N, G])."""
    assert group == GROUP
    w = np.asarray(w, np.float32)
    n, k = w.shape
    t = _lanes(w, group)
    lo = w.reshape(n, k // group, group).min(-1)
    hi = w.reshape(n, k // group, group).max(-1)
    width = hi - lo
    mid = (lo + hi) / np.float32(2)
    best_err = np.full(lo.shape, np.inf, np.float32)
    best_s = np.zeros(lo.shape, np.float32)
    best_z = np.zeros(lo.shape, np.float32)
    best_q = np.zeros(t.shape, np.float32)
    for f in (FRACTIONS if fractions is None else fractions):
        s = fp8.bf16_round((np.float32(f) * width) / np.float32(15))
        ok = (s > 0) & (width > 0)
        ss = np.where(ok, s, np.float32(1))
        u = np.rint(t / ss[..., None, None])
        z0 = np.clip(np.rint(np.float32(7.5) - mid / ss), -ZMAX, ZMAX)
        for dz in (ZERO_SHIFTS if shifts is None else shifts):
            z = np.clip(z0 + np.float32(dz), -ZMAX, ZMAX)
            q = np.clip(u + z[..., None, None], 0, 15)
            d = (q - z[..., None, None]) * ss[..., None, None] - t
            err = np.where(ok, lane_error(d * d), np.float32(np.inf))
            take = err < best_err
            best_err = np.where(take, err, best_err)
            best_s = np.where(take, s, best_s)
            best_z = np.where(take, z, best_z)
            best_q = np.where(take[..., None, None], q, best_q)
    # constant groups
    const = width == 0
    sc = fp8.bf16_round(np.abs(lo))
    zc = np.where(lo < 0, np.float32(1), np.float32(0))
    scs = np.where(sc > 0, sc, np.float32(1))
    qc = np.where((sc > 0)[..., None, None],
                  np.clip(np.rint(t / scs[..., None, None]) + zc[..., None, None], 0, 15),
                  np.float32(0))
    best_s = np.where(const, sc, best_s)
    best_z = np.where(const, np.where(sc > 0, zc, np.float32(0)), best_z)
    best_q = np.where(const[..., None, None], qc, best_q)
    return (_unlanes(best_q).astype(np.uint8), best_s.astype(np.float32),
            best_z.astype(np.int16))


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
