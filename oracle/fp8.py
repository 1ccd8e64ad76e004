"""Bit-exact float32 <-> OCP e4m3fn and the quantizers of the path (test infrastructure only).

Functions and what pins them (tests/test_oracle_quant.py):
  e4m3_table()      the 256 code values, from the format definition (1-4-3, bias 7, no inf,
                    S.1111.111 = NaN, max 448). Pinned against torch's float8_e4m3fn cast of
                    every code.
  f32_to_e4m3()     round-to-nearest-even encoder, built from the bit layout. Pinned against
                    torch's float32 -> float8_e4m3fn cast on every rounding midpoint of every
                    binade, random values and special cases.
  exp_f32()         e^x in float32 by Cody-Waite reduction (x = n ln2 + r, ln2 split in a
                    hi/lo pair) and the degree-7 Taylor polynomial of e^r, every operation
                    rounded separately. The device uses the same operation sequence, so both
                    sides agree bit for bit. Pinned against math.exp (<= 2 ulp over the range).
  silu_mul_quant()  kernels/fused_silu_mul_quant.py:43-57: s = bf16(g / (1 + exp(-g))),
                    a = bf16(float(s) * u), per-group amax of a, scale = max(amax / 448,
                    1 / (448 * 512)), q = e4m3(clamp(a / scale, +-448)) -- divide, not a
                    reciprocal multiply. group = 0 is the reference's per-token form; group =
                    128 is this path's per-token-group-128 form (same rules per group).
                    Pinned: the zero row lands on 1/(448*512) = 4.35965e-06
                    (docs/PATCHES.md:916-921); every q is the nearest e4m3 to a/scale;
                    dequantized error bounded by half an e4m3 ulp.
  group_quant()     per-token-group-128 activation quant (A9): the same scale and rounding rules
                    as silu_mul_quant applied to x directly. The exact eps/floor convention of
                    vLLM's per_token_group_quant_fp8 is parity unpinned (vLLM is absent); this is
                    the convention of this path, documented and pinned by its own fixtures.
  block_quant_weight()  kernels/fp8_target_lmhead.py:57-64: per 128x128 block, scale =
                    clamp(amax, 1e-12) / 448, wq = e4m3(clamp(w / scale, +-448)).
  shuffle_weight() / unshuffle_weight()  the gfx950 MFMA fragment order of the weight bytes
                    (the counterpart of shuffle_weight_gfx1201, kernels/fp8_target_lmhead.py:
                    47,64): byte (n, k), n = 16 nt + r, k = 128 kb + 64 h + 16 c + j, at
                    ((nt (K/128) + kb) 2 + h) 1024 + (16 c + r) 16 + j. Pinned by a brute-force
                    walk of that formula over every byte (as tests/k3/test_layout.py:1-31 pins
                    the gfx1201 layout) and by unshuffle(shuffle(w)) == w.
"""
from __future__ import annotations

import numpy as np

E4M3_MAX = np.float32(448.0)
MIN_SCALE = np.float32(1.0) / (np.float32(448.0) * np.float32(512.0))


def e4m3_table() -> np.ndarray:
    """float32 value of each of the 256 e4m3fn codes (NaN for 0x7f / 0xff)."""
    out = np.empty(256, np.float32)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 0x7
        if e == 0xF and m == 0x7:
            out[c] = np.nan
        elif e == 0:
            out[c] = s * (m / 8.0) * 2.0 ** -6
        else:
            out[c] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return out


_TABLE = e4m3_table()


def e4m3_to_f32(q: np.ndarray) -> np.ndarray:
    return _TABLE[np.asarray(q, np.uint8)]


def f32_to_e4m3(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> e4m3fn code (uint8). Overflow and NaN give NaN
    (0x7f | sign), as torch's cast does; callers clamp to +-448 first."""
    x = np.ascontiguousarray(np.asarray(x, np.float32))
    bits = x.view(np.uint32).astype(np.uint64)
    sign = ((bits >> 31) & 1).astype(np.uint8) << 7
    exp32 = ((bits >> 23) & 0xFF).astype(np.int64)
    man = bits & 0x7FFFFF
    full = man | 0x800000                       # implicit one (float32 normals)
    e = exp32 - 127                             # unbiased exponent
    code = np.zeros(x.shape, np.int64)
    # normal targets: e >= -6 -> keep 3 mantissa bits of 23
    norm = (exp32 != 0) & (e >= -6)
    q = (man >> 20).astype(np.int64)
    rem = (man & 0xFFFFF).astype(np.int64)
    up = (rem > 0x80000) | ((rem == 0x80000) & ((q & 1) == 1))
    q = q + up
    E = e + 7 + (q >> 3)
    q = q & 7
    code = np.where(norm, (E << 3) | q, code)
    over = norm & ((E > 15) | ((E == 15) & (q == 7)))
    # subnormal targets: value in units of 2^-9 = full * 2^(e - 23 + 9)
    sub = (exp32 != 0) & (e < -6)
    shift = np.clip(23 - 9 - e, 1, 63).astype(np.uint64)   # >= 21 here
    qs = (full >> shift).astype(np.int64)
    rems = (full & ((np.uint64(1) << shift) - np.uint64(1))).astype(np.int64)
    half = (np.uint64(1) << (shift - np.uint64(1))).astype(np.int64)
    ups = (rems > half) | ((rems == half) & ((qs & 1) == 1))
    qs = qs + ups
    code = np.where(sub, qs, code)              # qs == 8 is the smallest normal, 0x08
    nan = np.isnan(x) | over | (exp32 == 255)
    code = np.where(nan, 0x7F, code)
    return (code.astype(np.uint8) | sign)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest-even bfloat16, returned as float32."""
    b = np.ascontiguousarray(np.asarray(x, np.float32)).view(np.uint32).astype(np.uint64)
    nan = np.isnan(np.asarray(x, np.float32))
    lsb = (b >> 16) & 1
    r = ((b + 0x7FFF + lsb) >> 16) << 16
    out = (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    return np.where(nan, np.float32(np.nan), out).astype(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bits_to_f32(b16: np.ndarray) -> np.ndarray:
    return (np.asarray(b16, np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---- e^x: Cody-Waite + Taylor, every operation rounded separately (float32) ----------------
_LOG2E = np.float32(1.44269504)
_LN2_HI = np.float32(0.693145752)          # 0x3f317200: the top bits of ln 2 (exact * n)
_LN2_LO = np.float32(1.42860677e-06)       # ln 2 - _LN2_HI
_TAYLOR = [np.float32(1.0 / f) for f in (5040.0, 720.0, 120.0, 24.0, 6.0, 2.0, 1.0, 1.0)]


def exp_f32(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, np.float32)
    with np.errstate(over="ignore", invalid="ignore", under="ignore"):
        n = np.rint(np.float32(x * _LOG2E)).astype(np.float32)
        r = np.float32(x - np.float32(n * _LN2_HI))
        r = np.float32(r - np.float32(n * _LN2_LO))
        p = _TAYLOR[0]
        for c in _TAYLOR[1:]:
            p = np.float32(np.float32(p * r) + c)
        ni = np.clip(n, -200, 200).astype(np.int32)
        # 2^n in two steps so that n down to -149 and up to 127 stays exact
        h = ni // 2
        out = np.float32(np.float32(p * np.ldexp(np.float32(1), h).astype(np.float32))
                         * np.ldexp(np.float32(1), ni - h).astype(np.float32))
    out = np.where(x > np.float32(88.7228394), np.float32(np.inf), out)
    out = np.where(x < np.float32(-103.972076), np.float32(0.0), out)
    return np.where(np.isnan(x), x, out).astype(np.float32)


def silu_bf16(g: np.ndarray) -> np.ndarray:
    """bf16(g / (1 + exp(-g))) with float32 arithmetic, as float32."""
    g = np.asarray(g, np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        s = np.float32(g / np.float32(np.float32(1.0) + exp_f32(-g)))
    return bf16_round(s)


def _group_scale(a: np.ndarray, group: int) -> tuple[np.ndarray, int]:
    rows, d = a.shape
    gs = d if group == 0 else group
    assert d % gs == 0
    amax = np.abs(a).reshape(rows, d // gs, gs).max(-1).astype(np.float32)
    scale = np.maximum(np.float32(amax / E4M3_MAX), MIN_SCALE).astype(np.float32)
    return scale, gs


def quant_with_scale(a: np.ndarray, scale: np.ndarray, gs: int) -> np.ndarray:
    rows, d = a.shape
    s = np.repeat(scale, gs, axis=1)
    v = np.clip(np.float32(a / s), -E4M3_MAX, E4M3_MAX).astype(np.float32)
    return f32_to_e4m3(v)


def group_quant(x: np.ndarray, group: int = 128) -> tuple[np.ndarray, np.ndarray]:
    """x float32 (holding bf16 values) [rows, K] -> (q uint8 [rows, K], scale f32
    [rows, K/group]); group = 0 -> one scale per row."""
    a = np.asarray(x, np.float32)
    scale, gs = _group_scale(a, group)
    return quant_with_scale(a, scale, gs), scale


def silu_mul_quant(x: np.ndarray, group: int = 128):
    """x float32 (holding bf16 values) [rows, 2d] -> (act bf16-as-f32 [rows, d],
    q uint8 [rows, d], scale f32 [rows, d/group or 1])."""
    x = np.asarray(x, np.float32)
    d = x.shape[1] // 2
    g, u = x[:, :d], x[:, d:]
    s = silu_bf16(g)
    act = bf16_round(np.float32(s * u))
    scale, gs = _group_scale(act, group)
    return act, quant_with_scale(act, scale, gs), scale


def block_quant_weight(w: np.ndarray, blk: int = 128) -> tuple[np.ndarray, np.ndarray]:
    """w float32 [N, K] -> (wq uint8 [N, K], ws f32 [N/blk, K/blk])."""
    w = np.asarray(w, np.float32)
    N, K = w.shape
    assert N % blk == 0 and K % blk == 0
    b = w.reshape(N // blk, blk, K // blk, blk)
    amax = np.maximum(np.abs(b).max(axis=(1, 3)), np.float32(1e-12)).astype(np.float32)
    ws = np.float32(amax / E4M3_MAX).astype(np.float32)
    v = np.clip(np.float32(b / ws[:, None, :, None]), -E4M3_MAX, E4M3_MAX).astype(np.float32)
    return f32_to_e4m3(v).reshape(N, K), ws


def dequant_weight(wq: np.ndarray, ws: np.ndarray, blk: int = 128) -> np.ndarray:
    """e4m3 [N, K] x its [N/blk, K/blk] block scales -> float32 (one product per weight)."""
    v = e4m3_to_f32(wq)
    N, K = v.shape
    b = v.reshape(N // blk, blk, K // blk, blk)
    b *= np.asarray(ws, np.float32)[:, None, :, None]
    return v


def dequant_act(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    v = e4m3_to_f32(q)
    gs = v.shape[1] // scale.shape[1]
    return v * np.repeat(scale, gs, 1)


def shuffle_weight(w: np.ndarray) -> np.ndarray:
    """uint8 [..., N, K] row-major -> the same shape in fragment order."""
    *lead, N, K = w.shape
    assert N % 16 == 0 and K % 128 == 0
    v = np.ascontiguousarray(w).reshape(-1, N // 16, 16, K // 128, 2, 4, 16)
    # (e, nt, r, kb, h, c, j) -> (e, nt, kb, h, c, r, j)
    return np.ascontiguousarray(v.transpose(0, 1, 3, 4, 5, 2, 6)).reshape(w.shape)


def unshuffle_weight(s: np.ndarray) -> np.ndarray:
    """Inverse of shuffle_weight."""
    *lead, N, K = s.shape
    v = np.ascontiguousarray(s).reshape(-1, N // 16, K // 128, 2, 4, 16, 16)
    # (e, nt, kb, h, c, r, j) -> (e, nt, r, kb, h, c, j)
    return np.ascontiguousarray(v.transpose(0, 1, 5, 2, 3, 4, 6)).reshape(s.shape)
