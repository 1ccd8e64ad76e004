"""W4 draft lm_head: int4 group-128 weights, bf16 activations, bf16 logits, on librlu.so.

Mirrors kernels/draft_w4_lmhead.py: PackedW4 (:63-76), quantize_w4 (:154-198), pack_w4a16
(:228-259), unpack_w4 (:262-285), gemm_w4a16 (:393-403), in this build's gfx950 format:

  codes  q in 0..15 per weight, w ~ scale * (q - zero) per (row, 128-column group), asymmetric,
         the integer zero in [-1024, 1024] (a constant or all-positive group needs one outside
         0..15), the scale rounded to bf16 BEFORE the codes are chosen so the packed weight is
         exactly what the kernel reads, the clip fraction chosen per (row, group) by squared
         error over the reference's grid (:151).
  wq     uint8 [N_pad/16, K/128, 64, 16]: the 1 KB of a 16-row x 128-deep tile in
         v_mfma_f32_16x16x32_bf16 B-operand order (lane 16 c + r holds row r, four dwords, one
         per 32-deep step i, k = 128 g + 32 i + 8 c + j; nibble t of the low half is j = 2t,
         nibble t of the high half is j = 2t + 1).
  sz     int32 [N_pad/16, K/128, 16]: bf16 scale bits | int16 zero << 16.

The reference stores an f16 scale and widens bf16 activations to f16 for its gfx1201 WMMA;
here the activations stay bf16 and the scale is bf16. N is padded to a multiple of 32 (the
kernel's item is two 16-row strips) with zero rows (scale 0), sliced off again by gemm_w4a16.
M > 16 runs the kernel on 16-row slices.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from ._lib import check, lib, stream_ptr

GROUP = 128
MAX_M = 16
N_ALIGN = 32         # the kernel's item is two 16-row strips
CLIP_GRID = (1.0, 0.95, 0.9, 0.85, 0.8, 0.75, 0.7, 0.65, 0.6)
_P = ctypes.c_void_p


@dataclass(frozen=True)
class PackedW4:
    """Everything gemm_w4a16 needs; hold this on the layer."""
    wq: torch.Tensor     # uint8 [N_pad/16, K/128, 64, 16]  (= N_pad*K/2 bytes)
    sz: torch.Tensor     # int32 [N_pad/16, K/128, 16]
    n: int               # logical output features
    n_pad: int           # rows packed (multiple of N_ALIGN)
    k: int

    @property
    def nbytes(self) -> int:
        return self.wq.numel() + self.sz.numel() * 4


def available() -> bool:
    """True when the library with the W4 kernel loads."""
    try:
        lib()
        return True
    except Exception:  # noqa: BLE001
        return False


def quantize_w4(w: torch.Tensor, group: int = GROUP,
                clip_grid: tuple[float, ...] | None = None
                ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """[N, K] -> (q uint8 0..15 [N, K], scale bf16 [N, K/group], zero int16 [N, K/group]).

    Per (row, group) and clip fraction c of the min/max half-range: scale = bf16((hi_c - lo_c)
    / 15); a constant nonzero group gets scale bf16(|lo| / 7) and zero 8; zero = round(-lo_c /
    scale) clamped to +-1024; q = clamp(round(w / scale + zero), 0, 15); the c with the least
    squared error wins (ties keep the earlier c). Float32 arithmetic throughout."""
    n, k = w.shape
    assert k % group == 0, f"K={k} must be a multiple of the group {group}"
    wf = w.float().reshape(n, k // group, group)
    lo, hi = wf.amin(-1), wf.amax(-1)
    mid, half = (hi + lo) / 2, (hi - lo) / 2
    best_err = torch.full_like(lo, float("inf"))
    best_scale = torch.zeros_like(lo)
    best_zero = torch.zeros_like(lo)
    for c in (clip_grid if clip_grid is not None else CLIP_GRID):
        lo_c, hi_c = mid - c * half, mid + c * half
        scale = ((hi_c - lo_c) / 15.0).clamp(min=0.0).to(torch.bfloat16).float()
        flat = (scale == 0) & (lo != 0)
        scale = torch.where(flat, (lo.abs() / 7.0).to(torch.bfloat16).float(), scale)
        inv = torch.where(scale > 0, 1.0 / scale.clamp(min=1e-30), torch.zeros_like(scale))
        zero = torch.where(flat, torch.full_like(lo, 8.0),
                           torch.round(-lo_c * inv)).clamp_(-1024, 1024)
        q = torch.round(wf * inv.unsqueeze(-1) + zero.unsqueeze(-1)).clamp_(0, 15)
        err = ((q - zero.unsqueeze(-1)) * scale.unsqueeze(-1) - wf).square().sum(-1)
        take = err < best_err
        best_err = torch.where(take, err, best_err)
        best_scale = torch.where(take, scale, best_scale)
        best_zero = torch.where(take, zero, best_zero)
        del inv, zero, q, err
    inv = torch.where(best_scale > 0, 1.0 / best_scale.clamp(min=1e-30),
                      torch.zeros_like(best_scale))
    q = torch.round(wf * inv.unsqueeze(-1) + best_zero.unsqueeze(-1)).clamp_(0, 15)
    return (q.to(torch.uint8).reshape(n, k), best_scale.to(torch.bfloat16),
            best_zero.to(torch.int16))


# byte b of a lane's dword holds (low nibble, high nibble) = codes j of these pairs
_LO = (0, 4, 1, 5)
_HI = (2, 6, 3, 7)


def pack_codes(q: torch.Tensor) -> torch.Tensor:
    """[N, K] uint8 codes (N % 16 == 0) -> [N/16, K/128, 64, 16] in B-operand order."""
    n, k = q.shape
    v = q.reshape(n // 16, 16, k // 128, 4, 4, 8).permute(0, 2, 4, 1, 3, 5)  # nt g c r i j
    lo = v[..., list(_LO)]
    hi = v[..., list(_HI)]
    return (lo | (hi << 4)).contiguous().reshape(n // 16, k // 128, 64, 16)


def unpack_codes(wq: torch.Tensor) -> torch.Tensor:
    """Inverse of pack_codes -> [N, K] uint8."""
    nt, g = wq.shape[0], wq.shape[1]
    b = wq.reshape(nt, g, 4, 16, 4, 4)                    # nt g c r i byte
    q = torch.empty(nt, g, 4, 16, 4, 8, dtype=torch.uint8, device=wq.device)
    for byte in range(4):
        q[..., _LO[byte]] = b[..., byte] & 0xF
        q[..., _HI[byte]] = b[..., byte] >> 4
    return q.permute(0, 3, 1, 4, 2, 5).reshape(nt * 16, g * 128)   # nt r g i c j


def pack_sz(scale: torch.Tensor, zero: torch.Tensor) -> torch.Tensor:
    """(bf16 scale, int16 zero) [N, G] -> int32 [N/16, G, 16]."""
    n, g = scale.shape
    sb = scale.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
    zb = zero.to(torch.int32) << 16
    return (sb | zb).reshape(n // 16, 16, g).permute(0, 2, 1).contiguous()


def unpack_sz(sz: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """int32 [N/16, G, 16] -> (scale float32 [N, G], zero float32 [N, G])."""
    nt, g, _ = sz.shape
    d = sz.permute(0, 2, 1).reshape(nt * 16, g)
    b = d & 0xFFFF
    b = torch.where(b >= 0x8000, b - 0x10000, b)   # the bf16 bits as a signed 16-bit value
    scale = b.to(torch.int16).view(torch.bfloat16).float()
    zero = (d >> 16).float()                       # arithmetic shift keeps the sign
    return scale, zero


def pack_w4a16(weight: torch.Tensor, group: int = GROUP, chunk_tiles: int = 512,
               clip_grid: tuple[float, ...] | None = None) -> PackedW4:
    """[N, K] bf16/f32 lm_head weight -> PackedW4. Runs once at load, in chunks of
    chunk_tiles 16-row tiles so the float32 temporaries stay small."""
    assert weight.dim() == 2, f"expected [N, K], got {tuple(weight.shape)}"
    assert group == GROUP, "the kernel's group is 128"
    n, k = weight.shape
    if k % group:
        raise ValueError(f"K={k} must be a multiple of {group}")
    n_pad = (n + N_ALIGN - 1) // N_ALIGN * N_ALIGN
    dev = weight.device
    wq = torch.empty((n_pad // 16, k // group, 64, 16), dtype=torch.uint8, device=dev)
    sz = torch.empty((n_pad // 16, k // group, 16), dtype=torch.int32, device=dev)
    rows = chunk_tiles * 16
    for r0 in range(0, n_pad, rows):
        r1 = min(r0 + rows, n_pad)
        w = weight[r0:min(r1, n)]
        if w.shape[0] < r1 - r0:
            w = torch.cat([w, w.new_zeros(r1 - r0 - w.shape[0], k)], 0)
        q, scale, zero = quantize_w4(w, group, clip_grid)
        wq[r0 // 16:r1 // 16] = pack_codes(q)
        sz[r0 // 16:r1 // 16] = pack_sz(scale, zero)
        del q, scale, zero, w
    return PackedW4(wq=wq, sz=sz, n=n, n_pad=n_pad, k=k)


def unpack_w4(packed: PackedW4, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Dequantize to [N, K]: scale * (q - zero), in float32, then cast."""
    q = unpack_codes(packed.wq).float()
    scale, zero = unpack_sz(packed.sz)
    g = packed.k // GROUP
    w = (q.reshape(packed.n_pad, g, GROUP) - zero.unsqueeze(-1)) * scale.unsqueeze(-1)
    return w.reshape(packed.n_pad, packed.k)[:packed.n].to(dtype)


def gemm_w4a16(x: torch.Tensor, packed: PackedW4, out: torch.Tensor | None = None,
               wv: int = 0) -> torch.Tensor:
    """[M, K] bf16 hidden states -> [M, N] bf16 logits. No host sync, no allocation besides
    the output (none when `out` [M, N_pad] is given), so it can be captured in a HIP graph."""
    assert x.dim() == 2 and x.shape[1] == packed.k, f"expected [*, {packed.k}], got {tuple(x.shape)}"
    x = x.to(torch.bfloat16).contiguous()
    m = x.shape[0]
    y = torch.empty((m, packed.n_pad), dtype=torch.bfloat16, device=x.device) if out is None else out
    assert y.shape == (m, packed.n_pad) and y.is_contiguous()
    for r0 in range(0, m, MAX_M):
        r1 = min(m, r0 + MAX_M)
        rc = lib().rlu_gemm_w4_m16(_P(x[r0:r1].data_ptr()), r1 - r0, packed.k,
                                   _P(packed.wq.data_ptr()), _P(packed.sz.data_ptr()),
                                   _P(y[r0:r1].data_ptr()), packed.n_pad, wv, _P(stream_ptr()))
        check(rc, "rlu_gemm_w4_m16")
    return y if packed.n_pad == packed.n else y[:, :packed.n]
