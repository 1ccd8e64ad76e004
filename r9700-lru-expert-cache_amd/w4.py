"""W4 draft lm_head: int4 group-128 weights, bf16 activations, bf16 logits, on librlu.so.

Mirrors kernels/draft_w4_lmhead.py: PackedW4 (:63-76), quantize_w4 (:154-198), pack_w4a16
(:228-259), unpack_w4 (:262-285), the op draft_w4_lmhead_gemm (:351-390) and gemm_w4a16
(:393-403), in this build's gfx950 format:

  codes  q in 0..15 per weight, w ~ scale * (q - zero) per (row, 128-column group), asymmetric,
         a bf16 scale and an integer zero in [-1024, 1024] (a constant or all-positive group
         needs one outside 0..15).
  wq     uint8 [N_pad/16, K/128, 64, 16]: the 1 KB of a 16-row x 128-deep tile in
         v_mfma_f32_16x16x32_bf16 B-operand order (lane 16 c + r holds row r, four dwords, one
         per 32-deep step i, k = 128 g + 32 i + 8 c + j; nibble t of the low half is j = 2t,
         nibble t of the high half is j = 2t + 1).
  sz     int32 [N_pad/16, K/128, 16]: bf16 scale bits | int16 zero << 16.

Quantizing and packing is one kernel (rlu_pack_w4): a wave per 16-row x 128-column tile, each
lane choosing the codes of the nibbles it stores. Per (row, group) it tries 10 clip fractions of
the group's range (bf16 scale) and, for each, the centred integer zero and its two neighbours,
and keeps the least squared error; a constant group is stored exactly up to the bf16 scale.
The reference stores an f16 scale and widens bf16 activations to f16 for its gfx1201 WMMA; here
the activations stay bf16. N is padded to a multiple of 32 (the GEMV's item is two 16-row
strips) with zero rows, sliced off again by the op. M > 16 runs the kernel on 16-row slices.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from ._lib import check, lib, stream_ptr
from .lru import OPS_NAMESPACE as OPS_NS

GROUP = 128
MAX_M = 16
N_ALIGN = 32         # the kernel's item is two 16-row strips
_P = ctypes.c_void_p
_DTYPE_CODE = {torch.bfloat16: 0, torch.float32: 1, torch.float16: 2}


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


# byte b of a lane's dword holds (low nibble, high nibble) = codes j of these pairs
_LO = (0, 4, 1, 5)
_HI = (2, 6, 3, 7)


def unpack_codes(wq: torch.Tensor) -> torch.Tensor:
    """Packed codes [N/16, K/128, 64, 16] -> [N, K] uint8."""
    nt, g = wq.shape[0], wq.shape[1]
    b = wq.reshape(nt, g, 4, 16, 4, 4)                    # nt g c r i byte
    q = torch.empty(nt, g, 4, 16, 4, 8, dtype=torch.uint8, device=wq.device)
    for byte in range(4):
        q[..., _LO[byte]] = b[..., byte] & 0xF
        q[..., _HI[byte]] = b[..., byte] >> 4
    return q.permute(0, 3, 1, 4, 2, 5).reshape(nt * 16, g * 128)   # nt r g i c j


def unpack_sz(sz: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """int32 [N/16, G, 16] -> (scale float32 [N, G], zero float32 [N, G])."""
    nt, g, _ = sz.shape
    d = sz.permute(0, 2, 1).reshape(nt * 16, g)
    b = d & 0xFFFF
    b = torch.where(b >= 0x8000, b - 0x10000, b)   # the bf16 bits as a signed 16-bit value
    scale = b.to(torch.int16).view(torch.bfloat16).float()
    zero = (d >> 16).float()                       # arithmetic shift keeps the sign
    return scale, zero


def pack_w4a16(weight: torch.Tensor, group: int = GROUP) -> PackedW4:
    """[N, K] bf16 / f32 / f16 lm_head weight on the GPU -> PackedW4, one kernel launch
    (rlu_pack_w4). Runs once at load; the result is what gemm_w4a16 reads."""
    assert weight.dim() == 2, f"expected [N, K], got {tuple(weight.shape)}"
    assert group == GROUP, "the kernel's group is 128"
    if not weight.is_cuda:
        raise ValueError("pack_w4a16 packs on the GPU: move the weight to the device first")
    if weight.dtype not in _DTYPE_CODE:
        raise TypeError(f"pack_w4a16 takes bf16, f32 or f16 weights, not {weight.dtype}")
    n, k = weight.shape
    if k % group:
        raise ValueError(f"K={k} must be a multiple of {group}")
    if weight.stride(1) != 1:
        weight = weight.contiguous()
    n_pad = (n + N_ALIGN - 1) // N_ALIGN * N_ALIGN
    dev = weight.device
    wq = torch.empty((n_pad // 16, k // group, 64, 16), dtype=torch.uint8, device=dev)
    sz = torch.empty((n_pad // 16, k // group, 16), dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        rc = lib().rlu_pack_w4(_P(weight.data_ptr()), _DTYPE_CODE[weight.dtype],
                               weight.stride(0), n, k, n_pad, _P(wq.data_ptr()),
                               _P(sz.data_ptr()), _P(stream_ptr()))
    check(rc, "rlu_pack_w4")
    return PackedW4(wq=wq, sz=sz, n=n, n_pad=n_pad, k=k)


def quantize_w4(w: torch.Tensor, group: int = GROUP
                ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """[N, K] -> (q uint8 0..15 [N, K], scale bf16 [N, K/group], zero int16 [N, K/group]):
    the codes pack_w4a16 stores, read back out of the packed layout."""
    p = pack_w4a16(w, group)
    scale, zero = unpack_sz(p.sz)
    return (unpack_codes(p.wq)[:p.n], scale[:p.n].to(torch.bfloat16),
            zero[:p.n].to(torch.int16))


def unpack_w4(packed: PackedW4, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Dequantize to [N, K]: scale * (q - zero), in float32, then cast."""
    q = unpack_codes(packed.wq).float()
    scale, zero = unpack_sz(packed.sz)
    g = packed.k // GROUP
    w = (q.reshape(packed.n_pad, g, GROUP) - zero.unsqueeze(-1)) * scale.unsqueeze(-1)
    return w.reshape(packed.n_pad, packed.k)[:packed.n].to(dtype)


def _gemm_into(x: torch.Tensor, packed_wq: torch.Tensor, packed_sz: torch.Tensor, k: int,
               y: torch.Tensor, wv: int) -> None:
    m = x.shape[0]
    n_pad = packed_wq.shape[0] * 16
    for r0 in range(0, m, MAX_M):
        r1 = min(m, r0 + MAX_M)
        rc = lib().rlu_gemm_w4_m16(_P(x[r0:r1].data_ptr()), r1 - r0, k,
                                   _P(packed_wq.data_ptr()), _P(packed_sz.data_ptr()),
                                   _P(y[r0:r1].data_ptr()), n_pad, wv, _P(stream_ptr()))
        check(rc, "rlu_gemm_w4_m16")


def _draft_w4_lmhead_gemm(x: torch.Tensor, wq: torch.Tensor, wsz: torch.Tensor, n: int,
                          k: int, wv: int, sk: int, npw: int, nt: int) -> torch.Tensor:
    """The op of kernels/draft_w4_lmhead.py:351-390: [M, K] hidden states -> [M, n] bf16
    logits, every M in one opaque call (16-row slices inside). wv = workgroups per CU of the
    kernel's persistent grid (0: the kernel's default). sk / npw / nt name the closed kernel's
    K split, columns per wave and tile shape; this kernel derives its K split from K and has one
    item shape, so they are accepted for the schema (non-negative) and not used."""
    if min(wv, sk, npw, nt) < 0:
        raise ValueError("draft_w4_lmhead_gemm: negative config")
    assert x.dim() == 2 and x.shape[1] == k, f"expected [*, {k}], got {tuple(x.shape)}"
    x = x.to(torch.bfloat16).contiguous()
    n_pad = wq.shape[0] * 16
    y = torch.empty((x.shape[0], n_pad), dtype=torch.bfloat16, device=x.device)
    _gemm_into(x, wq, wsz, k, y, wv)
    return y if n_pad == n else y[:, :n].contiguous()


def _register():
    from .lru import OPS_NAMESPACE
    lib_ = torch.library.Library(OPS_NAMESPACE, "FRAGMENT")
    lib_.define("draft_w4_lmhead_gemm(Tensor x, Tensor wq, Tensor wsz, int n, int k, int wv, "
                "int sk, int npw, int nt) -> Tensor")
    lib_.impl("draft_w4_lmhead_gemm", _draft_w4_lmhead_gemm, "CUDA")
    lib_.impl("draft_w4_lmhead_gemm",
              lambda x, wq, wsz, n, *a: torch.empty((x.shape[0], n), dtype=torch.bfloat16,
                                                    device=x.device), "Meta")
    return lib_


_OPS_LIB = _register()


def gemm_w4a16(x: torch.Tensor, packed: PackedW4, out: torch.Tensor | None = None,
               wv: int = 0) -> torch.Tensor:
    """[M, K] bf16 hidden states -> [M, N] bf16 logits through the draft_w4_lmhead_gemm op
    (kernels/draft_w4_lmhead.py:393-403). With `out` ([M, N_pad] bf16) the kernel writes into
    it and nothing is allocated, for callers that capture it into a HIP graph."""
    assert x.dim() == 2 and x.shape[1] == packed.k, f"expected [*, {packed.k}], got {tuple(x.shape)}"
    if out is None:
        op = getattr(torch.ops, OPS_NS).draft_w4_lmhead_gemm
        return op(x, packed.wq, packed.sz, packed.n, packed.k, wv, 0, 0, 0)
    x = x.to(torch.bfloat16).contiguous()
    assert out.shape == (x.shape[0], packed.n_pad) and out.is_contiguous()
    _gemm_into(x, packed.wq, packed.sz, packed.k, out, wv)
    return out if packed.n_pad == packed.n else out[:, :packed.n]
