"""ctypes binding of lib/librlu.so (the C-ABI declared in include/rlu.h).

There is no fallback: if the library is missing or lacks a symbol, `lib()` raises, so a
caller can never silently run anything but the HIP kernels.
"""
from __future__ import annotations

import ctypes
import functools
import os
import pathlib

LIB_PATH = pathlib.Path(os.environ.get(
    "R4D_LRU_LIB", pathlib.Path(__file__).resolve().parent / "lib" / "librlu.so"))

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_long
_LL = ctypes.c_longlong

# name -> (restype, argtypes); one line per export of include/rlu.h
SIGNATURES: dict[str, tuple] = {
    "r4d_lru_manage": (_I, [_P] + [_I] * 5 + [_P] * 9),
    "r4d_lru_fused": (_I, [_P] + [_I] * 5 + [_P] * 8 + [_I] * 3 + [_P] * 7),
    "r4d_lru_gather": (_I, [_P, _P, _L] * 6 + [_P, _P, _I, _I, _P]),
    "rlu_lru_split_fresh": (_I, [_P, _I, _P, _P, _I, _I, _P, _P, _P]),
    "rlu_lru_fused_quant": (_I, [_P] + [_I] * 5 + [_P] * 8 + [_I] * 3 + [_P] * 7 + [_I] * 3
                            + [_P] * 3),
    "rlu_quant_fp8_group": (_I, [_P, _I, _I, _I, _I, _P, _P, _P]),
    "rlu_silu_mul_quant": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P]),
    "rlu_moe_sum": (_I, [_P, _I, _I, _I, _P, _P]),
    "r4d_gemm_moe_fp8blk_nt_b16": (_I, [_P] * 10 + [_I] * 8 + [_P]),
    "rlu_gemm_fp8blk_m16": (_I, [_P] * 5 + [_I] * 5 + [_P]),
    "rlu_moe_gemm_split": (_I, [_P] * 14 + [_I] * 8 + [_P]),
    "rlu_moe_gemm_split_act": (_I, [_P] * 13 + [_I] * 7 + [_P]),
    "rlu_moe_gemm_split_qin": (_I, [_P] * 13 + [_I] * 4 + [_P]),
    "rlu_shuffle_fp8_weight": (_I, [_P, _P, _LL, _I, _P]),
    "rlu_gemm_w4_m16": (_I, [_P, _I, _I, _P, _P, _P, _I, _I, _P]),
    "rlu_pack_w4": (_I, [_P, _I, _LL, _I, _I, _I, _P, _P, _P]),
    "rlu_moe_gemm_tiles": (_I, [_P, _P, _I, _P, _P, _P]),
    "rlu_moe_gemm_fp8blk_tiled": (_I, [_P] * 8 + [_I, _P, _P] + [_I] * 5 + [_P]),
    "rlu_moe_gemm_fp8blk_tiled_noalloc": (_I, [_P] * 7 + [_I, _P, _P] + [_I] * 5 + [_P]),
    "rlu_moe_gemm_fp8blk_tiled_silu_quant": (_I, [_P] * 8 + [_I, _P, _P] + [_I] * 4 + [_P]),
    "rlu_moe_gemm_tiles_split": (_I, [_P, _P, _I, _P, _P, _I, _P, _P, _P]),
    "rlu_moe_gemm_fp8blk_tiled_split": (_I, [_P] * 12 + [_I, _P, _P] + [_I] * 4 + [_P]),
    "rlu_moe_gemm_fp8blk_tiled_split_silu_quant": (_I, [_P] * 12 + [_I, _P, _P] + [_I] * 4 +
                                                   [_P]),
    "rlu_moe_down_sum": (_I, [_P] * 10 + [_I] * 5 + [_P]),
    "rlu_moe_down_sum_act": (_I, [_P] * 9 + [_I] * 5 + [_P]),
    "rlu_route_capture": (_I, [_P] + [_I] * 5 + [_P] * 4),
    "rlu_selftest_bf16": (_I, [_P, _P]),
}


class LibraryMissing(RuntimeError):
    pass


@functools.lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise LibraryMissing(
            f"{LIB_PATH} not found: build it first (python r9700-lru-expert-cache_amd/build.py "
            "or __graft_entry__.build()); there is no CPU fallback")
    h = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        try:
            f = getattr(h, name)
        except AttributeError as exc:
            raise LibraryMissing(f"{LIB_PATH} has no {name}; rebuild it") from exc
        f.restype = res
        f.argtypes = args
    return h


def stream_ptr(stream=None) -> int:
    import torch
    s = torch.cuda.current_stream() if stream is None else stream
    return s.cuda_stream


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed rc={rc}")


@functools.lru_cache(maxsize=1)
def _hip():
    return ctypes.CDLL("libamdhip64.so")


@functools.lru_cache(maxsize=4096)
def _pinned_device_ptr(host_ptr: int) -> int:
    dp = ctypes.c_void_p()
    rc = _hip().hipHostGetDevicePointer(ctypes.byref(dp), ctypes.c_void_p(host_ptr),
                                        ctypes.c_uint(0))
    if rc != 0:
        raise RuntimeError(f"hipHostGetDevicePointer rc={rc}")
    return dp.value


def device_ptr_of_pinned(t) -> int:
    """Device-visible address of a pinned host tensor (UVA); looked up once per address."""
    return _pinned_device_ptr(t.data_ptr())


def device_ptr(t) -> int:
    """The address a kernel uses for `t`: its own for device memory, the device-visible one
    for pinned host memory. Anything else (pageable host memory) is refused."""
    if t.is_cuda:
        return t.data_ptr()
    if t.is_pinned():
        return device_ptr_of_pinned(t)
    raise ValueError("operand must be device memory or pinned host memory")
