"""CPU: the C-ABI library loads and exports every entry point include/rlu.h declares, and
the host side refuses to run without it (no compute is launched here: there is no GPU)."""
from __future__ import annotations

import ctypes
import pathlib
import re

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent


def declared_symbols() -> list[str]:
    text = (ROOT / "include" / "rlu.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*int\s+(\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_reference_entry_points():
    syms = declared_symbols()
    for s in ("r4d_lru_manage", "r4d_lru_fused", "r4d_lru_gather"):
        assert s in syms


def test_library_exports_every_declared_symbol(pkg):
    if not pkg.LIB_PATH.exists():
        pytest.skip("librlu.so not built")
    h = ctypes.CDLL(str(pkg.LIB_PATH))
    missing = [s for s in declared_symbols() if not hasattr(h, s)]
    assert not missing, f"librlu.so lacks {missing}"


def test_binding_covers_every_declared_symbol(pkg):
    assert set(declared_symbols()) <= set(pkg._lib.SIGNATURES)


def test_bad_arguments_return_minus_one_without_launching(pkg):
    """The argument checks run before any launch, so they can be exercised without a GPU
    (kernels/lru/r4d_lru.hip:583-584,602-604,617-620)."""
    if not pkg.LIB_PATH.exists():
        pytest.skip("librlu.so not built")
    lib = pkg.lib()
    P = ctypes.c_void_p
    z = [P(0)] * 8
    assert lib.r4d_lru_manage(P(0), 0, 0, 4, 1, 1, *z, P(0)) == -1          # E <= 0
    assert lib.r4d_lru_manage(P(0), 0, 8, 1025, 1, 1, *z, P(0)) == -1       # S > 1024
    assert lib.r4d_lru_manage(P(0), 0, 8, 4, 1, 1025, *z, P(0)) == -1       # maxi > 1024
    assert lib.r4d_lru_manage(P(0), 0, 8, 4, 1, -1, *z, P(0)) == -1         # maxi < 0
    assert lib.r4d_lru_manage(P(0), 0, 1025, 4, 1, 1, *z, P(0)) == -1       # E > 1024
    o = [P(0)] * 6
    assert lib.r4d_lru_fused(P(0), 10, 1025, 4, 1, 1, *z, 16, 10, 1, *o, P(0)) == -1
    assert lib.r4d_lru_fused(P(0), 10, 8, 4, 1, 1, *z, 0, 10, 1, *o, P(0)) == -1
    assert lib.r4d_lru_fused(P(0), 10, 8, 4, 1, 1, *z, 16, 0, 1, *o, P(0)) == -1
    assert lib.r4d_lru_fused(P(0), -1, 8, 4, 1, 1, *z, 16, 10, 1, *o, P(0)) == -1
    g = [P(0), P(0), ctypes.c_long(32)] * 6
    g_bad = [P(0), P(0), ctypes.c_long(24)] + g[3:]
    assert lib.r4d_lru_gather(*g_bad, P(0), P(0), 8, 16, P(0)) == -1
    assert lib.r4d_lru_gather(*g, P(0), P(0), 0, 16, P(0)) == -1
    assert lib.r4d_lru_gather(*g, P(0), P(0), 8, 0, P(0)) == -1
    pk = lib.rlu_pack_w4
    assert pk(P(0), 0, 256, 16, 256, 16, P(0), P(0), P(0)) == -1            # null pointers
    a = P(4096)
    assert pk(a, 0, 256, 0, 256, 16, a, a, P(0)) == -1                      # N < 1
    assert pk(a, 0, 256, 32, 256, 16, a, a, P(0)) == -1                     # n_pad < N
    assert pk(a, 0, 100, 16, 128, 16, a, a, P(0)) == -1                     # ld < K
    assert pk(a, 0, 200, 16, 200, 16, a, a, P(0)) == -2                     # K % 128
    assert pk(a, 0, 256, 16, 256, 24, a, a, P(0)) == -2                     # n_pad % 16
    assert pk(a, 3, 256, 16, 256, 16, a, a, P(0)) == -3                     # dtype
    assert pk(a, 0, 260, 16, 256, 16, a, a, P(0)) == -4                     # row alignment
    assert pk(P(4098), 0, 256, 16, 256, 16, a, a, P(0)) == -4               # base alignment


def test_missing_library_fails_loudly(pkg, monkeypatch, tmp_path):
    monkeypatch.setattr(pkg._lib, "LIB_PATH", tmp_path / "nope.so")
    pkg._lib.lib.cache_clear()
    try:
        with pytest.raises(pkg.LibraryMissing):
            pkg._lib.lib()
    finally:
        pkg._lib.lib.cache_clear()


def test_fp8_target_head_routes_without_a_gpu(pkg):
    """Fp8TargetHead's dispatch (kernels/fp8_target_lmhead.py:85-93), host side only: more rows
    than VLLM_TARGET_FP8_LMHEAD_MAX_M, a bias, or a non-bf16 input go to the original method;
    attributes it does not define come from the original method."""
    import torch
    from importlib import import_module
    ops = import_module(pkg.__name__ + ".ops")

    class Orig:
        tag = "orig-attr"

        def __init__(self):
            self.calls = []

        def apply(self, layer, x, bias=None):
            self.calls.append((tuple(x.shape), x.dtype, bias is not None))
            return "orig"

    head = ops.Fp8TargetHead.__new__(ops.Fp8TargetHead)
    head.orig, head.wq, head.ws, head.n_fp8 = Orig(), None, None, 0
    m = ops.FP8_LMHEAD_MAX_M
    assert m == 64
    assert head.apply(None, torch.zeros(m + 1, 128, dtype=torch.bfloat16)) == "orig"
    assert head.apply(None, torch.zeros(2, 3, 128, dtype=torch.bfloat16),
                      bias=torch.zeros(8)) == "orig"
    assert head.apply(None, torch.zeros(4, 128, dtype=torch.float16)) == "orig"
    assert [c[0] for c in head.orig.calls] == [(m + 1, 128), (2, 3, 128), (4, 128)]
    assert head.n_fp8 == 0 and head.tag == "orig-attr"
    with pytest.raises(AttributeError):
        ops.Fp8TargetHead.__new__(ops.Fp8TargetHead).anything
