"""CPU: pin the W4 oracle and the host-side packing of the W4 draft lm_head.

* layout: the oracle's packer walks the byte formula; the package's reshape/permute packer
  (torch, on CPU tensors) must produce the same bytes, and both unpackers invert them;
* quantizer: the package's torch quantizer equals the oracle's numpy one on CPU (codes,
  scales, zeros; a group may differ only where two clip fractions tie in float32);
* closed forms: every code is the nearest grid point of its (scale, zero) unless clamped; the
  chosen clip has the least float64 error of the grid; plain min/max on Gaussian weights lands at
  the ~0.104 sigma RMS error of a 16-level grid over ~5.4 sigma (kernels/draft_w4_lmhead.py:
  143-150), and the clip search does no worse;
* special groups: all-zero (N padding) -> scale 0, code 0; constant nonzero -> zero 8, exact up
  to the bf16 scale; all-positive -> negative zero;
* GEMV reference against pure-Python loops.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import fp8, w4 as ow4

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def pw4():
    from conftest import load_pkg
    return load_pkg().w4


def test_pack_layout_formula(pw4):
    rng = np.random.default_rng(0)
    q = rng.integers(0, 16, (32, 256)).astype(np.uint8)
    packed = ow4.pack_codes(q)
    # byte walk: k = 128 g + 32 i + 8 c + j, lane 16 c + r, dword i, nibble pairs of j
    lo_j, hi_j = (0, 4, 1, 5), (2, 6, 3, 7)
    for nt in range(2):
        for g in range(2):
            for c in range(4):
                for r in range(16):
                    for i in range(4):
                        for b in range(4):
                            k = 128 * g + 32 * i + 8 * c
                            want = q[16 * nt + r, k + lo_j[b]] | (q[16 * nt + r, k + hi_j[b]] << 4)
                            assert packed[nt, g, 16 * c + r, 4 * i + b] == want
    # the dequant of dword i: ((D >> 4t) & 0x000F000F) gives (q[2t], q[2t+1])
    d = packed[0, 0, 5].view(np.uint32)              # lane 5: c = 0, r = 5
    for i in range(4):
        for t in range(4):
            v = (int(d[i]) >> (4 * t)) & 0x000F000F
            assert (v & 0xF, v >> 16) == (q[5, 32 * i + 2 * t], q[5, 32 * i + 2 * t + 1])
    assert np.array_equal(pw4.pack_codes(torch.from_numpy(q)).numpy(), packed)
    assert np.array_equal(pw4.unpack_codes(torch.from_numpy(packed)).numpy(), q)
    qq, _, _ = ow4.unpack(packed, np.zeros((2, 2, 16), np.int32), 32, 256)
    assert np.array_equal(qq, q)


def test_sz_layout(pw4):
    rng = np.random.default_rng(1)
    scale = fp8.bf16_round(rng.random((32, 3)).astype(np.float32) * 0.01)
    zero = rng.integers(-1024, 1025, (32, 3)).astype(np.int16)
    sz = ow4.pack_sz(scale, zero)
    assert sz.shape == (2, 3, 16)
    d = sz.view(np.uint32)
    assert d[1, 2, 7] & 0xFFFF == fp8.bf16_bits(scale[16 + 7, 2])
    assert np.int16(np.uint16(d[1, 2, 7] >> 16)) == zero[16 + 7, 2]
    got = pw4.pack_sz(torch.from_numpy(scale).to(torch.bfloat16), torch.from_numpy(zero))
    assert np.array_equal(got.numpy(), sz)
    s2, z2 = pw4.unpack_sz(got)
    assert np.array_equal(s2.numpy(), scale) and np.array_equal(z2.numpy(), zero.astype(np.float32))


def _torch_quant(pw4, w, grid=None):
    q, s, z = pw4.quantize_w4(torch.from_numpy(w), 128, grid)
    return q.numpy(), s.float().numpy(), z.numpy()


def test_quantizer_torch_equals_numpy(pw4):
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((64, 1024)) * 0.02).astype(np.float32)
    q0, s0, z0 = ow4.quantize_w4(w)
    q1, s1, z1 = _torch_quant(pw4, w)
    same = (s0 == s1) & (z0 == z1)
    assert same.mean() > 0.999, same.mean()
    rows, groups = np.nonzero(same)
    for r, g in zip(rows, groups):
        assert np.array_equal(q0[r, 128 * g:128 * g + 128], q1[r, 128 * g:128 * g + 128])


def test_codes_nearest_and_clip_optimal():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((16, 512)) * 0.03).astype(np.float32)
    q, s, z = ow4.quantize_w4(w)
    g = w.reshape(16, 4, 128).astype(np.float64)
    pos = g / s[..., None] + z[..., None]
    qq = q.reshape(16, 4, 128).astype(np.float64)
    inside = (pos > -0.5) & (pos < 15.5)
    assert (np.abs(pos - qq)[inside] <= 0.5 + 1e-5).all()
    assert (qq[pos <= -0.5] == 0).all() and (qq[pos >= 15.5] == 15).all()
    # the chosen clip's float64 error is within float32 rounding of the best of the grid
    chosen = ((qq - z[..., None]) * s[..., None] - g) ** 2
    chosen = chosen.sum(-1)
    for c in ow4.CLIP_GRID:
        qc, sc, zc = ow4.quantize_w4(w, clip_grid=(c,))
        e = (((qc.reshape(16, 4, 128) - zc[..., None].astype(np.float64)) * sc[..., None]
              - g) ** 2).sum(-1)
        assert (chosen <= e * (1 + 1e-5) + 1e-30).all()


def test_gaussian_error_level():
    rng = np.random.default_rng(4)
    w = rng.standard_normal((64, 2560)).astype(np.float32)
    q, s, z = ow4.quantize_w4(w, clip_grid=(1.0,))
    rel_plain = np.linalg.norm(ow4.dequant(q, s, z) - w) / np.linalg.norm(w)
    assert 0.095 < rel_plain < 0.115, rel_plain
    q, s, z = ow4.quantize_w4(w)
    rel_clip = np.linalg.norm(ow4.dequant(q, s, z) - w) / np.linalg.norm(w)
    assert rel_clip <= rel_plain and rel_clip < 0.105, (rel_clip, rel_plain)


def test_special_groups():
    w = np.zeros((16, 384), np.float32)
    w[1, 128:256] = 0.75                       # constant nonzero
    w[2, 256:] = np.linspace(0.5, 1.0, 128)    # all positive
    q, s, z = ow4.quantize_w4(w)
    assert s[0, 0] == 0 and not q[0].any()                       # all zero
    assert z[1, 1] == 8 and q[1, 128:256].min() == q[1, 128:256].max()
    deq = ow4.dequant(q, s, z)
    assert abs(deq[1, 130] - 0.75) <= 0.75 * 2 ** -8
    assert z[2, 2] < 0
    # plain min/max covers the ramp: every weight within half a step (plus the bf16 rounding
    # of the scale, which stretches or shrinks the 15-step grid by < 15 * 2^-9 of a step each)
    q, s, z = ow4.quantize_w4(w, clip_grid=(1.0,))
    deq = ow4.dequant(q, s, z)
    assert np.abs(deq[2, 256:] - w[2, 256:]).max() <= s[2, 2] * (0.5 + 15 * 2 ** -8)


def test_gemv_against_loops():
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((16, 256)) * 0.05).astype(np.float32)
    x = fp8.bf16_round(rng.standard_normal((3, 256)).astype(np.float32))
    q, s, z = ow4.quantize_w4(w)
    y = ow4.gemv(x, q, s, z)
    for m in range(3):
        for n in (0, 7, 15):
            acc = 0.0
            for k in range(256):
                acc += float(x[m, k]) * (float(q[n, k]) - float(z[n, k // 128])) * float(s[n, k // 128])
            assert abs(y[m, n] - acc) <= 1e-12 * max(1.0, abs(acc))
