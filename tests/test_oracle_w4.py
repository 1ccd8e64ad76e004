"""CPU: pin the W4 oracle (the quantizer and the layout the packing kernel writes).

* layout: the oracle's packer walks the byte formula; the package's unpackers (torch, CPU
  tensors) invert it; the oracle's lane view puts value k = 128 g + 32 i + 8 c + j of a row where
  lane 16 c + r keeps it (the order its error terms are summed in);
* quantizer, closed forms: every code is the nearest grid point of its (scale, zero) unless
  clamped; a hand-worked ramp; constant groups decode to bf16(v); an all-zero group is zeros;
* quantizer, brute force: for every group the chosen (scale, zero) has the least float64 error of
  the 30 candidates (up to float32 rounding of the sums), stays within 1% of the best over a
  wider family (every zero within +-6 of centre at every fraction), and is never worse than plain
  min/max;
* error level on Gaussian weights: plain min/max lands at the ~0.104 sigma RMS error of a
  16-level grid over the ~5.4 sigma range of 128 samples (kernels/draft_w4_lmhead.py:143-150
  quotes the same figure), the search below it;
* planted mistakes (centre sign, no zero neighbours, scale not rounded) fail these pins;
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
    assert np.array_equal(pw4.unpack_codes(torch.from_numpy(packed)).numpy(), q)
    qq, _, _ = ow4.unpack(packed, np.zeros((2, 2, 16), np.int32), 32, 256)
    assert np.array_equal(qq, q)


def test_lane_view_matches_layout():
    """_lanes puts value k = 128 g + 32 i + 8 c + j of row n at [n, g, c, 8 i + j]: the lane
    that stores its nibble, in the order of its dwords."""
    w = np.arange(2 * 256, dtype=np.float32).reshape(2, 256)
    t = ow4._lanes(w, 128)
    for n in range(2):
        for g in range(2):
            for c in range(4):
                for i in range(4):
                    for j in range(8):
                        assert t[n, g, c, 8 * i + j] == w[n, 128 * g + 32 * i + 8 * c + j]
    assert np.array_equal(ow4._unlanes(t), w)


def test_sz_layout(pw4):
    rng = np.random.default_rng(1)
    scale = fp8.bf16_round(rng.random((32, 3)).astype(np.float32) * 0.01)
    zero = rng.integers(-1024, 1025, (32, 3)).astype(np.int16)
    sz = ow4.pack_sz(scale, zero)
    assert sz.shape == (2, 3, 16)
    d = sz.view(np.uint32)
    assert d[1, 2, 7] & 0xFFFF == fp8.bf16_bits(scale[16 + 7, 2])
    assert np.int16(np.uint16(d[1, 2, 7] >> 16)) == zero[16 + 7, 2]
    s2, z2 = pw4.unpack_sz(torch.from_numpy(sz))
    assert np.array_equal(s2.numpy(), scale) and np.array_equal(z2.numpy(), zero.astype(np.float32))


def test_fraction_table():
    assert [float(f) for f in ow4.FRACTIONS] == [float(np.float32(x)) for x in
                                                  (1.0, 0.95, 0.9, 0.85, 0.8, 0.75, 0.7, 0.65,
                                                   0.6, 0.55)]


def _f(x) -> float:
    return float(np.asarray(x).reshape(-1)[0])


def _candidates(g: np.ndarray, wide: int = 1):
    """Every (s, z) candidate of one group, computed in float64 where the definition does not
    fix a float32 step: s = bf16(f * width / 15) (the stored scale), zero = the integer nearest
    7.5 - mid / s plus d for |d| <= wide. Returns [(err64, s, z)]."""
    lo, hi = float(g.min()), float(g.max())
    out = []
    for f in ow4.FRACTIONS:
        s = _f(fp8.bf16_round(np.float32(np.float32(f) * np.float32(hi - lo)) / np.float32(15)))
        if s <= 0:
            continue
        zc = np.rint(7.5 - (lo + hi) / 2 / s)
        for d in range(-wide, wide + 1):
            z = float(np.clip(zc + d, -1024, 1024))
            q = np.clip(np.rint(g.astype(np.float64) / s) + z, 0, 15)
            out.append((float((((q - z) * s - g) ** 2).sum()), s, z))
    return out


def _group_err(q, s, z, g):
    return float((((q.astype(np.float64) - float(z)) * float(s) - g) ** 2).sum())


def test_codes_nearest_grid_point():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((16, 512)) * 0.03).astype(np.float32)
    q, s, z = ow4.quantize_w4(w)
    g = w.reshape(16, 4, 128).astype(np.float64)
    pos = g / s[..., None] + z[..., None]
    qq = q.reshape(16, 4, 128).astype(np.float64)
    inside = (pos > -0.5) & (pos < 15.5)
    assert (np.abs(pos - qq)[inside] <= 0.5 + 1e-5).all()
    assert (qq[pos <= -0.5] == 0).all() and (qq[pos >= 15.5] == 15).all()


def test_choice_is_least_error_brute_force():
    rng = np.random.default_rng(7)
    w = np.concatenate([(rng.standard_normal((8, 512)) * 0.02),
                        rng.standard_t(3, (8, 512)) * 0.02,                  # heavy tails
                        rng.random((8, 512)) * 0.1 + 0.05]).astype(np.float32)   # one-sided
    q, s, z = ow4.quantize_w4(w)
    qp, sp, zp = ow4.quantize_w4(w, fractions=(ow4.FRACTIONS[0],), shifts=(0,))
    n = w.shape[0]
    for r in range(n):
        for gi in range(4):
            g = w[r, 128 * gi:128 * gi + 128].astype(np.float64)
            chosen = _group_err(q[r, 128 * gi:128 * gi + 128], s[r, gi], z[r, gi], g)
            best30 = min(e for e, _, _ in _candidates(g, 1))
            best_wide = min(e for e, _, _ in _candidates(g, 6))
            plain = _group_err(qp[r, 128 * gi:128 * gi + 128], sp[r, gi], zp[r, gi], g)
            assert chosen <= best30 * (1 + 1e-5) + 1e-30, (r, gi)
            assert chosen <= best_wide * 1.01 + 1e-30, (r, gi)
            assert chosen <= plain * (1 + 1e-5) + 1e-30, (r, gi)


def test_hand_worked_ramp():
    """A group holding 0.1 k for k = 0..15 (each 8 times): width 1.5, so s = bf16(0.1) =
    0.10009765625, centre 0.75 -> z = rint(7.5 - 7.4927) = 0, and code k for 0.1 k
    (0.1 k / s = 0.99902 k rounds to k up to k = 15)."""
    g = np.repeat(np.arange(16, dtype=np.float32) * np.float32(0.1), 8)
    w = np.tile(g, (16, 1))
    q, s, z = ow4.quantize_w4(w)
    assert s[0, 0] == np.float32(0.10009765625) and z[0, 0] == 0
    assert np.array_equal(q[0], np.repeat(np.arange(16), 8))


def test_special_groups():
    w = np.zeros((16, 512), np.float32)
    w[1, 128:256] = 0.75                        # constant positive
    w[3, 128:256] = -0.3                        # constant negative
    w[2, 256:384] = np.linspace(0.5, 1.0, 128)  # all positive
    w[4, 384:] = np.linspace(100.0, 100.01, 128)   # offset far beyond the zero range
    q, s, z = ow4.quantize_w4(w)
    assert s[0, 0] == 0 and z[0, 0] == 0 and not q[0].any()               # all zero
    deq = ow4.dequant(q, s, z)
    assert s[1, 1] == np.float32(0.75) and z[1, 1] == 0 and (q[1, 128:256] == 1).all()
    assert deq[1, 130] == 0.75
    assert z[3, 1] == 1 and (q[3, 128:256] == 0).all()
    assert deq[3, 200] == -_f(fp8.bf16_round(np.float32(0.3)))
    assert z[2, 2] < 0
    assert z[4, 3] == -1024 and q[4, 384:].min() >= 0 and q[4, 384:].max() <= 15


def test_plain_min_max_covers_a_ramp():
    """Plain min/max: every weight of a ramp within half a step, plus the bf16 rounding of the
    scale, which stretches or shrinks the 15-step grid by < 15 * 2^-9 of a step."""
    w = np.zeros((16, 128), np.float32)
    w[2] = np.linspace(0.5, 1.0, 128)
    q, s, z = ow4.quantize_w4(w, fractions=(ow4.FRACTIONS[0],), shifts=(0,))
    deq = ow4.dequant(q, s, z)
    assert z[2, 0] < 0
    assert np.abs(deq[2] - w[2]).max() <= s[2, 0] * (0.5 + 15 * 2 ** -8)


def test_gaussian_error_level():
    rng = np.random.default_rng(4)
    w = rng.standard_normal((64, 2560)).astype(np.float32)
    q, s, z = ow4.quantize_w4(w, fractions=(ow4.FRACTIONS[0],), shifts=(0,))
    rel_plain = np.linalg.norm(ow4.dequant(q, s, z) - w) / np.linalg.norm(w)
    assert 0.095 < rel_plain < 0.115, rel_plain
    q, s, z = ow4.quantize_w4(w)
    rel = np.linalg.norm(ow4.dequant(q, s, z) - w) / np.linalg.norm(w)
    assert rel <= rel_plain and rel < 0.098, (rel, rel_plain)


def _planted_quant(kind, w):
    """A copy of the oracle's candidate loop with one plausible mistake."""
    w = np.asarray(w, np.float32)
    n, k = w.shape
    gw = w.reshape(n, k // 128, 128)
    lo, hi = gw.min(-1), gw.max(-1)
    best = (np.full(lo.shape, np.inf), None)
    out_s = np.zeros(lo.shape, np.float32)
    out_z = np.zeros(lo.shape, np.float32)
    for f in ow4.FRACTIONS:
        s = np.float32(f) * (hi - lo) / np.float32(15)
        if kind != "scale-not-rounded":
            s = fp8.bf16_round(s)
        sign = 1 if kind == "centre-sign" else -1     # the centre is 7.5 - mid / s
        z0 = np.clip(np.rint(np.float32(7.5) + sign * ((hi + lo) / 2) / s), -1024, 1024)
        for dz in ((0,) if kind == "no-neighbours" else (0, -1, 1)):
            z = np.clip(z0 + dz, -1024, 1024)
            q = np.clip(np.rint(gw / s[..., None]) + z[..., None], 0, 15)
            e = (((q - z[..., None]) * s[..., None] - gw) ** 2).sum(-1)
            take = e < best[0]
            best = (np.where(take, e, best[0]), None)
            out_s = np.where(take, s, out_s)
            out_z = np.where(take, z, out_z)
    return out_s, out_z


@pytest.mark.parametrize("kind", ["centre-sign", "no-neighbours", "scale-not-rounded"])
def test_planted_quantizer_mistakes_are_caught(kind):
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((16, 512)) * 0.02 + 0.01).astype(np.float32)
    _, s, z = ow4.quantize_w4(w)
    ps, pz = _planted_quant(kind, w)
    if kind == "scale-not-rounded":
        assert not np.array_equal(fp8.bf16_round(ps), ps)    # the stored scale must be bf16
    else:
        assert not (np.array_equal(ps, s) and np.array_equal(pz, z.astype(np.float32)))


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
