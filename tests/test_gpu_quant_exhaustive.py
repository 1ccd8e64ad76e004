"""GPU: the e4m3 activation quant over its whole input domain, against IEEE division.

Every quant kernel of the path (group-128 and per-token quant, SiLU-mul-quant, the down
prologue, the prefill epilogue) takes bf16 values x and a scale s = max(RN(amax / 448),
1 / (448 * 512)) made from the bf16 amax of the group, and stores e4m3(clamp(x / s, +-448)) with
the division rounded to nearest (kernels/fused_silu_mul_quant.py:43-57). The input space is
finite: every positive finite bf16 amax, with every bf16 x of |x| <= amax and both signs
(1.07e9 pairs), plus a NaN amax (which falls to the floor scale) and an infinite one, each with
every bf16 x. All of it runs through rlu_quant_fp8_group in groups of 128 (the group's first
entry is its amax), and every code and every scale must equal the one torch computes with IEEE
division (float64, rounded once to float32), fmax / fmin clamps (the kernels' NaN rule) and its
float8_e4m3fn cast.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import gpu_case

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda"
MIN_SCALE = np.float32(1.0) / (np.float32(448.0) * np.float32(512.0))
CHUNK = 1 << 20            # groups of 128 per call


def _groups_finite():
    """Chunks of int16 bf16 bit patterns [<= CHUNK, 128]: entry 0 of a group is its amax
    (every positive finite bf16, ascending), the other 127 are up to 127 of the values b[0..i]
    (every positive bf16 up to that amax; +0.0 past them). The last chunk is padded with
    all-zero groups to a multiple of 16 groups (one 2048-column row)."""
    n = 0x7F80 - 1                                  # positive finite bf16: 0x0001..0x7F7F
    per = (np.arange(1, n + 1) + 126) // 127        # groups for amax index i (i + 1 values)
    amax_of = np.repeat(np.arange(n, dtype=np.int32), per)
    first = np.concatenate([[0], np.cumsum(per)[:-1]]).astype(np.int32)
    k = np.arange(amax_of.size, dtype=np.int32) - np.repeat(first, per)
    col = np.arange(127, dtype=np.int32)[None, :]
    for c0 in range(0, amax_of.size, CHUNK):
        a, kk = amax_of[c0:c0 + CHUNK], k[c0:c0 + CHUNK]
        g = np.zeros(((a.size + 15) // 16 * 16, 128), np.int16)
        g[:a.size, 0] = a + 1
        j = kk[:, None] * 127 + col                 # value index 0..i, past it -> +0.0
        g[:a.size, 1:] = np.where(j <= a[:, None], j + 1, 0)
        yield g


def _groups_special():
    """Groups whose amax is NaN (0x7FC0) or +Inf (0x7F80), each with every bf16 pattern x
    (NaN groups) or every non-NaN pattern (Inf groups) in the other 127 entries."""
    allb = np.arange(-32768, 32768, dtype=np.int32).astype(np.int16)
    u = allb.view(np.uint16)
    nonnan = allb[(u & 0x7FFF) <= 0x7F80]
    out = []
    for head, xs in ((0x7FC0, allb), (0x7F80, nonnan)):
        pad = (-xs.size) % 127
        xs = np.concatenate([xs, np.zeros(pad, np.int16)]).reshape(-1, 127)
        g = np.empty((xs.shape[0], 128), np.int16)
        g[:, 0] = np.int16(head)
        g[:, 1:] = xs
        out.append(g)
    g = np.concatenate(out)
    yield np.concatenate([g, np.zeros(((-g.shape[0]) % 16, 128), np.int16)])


def _div32(a, b):
    """float32 a / b rounded to nearest, through float64: the float64 quotient of two float32
    values rounded to float32 is the correctly rounded float32 quotient (double rounding is
    innocuous from 53 >= 2 x 24 + 2 bits). Tensor by tensor: torch turns a division by a
    Python scalar into a multiplication by its reciprocal."""
    return (a.double() / b.double()).float()


def _reference(xb):
    """codes and scales of the quant from bf16 bits [G, 128] with IEEE division."""
    x = xb.view(torch.bfloat16).float()
    amax_bits = (xb.int() & 0x7FFF).amax(1)         # the kernels' max over |x| bit patterns
    amax = (amax_bits << 16).view(torch.float32)
    s = _div32(amax, torch.full_like(amax, 448.0))
    s = torch.where(s > float(MIN_SCALE), s, torch.full_like(s, float(MIN_SCALE)))
    q = torch.fmin(torch.fmax(_div32(x, s[:, None].expand_as(x)),
                              torch.tensor(-448.0, device=DEV)),
                   torch.tensor(448.0, device=DEV))
    return q.to(torch.float8_e4m3fn).view(torch.uint8), s


@pytest.mark.parametrize("domain", ["finite", "special"])
def test_quant_equals_ieee_division_on_every_input(pkg, domain):
    chunks = _groups_finite() if domain == "finite" else _groups_special()
    bad_q = bad_s = pairs = 0
    for c, groups in enumerate(chunks):
        for sign in (0, 1):
            xb = torch.from_numpy(groups).to(DEV)
            if sign:
                xb = xb ^ torch.tensor(-32768, dtype=torch.int16, device=DEV)   # flip signs
            rows = xb.shape[0]
            pairs += rows * 127
            gpu_case(f"quant exhaustive {domain} chunk {c} sign {sign}: {rows} groups")
            q, s = pkg.ops.fp8_quant_group(xb.view(torch.bfloat16).reshape(rows // 16, 2048))
            q_ref, s_ref = _reference(xb)
            bad_q += int((q.view(torch.uint8).reshape(rows, 128) != q_ref).sum())
            bad_s += int((s.reshape(-1).view(torch.int32) != s_ref.view(torch.int32)).sum())
    assert pairs >= (2 * 532668480 if domain == "finite" else 2 * 130000)
    assert bad_s == 0, f"{bad_s} scales differ from amax / 448"
    assert bad_q == 0, f"{bad_q} codes differ from the IEEE-division quant"


def test_bf16_rounding_one_instruction_equals_integer_rounding(pkg):
    """The prefill SiLU-mul-quant epilogue rounds float32 to bf16 with gfx950's
    v_cvt_pk_bf16_f32; every other kernel, and the oracle, with integer nearest-even rounding
    (NaN kept, quiet bit set). rlu_selftest_bf16 runs both over all 2^32 float32 bit patterns:
    not one may differ, or the prefill layer's bits would depend on which kernel ran."""
    import ctypes
    bad = torch.zeros(1, dtype=torch.int64, device=DEV)
    gpu_case("bf16 rounding self-test over 2^32 inputs")
    rc = pkg.lib().rlu_selftest_bf16(ctypes.c_void_p(bad.data_ptr()),
                                     ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    torch.cuda.synchronize()
    assert int(bad.item()) == 0
    assert pkg.lib().rlu_selftest_bf16(None, None) == -1
