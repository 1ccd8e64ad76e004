"""GPU parity of the W4 draft lm_head (int4 g128, bf16 scale + integer zero) through the C-ABI.

* rlu_gemm_w4_m16 against the oracle's float64 GEMV over the SAME packed bytes (unpacked by
  the oracle's own formula walk), within 5e-3 of max|ref| (tests/k3/w4_verify.py:54-65 bar),
  at vocab 151936 x 2560 for M in {1, 4, 8}, plus M = 16 and the 16-row chunking at M = 20;
* small and edge shapes: N not a multiple of 16 (zero-row padding), K = 4096 (the LDS limit),
  M = 1 with one strip;
* the GPU packer equals the CPU packer (codes, scales, zeros), up to float32 clip ties;
* HIP-graph replay equals eager; bad arguments return codes.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import gpu_case
from oracle import fp8, w4 as ow4

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 5e-3


@pytest.fixture(scope="module")
def pw4(pkg):
    return pkg.w4


def ref_logits(packed, x):
    wq = packed.wq.cpu().numpy()
    sz = packed.sz.cpu().numpy()
    q, s, z = ow4.unpack(wq, sz, packed.n_pad, packed.k)
    return ow4.gemv(x, q[:packed.n], s[:packed.n], z[:packed.n])


def dequant32(packed):
    """float32 dequant of the packed bytes, by the oracle's unpacker (kept once for the big
    head: float64 would be 3 GB)."""
    q, s, z = ow4.unpack(packed.wq.cpu().numpy(), packed.sz.cpu().numpy(), packed.n_pad,
                         packed.k)
    n, k = packed.n, packed.k
    w = (q[:n].reshape(n, k // 128, 128).astype(np.float32) - z[:n, :, None]) * s[:n, :, None]
    return w.reshape(n, k)


def rel(got, ref):
    return float(np.abs(got - ref).max() / np.abs(ref).max())


@pytest.fixture(scope="module")
def big(pw4):
    N, K = 151936, 2560
    g = torch.Generator(device=DEV).manual_seed(5)
    w = torch.randn(N, K, device=DEV, generator=g) * 0.02
    packed = pw4.pack_w4a16(w)
    del w
    return packed, dequant32(packed)


@pytest.mark.parametrize("M", [1, 4, 8, 16, 20])
def test_w4_lmhead_vs_oracle(pw4, big, M):
    packed, wd = big
    rng = np.random.default_rng(M)
    x = fp8.bf16_round(rng.standard_normal((M, packed.k)).astype(np.float32))
    gpu_case(f"w4 lm_head M={M}")
    y = pw4.gemm_w4a16(torch.from_numpy(x).to(torch.bfloat16).to(DEV), packed)
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    ref = (x @ wd.T).astype(np.float64)     # float32 accumulation: ~1e-6 relative
    assert rel(got, ref) <= TOL
    # the argmax agrees unless the reference's top two are within one bf16 step
    am, ar = got.argmax(1), ref.argmax(1)
    for r in range(M):
        if am[r] != ar[r]:
            assert ref[r, ar[r]] - ref[r, am[r]] <= 2 ** -7 * abs(ref[r, ar[r]])


@pytest.mark.parametrize("N,K,M", [(40, 256, 3), (16, 128, 1), (1000, 4096, 5), (4096, 512, 16)])
def test_w4_shapes(pw4, N, K, M):
    g = torch.Generator(device=DEV).manual_seed(N + K)
    w = torch.randn(N, K, device=DEV, generator=g) * 0.05
    packed = pw4.pack_w4a16(w)
    x = fp8.bf16_round(np.random.default_rng(K).standard_normal((M, K)).astype(np.float32))
    gpu_case(f"w4 shape N={N} K={K} M={M}")
    y = pw4.gemm_w4a16(torch.from_numpy(x).to(torch.bfloat16).to(DEV), packed)
    torch.cuda.synchronize()
    assert y.shape == (M, N)
    assert rel(y.float().cpu().numpy(), ref_logits(packed, x)) <= TOL


def test_w4_gpu_packer_equals_cpu(pw4):
    g = torch.Generator().manual_seed(11)
    w = torch.randn(256, 1024, generator=g) * 0.02
    gpu_case("w4 packer gpu vs cpu")
    pg = pw4.pack_w4a16(w.to(DEV))
    pc = pw4.pack_w4a16(w)
    sg, sc = pg.sz.cpu().numpy(), pc.sz.numpy()
    same = sg == sc
    assert same.mean() > 0.999
    qg = pw4.unpack_codes(pg.wq.cpu()).numpy().reshape(256, 8, 128)
    qc = pw4.unpack_codes(pc.wq).numpy().reshape(256, 8, 128)
    nt, gg, r = np.nonzero(same)
    assert np.array_equal(qg[nt * 16 + r, gg], qc[nt * 16 + r, gg])


def test_w4_graph_replay(pw4):
    g = torch.Generator(device=DEV).manual_seed(3)
    packed = pw4.pack_w4a16(torch.randn(2048, 2560, device=DEV, generator=g) * 0.02)
    M = 4
    xs = [torch.randn(M, 2560, device=DEV, generator=g).to(torch.bfloat16) for _ in range(3)]
    x = torch.zeros_like(xs[0])
    y = torch.empty((M, packed.n_pad), dtype=torch.bfloat16, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        pw4.gemm_w4a16(x, packed, out=y)
    torch.cuda.current_stream().wait_stream(side)
    gr = torch.cuda.CUDAGraph()
    gpu_case("w4 graph capture")
    with torch.cuda.graph(gr):
        pw4.gemm_w4a16(x, packed, out=y)
    for xi in xs:
        x.copy_(xi)
        gr.replay()
        torch.cuda.synchronize()
        ye = pw4.gemm_w4a16(xi, packed)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ye.view(torch.int16))


def test_w4_return_codes(pkg):
    P = ctypes.c_void_p
    b = torch.empty(1 << 16, dtype=torch.uint8, device=DEV)
    s = P(torch.cuda.current_stream().cuda_stream)
    f = pkg.lib().rlu_gemm_w4_m16
    p = P(b.data_ptr())
    assert f(p, 0, 128, p, p, p, 16, 0, s) == -1          # M < 1
    assert f(p, 17, 128, p, p, p, 16, 0, s) == -1         # M > 16
    assert f(p, 1, 100, p, p, p, 16, 0, s) == -2          # K % 128
    assert f(p, 1, 128, p, p, p, 48, 0, s) == -2          # N % 32
    assert f(p, 1, 4224, p, p, p, 32, 0, s) == -2         # K > 4096
    assert f(p, 1, 128, p, p, p, 16, 17, s) == -1         # wv
