"""GPU parity of the W4 draft lm_head (int4 g128, bf16 scale + integer zero) through the C-ABI.

* rlu_gemm_w4_m16 against the oracle's float64 GEMV over the SAME packed bytes (unpacked by
  the oracle's own formula walk), within 5e-3 of max|ref| (tests/k3/w4_verify.py:54-65 bar),
  at vocab 151936 x 2560 for M in {1, 4, 8}, plus M = 16 and the 16-row chunking at M = 20;
* small and edge shapes: N not a multiple of 16 (zero-row padding), K = 4096 (the LDS limit),
  M = 1 with one strip;
* the packing kernel (rlu_pack_w4) writes the oracle's bytes exactly -- codes, scales and
  zeros -- for bf16 / f32 / f16 weights, N not a multiple of 16 or 32, K up to 4096, special
  groups (zero, constant, one-sided, offset past the zero range), and on sampled strips of the
  151936 x 2560 head;
* the draft_w4_lmhead_gemm op (torch.ops) equals the C-ABI call bit for bit, eagerly and
  inside a captured graph; HIP-graph replay equals eager; bad arguments return codes.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import check_argmax, gpu_case
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
    check_argmax(got, ref, f"w4 lm_head M={M}")


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


def _oracle_bytes(w32: np.ndarray, n_pad: int):
    n, k = w32.shape
    wp = np.zeros((n_pad, k), np.float32)
    wp[:n] = w32
    q, s, z = ow4.quantize_w4(wp)
    return ow4.pack_codes(q), ow4.pack_sz(s, z)


def _special_weight(N, K, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w[0, :128] = 0.0                                  # all zero
    w[1, :128] = 0.75                                 # constant positive
    w[2, 128:256] = -0.3                              # constant negative
    w[3, :128] = np.linspace(0.5, 1.0, 128)           # one-sided
    w[4, :128] = np.linspace(100.0, 100.01, 128)      # offset past the zero range
    w[5, :] = rng.standard_t(2, K) * 0.05             # heavy tails
    return w


@pytest.mark.parametrize("N,K,dtype", [(256, 1024, torch.float32), (40, 256, torch.bfloat16),
                                       (37, 128, torch.float16), (1000, 4096, torch.bfloat16),
                                       (96, 2560, torch.float32)])
def test_w4_packer_bit_exact_vs_oracle(pw4, N, K, dtype):
    w = torch.from_numpy(_special_weight(N, K, N + K)).to(dtype)
    w32 = w.float().numpy()                 # the values the kernel reads
    gpu_case(f"w4 pack N={N} K={K} {dtype}")
    p = pw4.pack_w4a16(w.to(DEV))
    torch.cuda.synchronize()
    wq, sz = _oracle_bytes(w32, p.n_pad)
    assert np.array_equal(p.wq.cpu().numpy(), wq)
    assert np.array_equal(p.sz.cpu().numpy(), sz)
    q, s, z = pw4.quantize_w4(w.to(DEV))
    q0, s0, z0 = ow4.quantize_w4(w32)
    assert np.array_equal(q.cpu().numpy(), q0)
    assert np.array_equal(s.float().cpu().numpy(), s0) and np.array_equal(z.cpu().numpy(), z0)


def test_w4_packer_bit_exact_on_the_head(pw4, big):
    """The 151936 x 2560 head packed once (the `big` fixture, f32 weights from seed 5): 64
    sampled 16-row strips, re-quantized by the oracle, match byte for byte."""
    packed, _ = big
    N, K = 151936, 2560
    g = torch.Generator(device=DEV).manual_seed(5)
    w = torch.randn(N, K, device=DEV, generator=g) * 0.02
    strips = np.random.default_rng(1).choice(N // 16, 64, replace=False)
    rows = (strips[:, None] * 16 + np.arange(16)[None, :]).reshape(-1)
    w32 = w[torch.from_numpy(rows).to(DEV)].cpu().numpy()
    del w
    q, s, z = ow4.quantize_w4(w32)
    wq = ow4.pack_codes(q).reshape(64, K // 128, 64, 16)
    sz = ow4.pack_sz(s, z).reshape(64, K // 128, 16)
    idx = torch.from_numpy(strips).to(DEV)
    assert np.array_equal(packed.wq[idx].cpu().numpy(), wq)
    assert np.array_equal(packed.sz[idx].cpu().numpy(), sz)


def test_w4_packer_deterministic(pw4):
    g = torch.Generator(device=DEV).manual_seed(2)
    w = torch.randn(4096, 2560, device=DEV, generator=g).to(torch.bfloat16) * 0.02
    a, b = pw4.pack_w4a16(w), pw4.pack_w4a16(w)
    torch.cuda.synchronize()
    assert torch.equal(a.wq, b.wq) and torch.equal(a.sz, b.sz)


def test_w4_op_equals_c_abi(pw4, pkg):
    """torch.ops.<ns>.draft_w4_lmhead_gemm (kernels/draft_w4_lmhead.py:351-390) equals the
    C-ABI call bit for bit, eagerly and replayed from a captured graph; M > 16 and N not a
    multiple of 32 go through the same op."""
    op = getattr(torch.ops, pkg.lru.OPS_NAMESPACE).draft_w4_lmhead_gemm
    g = torch.Generator(device=DEV).manual_seed(4)
    packed = pw4.pack_w4a16(torch.randn(2000, 2560, device=DEV, generator=g) * 0.02)
    for M in (1, 5, 20):
        x = torch.randn(M, 2560, device=DEV, generator=g).to(torch.bfloat16)
        gpu_case(f"w4 op eager M={M}")
        y_op = op(x, packed.wq, packed.sz, packed.n, packed.k, 0, 0, 0, 0)
        y_c = torch.empty((M, packed.n_pad), dtype=torch.bfloat16, device=DEV)
        pw4._gemm_into(x, packed.wq, packed.sz, packed.k, y_c, 0)
        torch.cuda.synchronize()
        assert y_op.shape == (M, 2000) and y_op.is_contiguous()
        assert torch.equal(y_op.view(torch.int16), y_c[:, :2000].view(torch.int16))
    M = 4
    xs = [torch.randn(M, 2560, device=DEV, generator=g).to(torch.bfloat16) for _ in range(3)]
    x = xs[0].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        op(x, packed.wq, packed.sz, packed.n, packed.k, 0, 0, 0, 0)
    torch.cuda.current_stream().wait_stream(side)
    gr = torch.cuda.CUDAGraph()
    gpu_case("w4 op graph capture")
    with torch.cuda.graph(gr):
        y = op(x, packed.wq, packed.sz, packed.n, packed.k, 0, 0, 0, 0)
    for xi in xs:
        x.copy_(xi)
        gr.replay()
        torch.cuda.synchronize()
        y_c = torch.empty((M, packed.n_pad), dtype=torch.bfloat16, device=DEV)
        pw4._gemm_into(xi, packed.wq, packed.sz, packed.k, y_c, 0)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), y_c[:, :2000].view(torch.int16))
    with pytest.raises(ValueError):
        op(x, packed.wq, packed.sz, packed.n, packed.k, -1, 0, 0, 0)


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
