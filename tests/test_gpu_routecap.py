"""GPU: the routing capture through rlu_route_capture (tools/routecap/routecap.py semantics),
eager and recorded into a HIP graph, against a host model of the ring, and the file it writes.
The capture hook of LruMoELayer is exercised inside a captured layer step in
test_gpu_layer.py::test_layer_overlap_graph_replay."""
from __future__ import annotations

import time

import numpy as np
import pytest

from conftest import gpu_case

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def rc(pkg):
    from importlib import import_module
    return import_module(pkg.__name__ + ".routecap")


class RingModel:
    """The capture on the host: what the device ring must hold."""

    def __init__(self, nlayer, ring, width):
        self.ctr = 0
        self.ids = np.full((nlayer, ring, width), -1, np.int16)
        self.step = np.full(ring, -1, np.int64)
        self.ring = ring

    def capture(self, layer, ids):
        if layer == 0:
            self.ctr += 1
            self.step[self.ctr % self.ring] = self.ctr
        row = self.ids[layer, self.ctr % self.ring]
        row[:] = -1
        row[:ids.size] = ids.reshape(-1).astype(np.int16)


def _check(r, m):
    assert int(r.ctr.item()) == m.ctr
    assert np.array_equal(r.ring_step.cpu().numpy(), m.step)
    assert np.array_equal(r.ring_ids.cpu().numpy(), m.ids)


def test_capture_eager_matches_the_model(rc):
    L, k, ring, maxrows, E = 3, 10, 8, 4, 512
    r = rc.RouteRing(L, k, DEV, ring=ring, maxrows=maxrows)
    m = RingModel(L, ring, maxrows * k)
    rng = np.random.default_rng(0)
    for t in range(21):                          # wraps the 8-slot ring twice
        rows = 1 + t % maxrows
        gpu_case(f"routecap eager step {t} rows {rows}")
        for li in range(L):
            ids = rng.integers(0, E, (rows, k)).astype(np.int32)
            r.capture(li, torch.from_numpy(ids).to(DEV))
            m.capture(li, ids)
        torch.cuda.synchronize()
        _check(r, m)
    # a prefill-wide step and another top-k are not captured: the counter stays
    r.capture(0, torch.zeros((maxrows + 1, k), dtype=torch.int32, device=DEV))
    r.capture(0, torch.zeros((2, k + 1), dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    _check(r, m)


def test_capture_rejects_bad_arguments(rc, pkg):
    import ctypes
    lib = pkg.lib()
    r = rc.RouteRing(2, 4, DEV, ring=4, maxrows=2)
    ids = torch.zeros(8, dtype=torch.int32, device=DEV)
    P = ctypes.c_void_p
    bufs = [P(r.ring_ids.data_ptr()), P(r.ring_step.data_ptr()), P(r.ctr.data_ptr())]
    st = P(torch.cuda.current_stream().cuda_stream)
    assert lib.rlu_route_capture(P(ids.data_ptr()), 9, 0, 2, 4, 8, *bufs, st) == -1   # n > width
    assert lib.rlu_route_capture(P(ids.data_ptr()), 8, 2, 2, 4, 8, *bufs, st) == -1   # layer
    assert lib.rlu_route_capture(P(ids.data_ptr()), 8, 0, 2, 0, 8, *bufs, st) == -1   # ring
    assert lib.rlu_route_capture(P(ids.data_ptr()), 8, 0, 2, 4, 8, P(0), bufs[1], bufs[2],
                                 st) == -1
    torch.cuda.synchronize()
    assert int(r.ctr.item()) == 0
    with pytest.raises(TypeError):
        r.capture(0, torch.zeros((2, 4), dtype=torch.int64, device=DEV))


def test_capture_in_a_graph_polls_and_writes_the_file(rc, tmp_path):
    """routecap.py's reason to exist: the capture keeps recording on every graph replay. A
    warm-up step, then 30 replays of a graph of three layers' captures with new routing copied
    into the static inputs before each, a poll every 5 replays (ring 8: nothing lost), then 12
    more replays before the next poll: steps 31..35 are overwritten before it reads them."""
    L, k, ring, maxrows, E, rows = 3, 10, 8, 4, 512, 4
    r = rc.RouteRing(L, k, DEV, ring=ring, maxrows=maxrows)
    m = RingModel(L, ring, maxrows * k)
    static = [torch.zeros((rows, k), dtype=torch.int32, device=DEV) for _ in range(L)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):                   # step 1, eager, off the capture
        for li in range(L):
            r.capture(li, static[li])
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for li in range(L):
        m.capture(li, static[li].cpu().numpy())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for li in range(L):
            r.capture(li, static[li])
    rng = np.random.default_rng(1)
    want = {1: [x.cpu().numpy() for x in static]}
    gpu_case("routecap graph replays")
    for t in range(30):                          # steps 2..31
        new = [rng.integers(0, E, (rows, k)).astype(np.int32) for _ in range(L)]
        for li in range(L):
            static[li].copy_(torch.from_numpy(new[li]))
            m.capture(li, new[li])
        g.replay()
        want[m.ctr] = new
        if t % 5 == 4:
            torch.cuda.synchronize()
            r.poll()
    torch.cuda.synchronize()
    _check(r, m)
    got = r.routes()
    assert list(got["steps"]) == list(range(1, 31))       # step 31, the newest, is unfinished
    assert int(got["lost_to_wrap"]) == 0
    for i, v in enumerate(got["steps"]):
        for li in range(L):
            assert np.array_equal(got["ids"][i, li, :rows * k], want[int(v)][li].reshape(-1))
            assert (got["ids"][i, li, rows * k:] == -1).all()
    for _ in range(12):                          # steps 32..43: the ring keeps 36..43
        for li in range(L):
            static[li].copy_(torch.from_numpy(rng.integers(0, E, (rows, k)).astype(np.int32)))
        g.replay()
    torch.cuda.synchronize()
    info = r.flush(out_dir=str(tmp_path), rank=0)
    assert info["ctr"] == 43 and info["saved"] == 37 and info["lost_to_wrap"] == 5
    back = rc.load_routes(tmp_path / "routes_rank0.npz")
    assert list(back["steps"]) == list(range(1, 31)) + list(range(36, 43))
    assert int(back["nlayer"]) == L and int(back["topk"]) == k and int(back["ring"]) == ring
    assert int(back["maxrows"]) == maxrows and int(back["ctr"]) == 43
    assert back["ids"].dtype == np.int16 and back["ids"].shape == (37, L, maxrows * k)
    assert int(back["lost_to_wrap"]) == 5


def test_dumper_thread_flushes_and_stops(rc, tmp_path):
    """The background dumper writes routes_rank<N>.npz on its own while steps run, and
    stop_dumper ends the thread and writes a last flush holding every finished step."""
    L, k, rows = 2, 10, 3
    r = rc.RouteRing(L, k, DEV, ring=64, maxrows=4)
    rng = np.random.default_rng(7)
    gpu_case("routecap dumper thread")
    r.start_dumper(every_s=0.02, out_dir=str(tmp_path))
    for _ in range(20):
        for li in range(L):
            r.capture(li, torch.from_numpy(rng.integers(0, 512, (rows, k)).astype(np.int32))
                      .to(DEV))
        torch.cuda.synchronize()
        time.sleep(0.005)
    r.stop_dumper(out_dir=str(tmp_path))
    assert r._thread is None and r.dumps >= 2
    files = sorted(p.name for p in tmp_path.iterdir())
    assert files == [f"routes_rank{rc._rank()}.npz"], files    # no staging file left behind
    back = rc.load_routes(tmp_path / files[0])
    assert list(back["steps"]) == list(range(1, 20)) and int(back["ctr"]) == 20
