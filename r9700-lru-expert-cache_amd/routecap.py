"""Routing capture under HIP graphs: every MoE layer's topk_ids, per decode step, into a device
ring that a captured graph keeps filling on every replay, read back to the host in between.

Mirrors tools/routecap/routecap.py (the capture fn :83-100, the host flush :119-152, the file it
writes and its environment variables). The device side is one launch per layer of
rlu_route_capture (include/rlu.h) instead of five torch ops, so a capture costs one kernel
boundary per layer. The ring is allocated when the RouteRing is made, never inside a capture.

File (np.savez, one per rank, routes_rank<N>.npz), as the reference writes it:
    steps int64 [n]                      step number of each saved slot, ascending
    ids int16 [n, nlayer, maxrows*topk]  routed expert ids, -1 past the step's rows
    nlayer, topk, maxrows, ring, ctr, lost_to_wrap   int64 scalars
lost_to_wrap counts the steps in [1, last saved] that the ring overwrote before a flush read
them. The reference's formula (routecap.py:135-136) also counts step 0, which is never
written (the counter is 1 at the first step), so its value is this one plus one.

Env (defaults as the reference's):
    ROUTECAP_DIR      where routes_rank<N>.npz goes (default: the current directory)
    ROUTECAP_RING     steps held on the device (1024)
    ROUTECAP_MAXROWS  steps with more rows than this are not captured: prefill (32)
    ROUTECAP_DUMP_S   seconds between host flushes of the background dumper (20)
"""
from __future__ import annotations

import ctypes
import os
import threading
import time

import numpy as np
import torch

from ._lib import check, lib, stream_ptr

RING = int(os.environ.get("ROUTECAP_RING", "1024"))
MAXROWS = int(os.environ.get("ROUTECAP_MAXROWS", "32"))
DUMP_S = float(os.environ.get("ROUTECAP_DUMP_S", "20"))
OUT_DIR = os.environ.get("ROUTECAP_DIR", ".")


def _rank() -> int:
    """routecap.py:103-116: the torch.distributed rank, else the launcher's, else the device."""
    import torch.distributed as dist
    if dist.is_available() and dist.is_initialized():
        return dist.get_rank()
    for v in ("VLLM_WORKER_RANK", "RANK", "LOCAL_RANK"):
        if os.environ.get(v):
            return int(os.environ[v])
    return torch.cuda.current_device()


def complete_slots(steps: np.ndarray, ctr: int, high: int) -> list[int]:
    """The ring slots a poll keeps, in ascending step order (routecap.py:127-133): written
    (step >= 0), newer than the last saved step `high`, and finished -- below the counter
    `ctr`, since the slot of step ctr may still be being written."""
    out = []
    for s in np.argsort(steps, kind="stable"):
        v = int(steps[s])
        if v <= high or v < 0 or v >= ctr:
            continue
        out.append(int(s))
        high = v
    return out


class RouteRing:
    """The device ring of routecap.py's _State plus the host trace it accumulates.

    ring_ids int16 [nlayer, ring, maxrows * topk], ring_step int64 [ring] (-1 = never
    written), ctr int64 [1]: the step number, advanced by each step's layer-0 capture."""

    def __init__(self, nlayer: int, topk: int, device="cuda", ring: int = RING,
                 maxrows: int = MAXROWS):
        if nlayer <= 0 or topk <= 0 or ring <= 0 or maxrows <= 0:
            raise ValueError("nlayer, topk, ring and maxrows must be positive")
        self.dev, self.nlayer, self.topk = torch.device(device), nlayer, topk
        self.ring, self.maxrows = ring, maxrows
        self.width = maxrows * topk
        self.ctr = torch.zeros(1, dtype=torch.int64, device=self.dev)
        self.dev = self.ctr.device                  # "cuda" -> "cuda:<index>"
        self.ring_ids = torch.full((nlayer, ring, self.width), -1, dtype=torch.int16,
                                   device=self.dev)
        self.ring_step = torch.full((ring,), -1, dtype=torch.int64, device=self.dev)
        self.dump_stream = torch.cuda.Stream(device=self.dev)
        self.saved_steps: list[int] = []
        self.saved_ids: list[np.ndarray] = []
        self.high = -1          # the highest step already saved
        self.dumps = 0
        self._lock = threading.Lock()
        self._thread = None

    # -- device side ------------------------------------------------------------------------
    def capture(self, layer: int, topk_ids: torch.Tensor) -> None:
        """routecap.py:83-100 for router `layer`: steps wider than maxrows rows (prefill) or
        with another top-k are skipped, before the counter moves."""
        if layer < 0 or layer >= self.nlayer:
            return
        rows, k = topk_ids.shape[0], topk_ids.shape[-1]
        if rows > self.maxrows or k != self.topk:
            return
        ids = topk_ids.reshape(-1)
        if ids.dtype != torch.int32 or not ids.is_contiguous():
            raise TypeError("topk_ids must be contiguous int32 (as the LRU entry points take)")
        if ids.device != self.dev:
            raise ValueError(f"topk_ids on {ids.device}, ring on {self.dev}")
        check(lib().rlu_route_capture(ctypes.c_void_p(ids.data_ptr()), ids.numel(), layer,
                                      self.nlayer, self.ring, self.width,
                                      ctypes.c_void_p(self.ring_ids.data_ptr()),
                                      ctypes.c_void_p(self.ring_step.data_ptr()),
                                      ctypes.c_void_p(self.ctr.data_ptr()), stream_ptr()),
              "rlu_route_capture")

    def fn(self, layer: int):
        """The capture fn for router `layer` (routecap.py:_make_fn)."""
        return lambda topk_ids: self.capture(layer, topk_ids)

    # -- host side --------------------------------------------------------------------------
    def poll(self) -> int:
        """Copy the ring to the host on the dump stream and keep every newly completed slot:
        a slot is complete once a later step has started (its step number is below the
        counter); the newest one may still be being written. Returns the counter read."""
        with torch.cuda.stream(self.dump_stream):
            ctr = int(self.ctr.item())
            steps = self.ring_step.to("cpu", copy=True).numpy()
            ring = self.ring_ids.to("cpu", copy=True).numpy()
        self.dump_stream.synchronize()
        with self._lock:
            for s in complete_slots(steps, ctr, self.high):
                self.saved_steps.append(int(steps[s]))
                self.saved_ids.append(ring[:, s, :].copy())
                self.high = int(steps[s])
            self.dumps += 1
        return ctr

    def lost_to_wrap(self) -> int:
        with self._lock:
            return (self.saved_steps[-1] - len(self.saved_steps)) if self.saved_steps else 0

    def routes(self, ctr: int | None = None) -> dict[str, np.ndarray]:
        """The host trace in the file's layout."""
        with self._lock:
            ids = (np.stack(self.saved_ids) if self.saved_ids
                   else np.zeros((0, self.nlayer, self.width), dtype=np.int16))
            steps = np.asarray(self.saved_steps, dtype=np.int64)
        if ctr is None:
            ctr = int(self.ctr.item())
        return dict(steps=steps, ids=ids, nlayer=np.int64(self.nlayer),
                    topk=np.int64(self.topk), maxrows=np.int64(self.maxrows),
                    ring=np.int64(self.ring), ctr=np.int64(ctr),
                    lost_to_wrap=np.int64(self.lost_to_wrap()))

    def flush(self, out_dir: str | None = None, rank: int | None = None) -> dict:
        """routecap.py:119-152: poll, then rewrite routes_rank<rank>.npz atomically (a temporary
        file renamed over the old one)."""
        ctr = self.poll()
        out_dir = OUT_DIR if out_dir is None else out_dir
        os.makedirs(out_dir, exist_ok=True)
        p = os.path.join(out_dir, f"routes_rank{_rank() if rank is None else rank}.npz")
        tmp = p + ".tmp"
        r = self.routes(ctr)
        with open(tmp, "wb") as fh:        # a bare path would get ".npz" appended
            np.savez(fh, **r)
        os.replace(tmp, p)
        return dict(path=p, ctr=ctr, saved=int(r["steps"].size),
                    lost_to_wrap=int(r["lost_to_wrap"]))

    def start_dumper(self, every_s: float = DUMP_S, out_dir: str | None = None):
        """routecap.py:155-161: a daemon thread that flushes every every_s seconds."""
        def loop():
            torch.cuda.set_device(self.dev)
            while True:
                time.sleep(every_s)
                try:
                    self.flush(out_dir)
                except Exception as exc:                            # noqa: BLE001
                    print(f"[routecap] flush failed: {type(exc).__name__}: {exc}", flush=True)
        if self._thread is None:
            self._thread = threading.Thread(target=loop, daemon=True, name="routecap")
            self._thread.start()
        return self._thread

    def status(self) -> dict:
        """routecap.py:189-197 (routecap_status)."""
        return dict(installed=self.nlayer, armed=True, nlayer=self.nlayer, topk=self.topk,
                    ctr=int(self.ctr.item()), saved=len(self.saved_steps), dumps=self.dumps)


def load_routes(path) -> dict[str, np.ndarray]:
    """A routes_rank<N>.npz (this module's or the reference's), without unpickling."""
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def decode_counts(routes: dict, num_experts: int) -> np.ndarray:
    """Routings per (layer, expert) over the captured steps: int64 [nlayer, E]. Only decode
    steps are captured; -1 padding and ids outside [0, E) are not counted."""
    ids = np.asarray(routes["ids"]).astype(np.int64)
    n, L, _ = ids.shape
    out = np.zeros((L, num_experts), dtype=np.int64)
    for li in range(L):
        v = ids[:, li, :].reshape(-1)
        v = v[(v >= 0) & (v < num_experts)]
        out[li] = np.bincount(v, minlength=num_experts)
    return out


def hot_profile_from_routes(routes: dict, num_experts: int, layer_ids=None, source: str = ""):
    """A capture -> the warm-start profile (hot_profile's format), the step the reference runs
    through tools/routecap/build_hot_profile.py."""
    from . import hot_profile
    return hot_profile.build(decode_counts(routes, num_experts), layer_ids=layer_ids,
                             source=source, top_k=int(routes["topk"]))
