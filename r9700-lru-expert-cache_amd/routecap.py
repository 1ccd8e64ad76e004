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
import io
import os
import tempfile
import threading
import warnings

import numpy as np
import torch

from ._lib import check, lib, stream_ptr

RING = int(os.environ.get("ROUTECAP_RING", "1024"))
MAXROWS = int(os.environ.get("ROUTECAP_MAXROWS", "32"))
DUMP_S = float(os.environ.get("ROUTECAP_DUMP_S", "20"))
OUT_DIR = os.environ.get("ROUTECAP_DIR", ".")


def _rank() -> int:
    """The N of routes_rank<N>.npz (the precedence of routecap.py:103-116): a live process
    group names it; failing that, the launcher's variables in the order VLLM_WORKER_RANK, RANK,
    LOCAL_RANK; failing those, the current device index."""
    dist = torch.distributed
    if dist.is_available() and dist.is_initialized():
        return dist.get_rank()
    set_vars = [name for name in ("VLLM_WORKER_RANK", "RANK", "LOCAL_RANK") if os.environ.get(name)]
    return int(os.environ[set_vars[0]]) if set_vars else torch.cuda.current_device()


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
        # host mirrors of the ring, pinned once here so that a poll allocates nothing and its
        # copies run asynchronously on the dump stream
        self._h_ctr = torch.empty(1, dtype=torch.int64, pin_memory=True)
        self._h_step = torch.empty(ring, dtype=torch.int64, pin_memory=True)
        self._h_ids = torch.empty((nlayer, ring, self.width), dtype=torch.int16, pin_memory=True)
        self._copied = torch.cuda.Event()
        self.saved_steps: list[int] = []
        self.saved_ids: list[np.ndarray] = []
        self.high = -1          # the highest step already saved
        self.dumps = 0
        self._lock = threading.Lock()
        self._thread = None
        self._stop = threading.Event()

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
        """Bring the ring to the host and append every slot that completed since the last poll.
        The counter is copied first, then the step numbers and ids, all on the dump stream, so
        a slot whose step is below the copied counter was finished before its copy began (the
        capture of a later step has started); the slot of the counter's own step may be half
        written and waits for the next poll. Returns the counter."""
        with torch.cuda.stream(self.dump_stream):
            self._h_ctr.copy_(self.ctr, non_blocking=True)
            self._h_step.copy_(self.ring_step, non_blocking=True)
            self._h_ids.copy_(self.ring_ids, non_blocking=True)
            self._copied.record(self.dump_stream)
        self._copied.synchronize()
        ctr = int(self._h_ctr[0])
        steps = self._h_step.numpy()
        with self._lock:
            keep = complete_slots(steps, ctr, self.high)
            if keep:
                self.saved_steps.extend(int(steps[s]) for s in keep)
                self.saved_ids.extend(self._h_ids.numpy()[:, keep, :].transpose(1, 0, 2))
                self.high = self.saved_steps[-1]
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
        """Poll, then replace routes_rank<rank>.npz (routecap.py:119-152) so that a reader
        never sees a partial file: the archive is built in memory, written to a fresh file
        beside the target and renamed over it."""
        ctr = self.poll()
        target_dir = OUT_DIR if out_dir is None else out_dir
        os.makedirs(target_dir, exist_ok=True)
        rank = _rank() if rank is None else rank
        path = os.path.join(target_dir, f"routes_rank{rank}.npz")
        r = self.routes(ctr)
        blob = io.BytesIO()
        np.savez(blob, **r)
        fd, staged = tempfile.mkstemp(prefix=f".routes_rank{rank}.", dir=target_dir)
        try:
            with os.fdopen(fd, "wb") as fh:
                fh.write(blob.getbuffer())
            os.replace(staged, path)
        except BaseException:
            if os.path.exists(staged):
                os.unlink(staged)
            raise
        return dict(path=path, ctr=ctr, saved=int(r["steps"].size),
                    lost_to_wrap=int(r["lost_to_wrap"]))

    def start_dumper(self, every_s: float = DUMP_S, out_dir: str | None = None):
        """A daemon thread that flushes every every_s seconds until stop_dumper()
        (routecap.py:155-161). A failed flush is reported as a warning and the next period
        tries again."""
        if self._thread is not None:
            return self._thread

        def run():
            torch.cuda.set_device(self.dev)
            while not self._stop.wait(every_s):
                try:
                    self.flush(out_dir)
                except Exception as exc:                            # noqa: BLE001
                    warnings.warn(f"routecap flush to {out_dir or OUT_DIR!r} failed: {exc!r}")

        self._stop.clear()
        self._thread = threading.Thread(target=run, daemon=True, name="routecap-dumper")
        self._thread.start()
        return self._thread

    def stop_dumper(self, flush: bool = True, out_dir: str | None = None) -> None:
        """Stop the dumper thread (if any) and, by default, write one last flush."""
        if self._thread is not None:
            self._stop.set()
            self._thread.join()
            self._thread = None
        if flush:
            self.flush(out_dir)

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
