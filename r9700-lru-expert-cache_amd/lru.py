"""Host side of the device LRU expert cache: the op wrappers of the reference, on librlu.so.

Mirrors patches/model_executor/layers/fused_moe/experts/r4d_mxfp4_moe.py.lru.diff:
  _r4d_lru_manage  :208-249     _r4d_lru_gather :252-287     _align_sizes :290-296
  _r4d_lru_fused   :299-354     _build_lru      :502-541     _lru_step(_fused) :543-579
Same argument meaning, same RuntimeError on a nonzero return code. The ops are also
registered as torch custom ops with the reference's names and mutates_args, in the "vllm"
namespace when vLLM is importable and in "rlu" otherwise.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import torch

from ._lib import check, lib, stream_ptr

_P = ctypes.c_void_p

# the reference's knobs and defaults (r4d_mxfp4_moe.py.lru.diff:144-151), except the gather
# geometry: the reference's 8 chunks x 16 lanes keeps ~2 MB of host reads in flight on
# MI355X, which the link does not need (it saturates at ~58 GB/s with far less) and which
# slows every kernel running beside the gather several-fold. 4 x 32 was the fastest
# measured for a 52-layer decode step with the gather overlapped (20 rows, ~9 misses/layer).
LRU_THRESH = float(os.environ.get("VLLM_R4D_LRU_THRESH", "0.5"))
LRU_MAX_INSERTS = int(os.environ.get("VLLM_R4D_LRU_MAX_INSERTS", "64"))
LRU_CHUNKS = int(os.environ.get("VLLM_R4D_LRU_CHUNKS", "4"))
LRU_LANES = int(os.environ.get("VLLM_R4D_LRU_LANES", "32"))
BLOCK = 16


def _ptr(t: torch.Tensor) -> _P:
    return _P(t.data_ptr())


def _align_sizes(mk: int, num_experts: int, block_size: int) -> tuple[int, int]:
    """The lengths vLLM's moe_align_block_size wrapper allocates for `mk` (token, k) slots."""
    n = mk + num_experts * (block_size - 1)
    if mk < num_experts:
        n = min(mk * block_size, n)
    return n, (n + block_size - 1) // block_size


def _check_state(topk_ids, table, slot_expert, slot_stamp, routed, step, miss, n_miss):
    # the C boundary has no type safety (the reference leaves these unasserted)
    assert topk_ids.dtype == torch.int32 and topk_ids.is_contiguous()
    assert table.dtype == torch.int32 and slot_expert.dtype == torch.int32
    assert slot_stamp.dtype == torch.int64 and step.dtype == torch.int64
    assert routed.dtype == torch.uint8 and routed.numel() == table.numel()
    assert miss.dtype == torch.int32 and miss.is_contiguous() and miss.dim() == 2 \
        and miss.shape[1] == 2
    assert n_miss.dtype == torch.int32


def _r4d_lru_manage(topk_ids: torch.Tensor, table: torch.Tensor, map_cold: torch.Tensor,
                    slot_expert: torch.Tensor, slot_stamp: torch.Tensor, routed: torch.Tensor,
                    step: torch.Tensor, miss: torch.Tensor, n_miss: torch.Tensor,
                    max_distinct: int, max_inserts: int) -> None:
    """One workgroup: refresh stamps of the routed resident experts, evict the least recently
    routed slots this step does not need, rewrite table/map_cold and emit the (expert, slot)
    miss list. Deterministic."""
    _check_state(topk_ids, table, slot_expert, slot_stamp, routed, step, miss, n_miss)
    assert max_inserts <= miss.shape[0]
    rc = lib().r4d_lru_manage(
        _ptr(topk_ids), topk_ids.numel(), table.numel(), slot_expert.numel(), max_distinct,
        max_inserts, _ptr(table), _ptr(map_cold), _ptr(slot_expert), _ptr(slot_stamp),
        _ptr(routed), _ptr(step), _ptr(miss), _ptr(n_miss), _P(stream_ptr()))
    check(rc, "r4d_lru_manage")


def _per_expert_bytes(t: torch.Tensor) -> int:
    return t[0].numel() * t.element_size()


def _r4d_lru_gather(dsts: list[torch.Tensor], srcs: list[torch.Tensor], miss: torch.Tensor,
                    n_miss: torch.Tensor, chunks: int, lanes: int,
                    src_ptrs: list[int] | None = None) -> None:
    """Copy the six per-expert buffers of each missing expert into its new slot. `srcs` may
    live in pinned host memory; `src_ptrs` then carries their device-visible addresses."""
    if len(dsts) != 6 or len(srcs) != 6:
        raise ValueError("lru gather takes exactly six (dst, src) buffer pairs")
    args = []
    for i, (d, s) in enumerate(zip(dsts, srcs)):
        nb = _per_expert_bytes(s)
        if nb != _per_expert_bytes(d):
            raise ValueError(f"lru gather: slab size mismatch {nb} vs {_per_expert_bytes(d)}")
        sp = s.data_ptr() if src_ptrs is None else src_ptrs[i]
        args += [_ptr(d), _P(sp), ctypes.c_long(nb)]
    rc = lib().r4d_lru_gather(*args, _ptr(miss), _ptr(n_miss), chunks, lanes,
                              _P(stream_ptr()))
    check(rc, "r4d_lru_gather (slab sizes must be 16B multiples)")


def split_fresh(eids_hot: torch.Tensor, miss: torch.Tensor, n_miss: torch.Tensor, S: int,
                eids_res: torch.Tensor, eids_new: torch.Tensor) -> None:
    """The bucket split of the three-way gather overlap (docs/REVIEW.md:281-301): eids_res
    <- the blocks of eids_hot whose slot was resident before this step's manager ran,
    eids_new <- the blocks whose slot it installed (the slot column of miss[:n_miss]); -1 in
    the other. Each is a valid expert-id array for the grouped GEMM's row contract."""
    for t in (eids_hot, miss, n_miss, eids_res, eids_new):
        assert t.dtype == torch.int32 and t.is_contiguous()
    nb = eids_hot.numel()
    assert eids_res.numel() == nb and eids_new.numel() == nb and miss.shape[-1] == 2
    rc = lib().rlu_lru_split_fresh(_ptr(eids_hot), nb, _ptr(miss), _ptr(n_miss),
                                   miss.numel() // 2, S, _ptr(eids_res), _ptr(eids_new),
                                   _P(stream_ptr()))
    check(rc, "rlu_lru_split_fresh")


def _r4d_lru_fused(topk_ids: torch.Tensor, table: torch.Tensor, map_cold: torch.Tensor,
                   slot_expert: torch.Tensor, slot_stamp: torch.Tensor, routed: torch.Tensor,
                   step: torch.Tensor, miss: torch.Tensor, n_miss: torch.Tensor,
                   sorted_hot: torch.Tensor, eids_hot: torch.Tensor, npad_hot: torch.Tensor,
                   sorted_cold: torch.Tensor, eids_cold: torch.Tensor,
                   npad_cold: torch.Tensor, max_distinct: int, max_inserts: int,
                   block_size: int) -> None:
    """The manager plus both moe_align_block_size outputs (resident side bucketed by slot,
    fallback side by expert id) from the table it just rewrote. Every element of the six
    outputs is written on every call, read-through and zero-miss steps included."""
    _check_state(topk_ids, table, slot_expert, slot_stamp, routed, step, miss, n_miss)
    assert max_inserts <= miss.shape[0]
    rc = lib().r4d_lru_fused(
        _ptr(topk_ids), topk_ids.numel(), table.numel(), slot_expert.numel(), max_distinct,
        max_inserts, _ptr(table), _ptr(map_cold), _ptr(slot_expert), _ptr(slot_stamp),
        _ptr(routed), _ptr(step), _ptr(miss), _ptr(n_miss), block_size, sorted_hot.numel(),
        eids_hot.numel(), _ptr(sorted_hot), _ptr(eids_hot), _ptr(npad_hot), _ptr(sorted_cold),
        _ptr(eids_cold), _ptr(npad_cold), _P(stream_ptr()))
    check(rc, "r4d_lru_fused (E and slots must be <= 1024)")


def _rlu_lru_fused_quant(topk_ids: torch.Tensor, state: list[torch.Tensor],
                        out: list[torch.Tensor], max_distinct: int, max_inserts: int,
                        block_size: int, x: torch.Tensor, q: torch.Tensor,
                        scale: torch.Tensor) -> None:
    """_r4d_lru_fused and, in the same launch, the per-token-group-128 e4m3 quant of x
    [rows, K] bf16 into q [rows, K] / scale [rows, K/128] (no reference counterpart: the
    reference launched the activation quant separately)."""
    table, map_cold, slot_expert, slot_stamp, routed, step, miss, n_miss = state
    _check_state(topk_ids, table, slot_expert, slot_stamp, routed, step, miss, n_miss)
    assert max_inserts <= miss.shape[0]
    assert x.dtype == torch.bfloat16 and x.stride(1) == 1 and q.is_contiguous()
    rows, K = x.shape
    rc = lib().rlu_lru_fused_quant(
        _ptr(topk_ids), topk_ids.numel(), table.numel(), slot_expert.numel(), max_distinct,
        max_inserts, _ptr(table), _ptr(map_cold), _ptr(slot_expert), _ptr(slot_stamp),
        _ptr(routed), _ptr(step), _ptr(miss), _ptr(n_miss), block_size, out[0].numel(),
        out[1].numel(), *[_ptr(o) for o in out], _ptr(x), rows, K, x.stride(0), _ptr(q),
        _ptr(scale), _P(stream_ptr()))
    check(rc, "rlu_lru_fused_quant")


# ---- torch custom op registration (names and mutates_args of the reference) ---------------
def _register():
    try:  # pragma: no cover - vLLM is not part of this image
        from vllm.utils.torch_utils import direct_register_custom_op  # noqa: F401
        ns = "vllm"
    except Exception:  # noqa: BLE001
        ns = "rlu"
    lib_ = torch.library.Library(ns, "FRAGMENT")
    lib_.define("r4d_lru_manage(Tensor topk_ids, Tensor(a!) table, Tensor(b!) map_cold, "
                "Tensor(c!) slot_expert, Tensor(d!) slot_stamp, Tensor(e!) routed, "
                "Tensor(f!) step, Tensor(g!) miss, Tensor(h!) n_miss, int max_distinct, "
                "int max_inserts) -> ()")
    lib_.define("r4d_lru_gather(Tensor(a!)[] dsts, Tensor[] srcs, Tensor miss, Tensor n_miss, "
                "int chunks, int lanes) -> ()")
    lib_.define("r4d_lru_fused(Tensor topk_ids, Tensor(a!) table, Tensor(b!) map_cold, "
                "Tensor(c!) slot_expert, Tensor(d!) slot_stamp, Tensor(e!) routed, "
                "Tensor(f!) step, Tensor(g!) miss, Tensor(h!) n_miss, Tensor(i!) sorted_hot, "
                "Tensor(j!) eids_hot, Tensor(k!) npad_hot, Tensor(l!) sorted_cold, "
                "Tensor(m!) eids_cold, Tensor(n!) npad_cold, int max_distinct, "
                "int max_inserts, int block_size) -> ()")
    lib_.impl("r4d_lru_manage", _r4d_lru_manage, "CUDA")
    lib_.impl("r4d_lru_gather",
              lambda d, s, m, n, c, l: _r4d_lru_gather(list(d), list(s), m, n, c, l), "CUDA")
    lib_.impl("r4d_lru_fused", _r4d_lru_fused, "CUDA")
    for name in ("r4d_lru_manage", "r4d_lru_gather", "r4d_lru_fused"):
        lib_.impl(name, lambda *a, **k: None, "Meta")
    return ns, lib_


OPS_NAMESPACE, _OPS_LIB = _register()


# ---- per-layer cache state: _build_lru / _lru_step / _lru_step_fused ------------------------
@dataclass
class LruCache:
    """The per-layer tensors of `_build_lru` (r4d_mxfp4_moe.py.lru.diff:524-534). Allocated
    once and never reallocated, so HIP-graph pointers stay valid."""
    table: torch.Tensor
    map_cold: torch.Tensor
    slot_expert: torch.Tensor
    slot_stamp: torch.Tensor
    routed: torch.Tensor
    step: torch.Tensor
    miss: torch.Tensor
    n_miss: torch.Tensor
    max_distinct: int
    max_inserts: int

    @property
    def E(self) -> int:
        return self.table.numel()

    @property
    def S(self) -> int:
        return self.slot_expert.numel()

    @classmethod
    def build(cls, E: int, hot_ids, rank: dict | None, device, thresh: float = LRU_THRESH,
              max_inserts: int = LRU_MAX_INSERTS) -> "LruCache":
        """Warm start (r4d_mxfp4_moe.py.lru.diff:502-541): slot i holds the i-th smallest hot
        id; stamps in profile-rank order, hottest = S, coldest = 1 (zeros without a profile);
        step = S; read-through above max(1, int(S * thresh)) distinct experts per step."""
        hot = sorted(int(e) for e in hot_ids)
        S = len(hot)
        if not (0 < S <= 1024 and 0 < E <= 1024):
            raise ValueError(f"LRU cache needs 1 <= S, E <= 1024 (got S={S}, E={E})")
        dev = torch.device(device)
        hot_t = torch.tensor(hot, dtype=torch.int64)
        table = torch.full((E,), -1, dtype=torch.int32)
        table[hot_t] = torch.arange(S, dtype=torch.int32)
        map_cold = torch.arange(E, dtype=torch.int32)
        map_cold[hot_t] = -1
        if rank is None:
            stamp = torch.zeros(S, dtype=torch.int64)
        else:
            r = torch.tensor([rank.get(e, len(rank)) for e in hot], dtype=torch.int64)
            stamp = S - torch.argsort(torch.argsort(r, stable=True), stable=True)
        assert int(stamp.min()) >= 0, "stamps must be non-negative"
        cap = min(max_inserts, S)
        return cls(table=table.to(dev), map_cold=map_cold.to(dev),
                   slot_expert=hot_t.to(torch.int32).to(dev), slot_stamp=stamp.to(dev),
                   routed=torch.zeros(E, dtype=torch.uint8, device=dev),
                   step=torch.full((1,), S, dtype=torch.int64, device=dev),
                   miss=torch.full((cap, 2), -1, dtype=torch.int32, device=dev),
                   n_miss=torch.zeros(1, dtype=torch.int32, device=dev),
                   max_distinct=max(1, int(S * thresh)), max_inserts=cap)

    def state(self) -> list[torch.Tensor]:
        return [self.table, self.map_cold, self.slot_expert, self.slot_stamp, self.routed,
                self.step, self.miss, self.n_miss]

    def manage(self, topk_ids: torch.Tensor) -> None:
        _r4d_lru_manage(topk_ids.reshape(-1).to(torch.int32), *self.state(),
                        self.max_distinct, self.max_inserts)

    def alloc_align(self, mk: int, block_size: int = BLOCK) -> list[torch.Tensor]:
        n, nb = _align_sizes(mk, self.E, block_size)
        dev = self.table.device
        return [torch.empty(n, dtype=torch.int32, device=dev),
                torch.empty(nb, dtype=torch.int32, device=dev),
                torch.empty(1, dtype=torch.int32, device=dev),
                torch.empty(n, dtype=torch.int32, device=dev),
                torch.empty(nb, dtype=torch.int32, device=dev),
                torch.empty(1, dtype=torch.int32, device=dev)]

    def fused(self, topk_ids: torch.Tensor, out: list[torch.Tensor] | None = None,
              block_size: int = BLOCK):
        """-> ((sorted_hot, eids_hot, npad_hot), (sorted_cold, eids_cold, npad_cold))."""
        ids = topk_ids.reshape(-1).to(torch.int32)
        if out is None:
            out = self.alloc_align(ids.numel(), block_size)
        _r4d_lru_fused(ids, *self.state(), *out, self.max_distinct, self.max_inserts,
                       block_size)
        return tuple(out[0:3]), tuple(out[3:6])

    def fused_quant(self, topk_ids: torch.Tensor, out: list[torch.Tensor], x: torch.Tensor,
                    q: torch.Tensor, scale: torch.Tensor, block_size: int = BLOCK):
        """fused() plus the group-128 quant of x into (q, scale), one launch."""
        ids = topk_ids.reshape(-1).to(torch.int32)
        _rlu_lru_fused_quant(ids, self.state(), out, self.max_distinct, self.max_inserts,
                             block_size, x, q, scale)
        return tuple(out[0:3]), tuple(out[3:6])
