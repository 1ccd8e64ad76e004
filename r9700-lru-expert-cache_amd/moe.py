"""One MoE layer of the decode hot path: device LRU cache, align, miss gather and the fp8 expert
GEMMs, all on librlu.so.

Mirrors R4dMxfp4MoEExperts' split path (patches/model_executor/layers/fused_moe/experts/
r4d_mxfp4_moe.py.lru.diff): _build_hot / _build_lru (:453-541) -> LruMoELayer.__init__,
_lru_step_fused (:557-579) -> _lru_step_fused, _gemm_split (:584-607) -> _gemm_split,
_act_quant (:640-657) -> _act_quant, _apply_split (:659-696) -> apply. The experts are fp8 e4m3
with 128x128 float32 block scales (w13 [E, 2I, H], w2 [E, H, I]); the activation quant is
per-token-group-128. The miss gather runs on a side stream; the GEMMs over rows it does not
write run beside it, the others wait for it (apply's overlap).

Every buffer a step touches is allocated here, once, for a fixed token count, so a step can be
captured into a HIP graph and replayed with new routing (only contents change).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import ops
from ._lib import check, device_ptr_of_pinned, lib, stream_ptr  # noqa: F401
from .lru import LRU_CHUNKS, LRU_LANES, LruCache, _r4d_lru_gather, split_fresh

_P = ctypes.c_void_p
BLOCK = 16
# Routed rows per expert (tokens x top_k / E) from which a layer runs the prefill grouped GEMMs
# instead of the decode one. Measured crossover of the whole layer step at E = 512, top-10,
# every expert resident, graph-replayed (us, decode / prefill kernels):
#   tokens (rows per expert)   Zipf(1.1) routing   uniform routing
#   256 (5.0)                  429 / 464           508 / 530
#   320 (6.25)                 500 / 482           527 / 514
#   512 (10)                   613 / 546           548 / 553
#   1024 (20)                  852 / 648           856 / 582
# The decode kernel reads an expert's weights once per 16-row block, the prefill kernels once
# per tile of up to 128 rows, behind a fixed cost of their own (tile list, persistent grid).
PREFILL_ROWS_PER_EXPERT = 6
# Tokens up to which a decode step folds moe_sum into the down projection (ops.moe_down_sum):
# the token-major kernel reads each expert strip once per token routed to it, which pays at
# B=1 (5 tokens: 16.3 vs 18.9 us per layer for down + moe_sum) and loses at B=4 (20 tokens:
# 41.0 vs 22.9 us).
FOLD_SUM_TOKENS = 8


@dataclass
class ExpertWeights:
    """fp8 experts with block scales; the four per-expert buffers of the fp8 format. The e4m3
    tensors are in fragment order (ops.shuffle_fp8_weight), as loaded once at start-up."""
    w13: torch.Tensor     # e4m3 [E, 2I, H], fragment order
    s13: torch.Tensor     # f32  [E, 2I/128, H/128]
    w2: torch.Tensor      # e4m3 [E, H, I], fragment order
    s2: torch.Tensor      # f32  [E, H/128, I/128]

    def tensors(self):
        return [self.w13, self.s13, self.w2, self.s2]

    def per_expert_bytes(self) -> int:
        """Bytes one expert occupies in the four buffers (what one slot costs in HBM)."""
        return sum(t[0].numel() * t.element_size() for t in self.tensors())

    def ptrs(self) -> list[int]:
        """Device-visible addresses (pinned host tensors are translated)."""
        return [device_ptr_of_pinned(t) if t.is_pinned() else t.data_ptr()
                for t in self.tensors()]


class LruMoELayer:
    def __init__(self, full: ExpertWeights, hot_ids, rank: dict | None, max_tokens: int,
                 top_k: int, device="cuda", slots: ExpertWeights | None = None,
                 npw1: int = 2, npw2: int = 4, sk1: int | None = None, sk2: int = 1,
                 wv: int = 0, max_inserts: int | None = None,
                 prefill_rows: int | None = None, fold_sum: bool | None = None,
                 fuse_act: bool | None = None):
        """npw / sk: 16-column tiles per item and K split of gate_up (1) and down (2); the
        defaults are the fastest measured at the decode shapes (hidden 2560, intermediate
        768): gate_up splits K over 2 waves above 8 tokens (20 tokens: 3.70 vs 3.95 ms per
        52-layer step) and not at all up to 8 (5 tokens: 3.007 vs 3.038 ms).

        max_inserts: cap on cache inserts per step (default VLLM_R4D_LRU_MAX_INSERTS, 64); 0 is
        the static hot/cold arm -- the warm-start set stays resident and every other routed
        expert is read from the full tensor (r4d_mxfp4_moe.py.static.diff, and the README's
        MAX_INSERTS=0 ablation).

        prefill_rows: from this many routed rows (max_tokens x top_k) on, both GEMMs run the
        tiled prefill kernel (ops.moe_gemm_tiled: whole expert tiles, the weights streamed
        once per tile) over the hot and the cold align, in place of the decode kernel; npw /
        sk / wv do not apply to it. Default PREFILL_ROWS_PER_EXPERT x E (3072 rows, about
        307 tokens at top-10, over 512 experts). Its output equals the decode kernel's with sk = 1 bit
        for bit. The reference runs prefill chunks through the same split path
        (r4d_mxfp4_moe.py.lru.diff:659-696; tests/lru/test_numerics_prod.py:44-48).

        fold_sum: run down and moe_sum as one token-major kernel (ops.moe_down_sum, or
        ops.moe_down_sum_act from the activation with fuse_act; the same output bit for bit)
        when the gather is not overlapped; default on up to
        FOLD_SUM_TOKENS tokens at the shapes the kernel is built for (intermediate 768,
        top-10).

        fuse_act (decode): gate_up writes the SiLU-mul activation from its epilogue
        (ops.moe_gemm_split_act) and down quantizes it per workgroup
        (ops.moe_gemm_split_qin, or ops.moe_down_sum_act where down and moe_sum are folded),
        in place of gate_up into ic1, silu_mul_quant and down on q2 / s2: the same output bit
        for bit, one launch fewer per layer (two with the gather overlap). Default on for
        decode layers at npw 2 / 4, sk2 = 1, wv = 0, 2 I % 256 == 0, hidden % 256 == 0 and
        I <= 768; prefill layers fuse the activation into their own gate_up."""
        dev = torch.device(device)
        self.full = full
        self.full_ptrs = full.ptrs()
        self.E = full.w13.shape[0]
        self.N1, self.H = full.w13.shape[1], full.w13.shape[2]
        self.I = self.N1 // 2
        self.top_k = top_k
        self.M = max_tokens
        self.mtk = max_tokens * top_k
        if sk1 is None:
            sk1 = 1 if max_tokens <= 8 else 2
        self.npw1, self.npw2, self.sk1, self.sk2, self.wv = npw1, npw2, sk1, sk2, wv
        for t in full.tensors():
            slab = t[0].numel() * t.element_size()
            if slab % 16:
                raise ValueError(f"per-expert slab of {tuple(t.shape)} is {slab} B: the miss "
                                 "gather copies 16-byte units (r4d_lru.hip:271-301)")
        hot = sorted(int(e) for e in hot_ids)
        if slots is None:
            idx = torch.tensor(hot, dtype=torch.int64)
            slots = ExpertWeights(*[t.index_select(0, idx.to(t.device)).to(dev).contiguous()
                                    for t in full.tensors()])
        self.slots = slots
        self.cache = (LruCache.build(self.E, hot, rank, dev) if max_inserts is None else
                      LruCache.build(self.E, hot, rank, dev, max_inserts=max_inserts))
        # align outputs and intermediates for exactly max_tokens rows
        self.align = self.cache.alloc_align(self.mtk, BLOCK)
        self.eids_res = torch.empty_like(self.align[1])
        self.eids_new = torch.empty_like(self.align[1])
        self.ev_up = torch.cuda.Event()
        # optional routing capture (routecap.RouteRing.fn(layer)), called with each step's
        # topk_ids before the cache runs, as the router's capture_fn is
        self.route_capture = None
        self.qx = torch.empty((self.M, self.H), dtype=ops.FP8, device=dev)
        self.xs = torch.empty((self.M, self.H // 128), dtype=torch.float32, device=dev)
        if prefill_rows is None:
            prefill_rows = PREFILL_ROWS_PER_EXPERT * self.E
        self.prefill = self.mtk >= prefill_rows
        if fold_sum is None:
            # not for the static arm: its cold experts are the common case, and the folded
            # kernel reads an expert's strip once per token routed to it -- over the host
            # link for a cold one
            fold_sum = (not self.prefill and max_tokens <= FOLD_SUM_TOKENS and self.I == 768
                        and top_k == 10 and self.cache.max_inserts > 0)
        self.fold_sum = fold_sum
        self.ids32 = torch.empty((self.M, top_k), dtype=torch.int32, device=dev)
        # prefill gate_up with SiLU-mul-quant in its epilogue where a kernel is built for the
        # shape: no [mtk, 2I] bf16 intermediate (same q2 / s2 bits)
        self.fuse_act = self.prefill and ops.moe_gemm_tiled_silu_quant_built(self.H, self.N1)
        # decode: gate_up with its activation, down quantizing it (no activation launch)
        if fuse_act is None:
            fuse_act = (not self.prefill and npw1 == 2 and npw2 == 4 and sk2 == 1 and wv == 0
                        and self.N1 % 256 == 0 and self.H % 256 == 0 and self.I <= 768)
        self.fuse_dec = bool(fuse_act) and not self.prefill
        self.act = (torch.empty((self.mtk, self.I), dtype=torch.bfloat16, device=dev)
                    if self.fuse_dec else None)
        self.ic1 = (None if self.fuse_act or self.fuse_dec else
                    torch.empty((self.mtk, self.N1), dtype=torch.bfloat16, device=dev))
        self.q2 = torch.empty((self.mtk, self.I), dtype=ops.FP8, device=dev)
        self.s2 = torch.empty((self.mtk, self.I // 128), dtype=torch.float32, device=dev)
        self.ic3 = torch.empty((self.mtk, self.H), dtype=torch.bfloat16, device=dev)
        self.tw = torch.empty((self.mtk,), dtype=torch.float32, device=dev)
        if self.prefill:
            # one tile list per block-expert-id array the tiled GEMMs read (the hot align's,
            # the cold align's, the overlap's two buckets), built by the first GEMM of a step
            # that reads it and reused by the rest of that step
            self.tiles = {t.data_ptr(): torch.empty(2 * t.numel() + 1, dtype=torch.int32,
                                                    device=dev)
                          for t in (self.align[1], self.align[4], self.eids_res, self.eids_new)}
            # where the streamed kernel is built for both GEMMs, a GEMM over the hot align (or
            # the overlap's resident bucket) and the cold align is one launch over one tile
            # list of both (an empty cold align then costs no launch of its own)
            self.pf_split = (ops.moe_gemm_tiled_split_built(self.H, self.N1) and
                             ops.moe_gemm_tiled_split_built(self.I, self.H))
            ec = self.align[4]
            self.split_tiles = {
                (t.data_ptr(), ec.data_ptr()): torch.empty(2 * (t.numel() + ec.numel()) + 1,
                                                           dtype=torch.int32, device=dev)
                for t in (self.align[1], self.eids_res)} if self.pf_split else {}
            self.tiles_built = set()

    @classmethod
    def from_profile(cls, full: ExpertWeights, profile, layer: int, budget_gb: float,
                     max_tokens: int, top_k: int, device="cuda", **kw) -> "LruMoELayer":
        """The layer's warm start from a hot profile (hot_profile.HotProfile): its share of the
        global budget_gb water-fill as the slots (r4d_mxfp4_moe.py.lru.diff:502-541 with
        hot_ids_for_layer / profile_rank_for_layer), stamps by profile rank. Raises
        ValueError when the layer is not profiled or gets no slot."""
        from . import hot_profile as hp
        sets = hp.hot_sets(profile, full.per_expert_bytes(), budget_gb)
        if layer not in sets:
            raise ValueError(f"layer {layer} is not in the hot profile")
        if not sets[layer]:
            raise ValueError(f"the {budget_gb} GB budget leaves layer {layer} no slot")
        return cls(full, sets[layer], profile.rank(layer), max_tokens, top_k, device, **kw)

    # -- _lru_step_fused: manager + both aligns in one launch, then the miss gather -----------
    def _lru_step_fused(self, topk_ids: torch.Tensor, gather: bool, side: torch.cuda.Stream | None,
                        hidden_states: torch.Tensor | None = None, split: bool = False):
        """The fused manager + align; with hidden_states, the same launch also quantizes them
        into (qx, xs) (the cache and the quant are independent and both feed GEMM1).

        split (with a side stream): the gather runs as two launches, the gate_up buffers
        (w13, s13) first and then the down buffers (w2, s2), with self.ev_up recorded between
        them, so that gate_up over the installed slots can start while w2 is still arriving."""
        if hidden_states is None:
            self.cache.fused(topk_ids, out=self.align, block_size=BLOCK)
        else:
            self.cache.fused_quant(topk_ids, self.align, hidden_states, self.qx, self.xs,
                                   block_size=BLOCK)
        if not gather:
            return None
        w13, s13, w2, s2 = ((self.slots.w13, self.full.w13, self.full_ptrs[0]),
                            (self.slots.s13, self.full.s13, self.full_ptrs[1]),
                            (self.slots.w2, self.full.w2, self.full_ptrs[2]),
                            (self.slots.s2, self.full.s2, self.full_ptrs[3]))
        # six-buffer ABI of the reference gather: the fp8 format has four per-expert buffers;
        # spare pairs repeat a (small) scale buffer -- the same bytes to the same place
        if split and side is not None:
            parts = [[w13, s13, s13, s13, s13, s13], [w2, s2, s2, s2, s2, s2]]
        else:
            parts = [[w13, w2, s13, s2, s13, s2]]
        cur = torch.cuda.current_stream()
        if side is None:
            for p in parts:
                self._gather(p)
            return None
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            for i, p in enumerate(parts):
                self._gather(p)
                if i + 1 < len(parts):
                    self.ev_up.record(side)
        return side

    def _gather(self, pairs):
        _r4d_lru_gather([d for d, _, _ in pairs], [s for _, s, _ in pairs], self.cache.miss,
                        self.cache.n_miss, LRU_CHUNKS, LRU_LANES,
                        src_ptrs=[p for _, _, p in pairs])

    # -- _gemm_split: resident slots + the full tensor, one launch ----------------------------
    def _down(self, tw, eh=None, cold=True):
        """The down projection into ic3 over the hot align (block ids eh) and, with cold, the
        cold align."""
        if self.fuse_dec:
            sh, eh0, nh, sc, ec, nc = self.align
            ops.moe_gemm_split_qin(
                self.ic3, self.act, self.slots.w2, self.slots.s2,
                (sh, eh0 if eh is None else eh, nh), tw, self.mtk,
                *((self.full.w2, self.full.s2, (sc, ec, nc)) if cold else ()))
            return
        down = (self.ic3, self.q2, self.s2, self.slots.w2, self.slots.s2)
        if cold:
            self._gemm_split(*down, 2, tw, 1, self.npw2, self.sk2, eh=eh)
        else:
            self._gemm_hot(*down, tw, 1, self.npw2, self.sk2, eh)

    def _gemm_split(self, y, qx, xs, slot_w, slot_s, part, tw, top_k, npw, sk, eh=None):
        """part: 0 gate_up, 2 down (the index of its weight buffer in ExpertWeights.tensors);
        eh replaces the hot align's block expert ids (the overlap's resident bucket)."""
        sh, eh0, nh, sc, ec, nc = self.align
        eh = eh0 if eh is None else eh
        if self.prefill:
            full = self.full.tensors()
            if self.pf_split:
                ops.moe_gemm_tiled_split(y, qx, xs, slot_w, slot_s, (sh, eh, nh), full[part],
                                         full[part + 1], (sc, ec, nc), tw, y.shape[0], top_k,
                                         tiles=self._split_tiles_of(eh, nh), tiles_ready=True)
                return
            self._gemm_tiled(y, qx, xs, slot_w, slot_s, sh, eh, nh, tw, top_k)
            self._gemm_tiled(y, qx, xs, full[part], full[part + 1], sc, ec, nc, tw, top_k)
            return
        full_w_ptr, full_s_ptr = self.full_ptrs[part], self.full_ptrs[part + 1]
        K = qx.shape[1]
        N = slot_w.shape[1]
        rc = lib().rlu_moe_gemm_split(
            _P(qx.data_ptr()), _P(xs.data_ptr()), _P(slot_w.data_ptr()), _P(slot_s.data_ptr()),
            _P(sh.data_ptr()), _P(eh.data_ptr()), _P(nh.data_ptr()), _P(full_w_ptr),
            _P(full_s_ptr), _P(sc.data_ptr()), _P(ec.data_ptr()), _P(nc.data_ptr()),
            _P(0 if tw is None else tw.data_ptr()), _P(y.data_ptr()), sh.numel(),
            y.shape[0], top_k, K, N, self.wv, sk, npw, _P(stream_ptr()))
        check(rc, "rlu_moe_gemm_split")

    # -- the hot GEMM alone over a bucket of slots (the overlap's installed bucket) -----------
    def _gemm_hot(self, y, qx, xs, slot_w, slot_s, tw, top_k, npw, sk, eh):
        sh, _, nh = self.align[:3]
        if self.prefill:
            self._gemm_tiled(y, qx, xs, slot_w, slot_s, sh, eh, nh, tw, top_k)
            return
        ops._r4d_fp8_moe_gemm_into(y, qx, xs, slot_w, slot_s, None, sh, eh, nh, tw, y.shape[0],
                                   top_k, self.wv, sk, npw)

    # -- the tiled (prefill) GEMM over one align ----------------------------------------------
    def _tiles_of(self, eids, npad):
        """The tile list of block expert ids eids, built on its first use in a step."""
        key = eids.data_ptr()
        ready = key in self.tiles_built
        if not ready:
            ops.moe_gemm_tiles(eids, npad, self.tiles[key])
            self.tiles_built.add(key)
        return self.tiles[key]

    def _split_tiles_of(self, eh, nh):
        """The tile list of hot block expert ids eh and the cold align, built on its first use
        in a step."""
        ec, nc = self.align[4], self.align[5]
        key = (eh.data_ptr(), ec.data_ptr())
        if key not in self.tiles_built:
            ops.moe_gemm_tiles_split((eh, nh), (ec, nc), self.split_tiles[key])
            self.tiles_built.add(key)
        return self.split_tiles[key]

    def _gemm_tiled(self, y, qx, xs, w, s, sorted_ids, eids, npad, tw, top_k):
        ops.moe_gemm_tiled(y, qx, xs, w, s, sorted_ids, eids, npad, tw, y.shape[0], top_k,
                           tiles=self._tiles_of(eids, npad), tiles_ready=True)

    # -- _act_quant: fused silu-and-mul + group-128 quant --------------------------------------
    def _act_quant(self):
        ops.silu_mul_quant(self.ic1, group=ops.GROUP, out=(self.q2, self.s2))

    # -- gate_up and the activation quant over the hot align (block ids eh) and, with cold,
    # the cold align -------------------------------------------------------------------------
    def _gate_up_act(self, eh=None, cold=True):
        if self.fuse_dec:
            sh, eh0, nh, sc, ec, nc = self.align
            ops.moe_gemm_split_act(
                self.act, self.qx, self.xs, self.slots.w13, self.slots.s13,
                (sh, eh0 if eh is None else eh, nh), self.mtk, self.top_k,
                *((self.full.w13, self.full.s13, (sc, ec, nc)) if cold else ()), wv=self.wv,
                sk=self.sk1)
            return
        if self.fuse_act:
            sh, eh0, nh, sc, ec, nc = self.align
            eh = eh0 if eh is None else eh
            if cold and self.pf_split:
                ops.moe_gemm_tiled_split_silu_quant(
                    self.q2, self.s2, self.qx, self.xs, self.slots.w13, self.slots.s13,
                    (sh, eh, nh), self.full.w13, self.full.s13, (sc, ec, nc), self.mtk,
                    self.top_k, tiles=self._split_tiles_of(eh, nh), tiles_ready=True)
                return
            for w, s, al in (((self.slots.w13, self.slots.s13, (sh, eh, nh)),) +
                             (((self.full.w13, self.full.s13, (sc, ec, nc)),) if cold else ())):
                ops.moe_gemm_tiled_silu_quant(self.q2, self.s2, self.qx, self.xs, w, s, *al,
                                              self.mtk, self.top_k,
                                              tiles=self._tiles_of(al[1], al[2]),
                                              tiles_ready=True)
            return
        up = (self.ic1, self.qx, self.xs, self.slots.w13, self.slots.s13)
        if cold:
            self._gemm_split(*up, 0, None, self.top_k, self.npw1, self.sk1, eh=eh)
        else:
            self._gemm_hot(*up, None, self.top_k, self.npw1, self.sk1, eh)
        self._act_quant()

    def apply(self, output: torch.Tensor, hidden_states: torch.Tensor, topk_weights: torch.Tensor,
              topk_ids: torch.Tensor, gather: bool = True,
              side: torch.cuda.Stream | None = None, overlap: bool | None = None) -> None:
        """_apply_split: output [M, H] bf16 <- hidden_states [M, H] bf16 routed by topk_ids /
        topk_weights [M, top_k].

        overlap (needs gather and a side stream; default on when the cache can insert): the
        three-way split of docs/REVIEW.md:281-301. While the side stream gathers this step's
        installs, the main stream runs gate_up, SiLU-quant and down over the rows of slots
        resident before the manager ran plus the cold rows. Then gate_up and SiLU-quant over
        the rows of the installed slots, once their w13 has arrived (the gather copies w13
        and s13 first, w2 and s2 second), down over them once all of it has, and moe_sum.
        Every row is computed by the same kernel with the same split as without the overlap,
        so the output is bit-identical. The price at decode is one more SiLU-mul-quant launch
        per layer (a second pass for the installed slots' rows; at 200 rows the launch, not
        the rows, is its cost, so a row-list variant would cost the same); the 52-layer B=4
        step with the gather still runs faster overlapped (54.7 vs 56.2 ms). Prefill layers
        fuse the activation into gate_up and pay nothing extra."""
        M = hidden_states.shape[0]
        assert M == self.M and topk_ids.shape == (M, self.top_k)
        if self.route_capture is not None:
            self.route_capture(topk_ids)
        if overlap is None:
            overlap = self.cache.max_inserts > 0
        overlap = overlap and gather and side is not None
        waited = self._lru_step_fused(topk_ids, gather, side, hidden_states, split=overlap)
        if self.prefill:
            self.tiles_built.clear()                  # this step's aligns: lists rebuilt
        tw = topk_weights.reshape(-1)
        if tw.dtype != torch.float32 or not tw.is_contiguous():   # as fused_topk already gives
            self.tw.copy_(tw)
            tw = self.tw
        if overlap:
            split_fresh(self.align[1], self.cache.miss, self.cache.n_miss, self.cache.S,
                        self.eids_res, self.eids_new)
            self._gate_up_act(eh=self.eids_res)
            self._down(tw, eh=self.eids_res)
            torch.cuda.current_stream().wait_event(self.ev_up)
            self._gate_up_act(eh=self.eids_new, cold=False)
            torch.cuda.current_stream().wait_stream(waited)
            self._down(tw, eh=self.eids_new, cold=False)
        else:
            if waited is not None:
                torch.cuda.current_stream().wait_stream(waited)
            self._gate_up_act()
            if self.fold_sum:
                ids = topk_ids
                if ids.dtype != torch.int32 or not ids.is_contiguous():
                    self.ids32.copy_(ids)
                    ids = self.ids32
                w = (self.cache.table, self.slots.w2, self.slots.s2, self.full.w2, self.full.s2,
                     output)
                if self.fuse_dec:                  # the folded down quantizes the activation
                    ops.moe_down_sum_act(self.act, ids, tw.view(M, self.top_k), *w)
                else:
                    ops.moe_down_sum(self.q2, self.s2, ids, tw.view(M, self.top_k), *w)
                return
            self._down(tw)
        ops.moe_sum(self.ic3.view(M, self.top_k, self.H), output)
