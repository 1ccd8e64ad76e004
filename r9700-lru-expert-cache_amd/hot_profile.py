"""Hot-expert profiles: the on-disk warm-start format and the global budget split.

Mirrors the reference's profile handling (patches/model_executor/layers/fused_moe/experts/
r4d_mxfp4_moe.py.lru.diff:87-141: _hot_profile, _hot_sets, hot_ids_for_layer,
profile_rank_for_layer) and the file's writer (tools/routecap/build_hot_profile.py).

File format (JSON):
    {"source": str, "decode_tokens": int, "prefill_tokens": int,
     "layers": {"<layer index>": {"ranked": [expert ids, most routed first],
                                  "counts": [routings of those experts, same order]}}}

The budget split is a global water-fill: each layer's counts are normalized to fractions of
that layer's routings, every (layer, expert) pair is ordered by its fraction, highest first
(ties keep layer order, then rank order: a stable sort of the layers' lists concatenated in
the profile's layer order), and the first budget = floor(GB * 1e9 / per_expert_bytes) pairs
are kept. A layer's hot set is therefore a prefix of its ranked list; it is returned in
ascending expert order, the order the LRU warm start gives to the slots (slot i = i-th
smallest hot id, stamps by profile rank: LruCache.build).
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass

import numpy as np

ENV_PROFILE = "VLLM_R4D_HOT_PROFILE"
ENV_GB = "VLLM_R4D_HOT_GB"


@dataclass
class HotProfile:
    """layers: layer index -> (ranked expert ids int64 [E], counts float64 [E]), in the
    file's layer order (the water-fill's tie order)."""
    layers: dict[int, tuple[np.ndarray, np.ndarray]]
    source: str = ""
    decode_tokens: int = 0
    prefill_tokens: int = 0

    def rank(self, layer: int) -> dict[int, int] | None:
        """expert id -> rank in the layer's profile (0 = most frequently routed)."""
        if layer not in self.layers:
            return None
        return {int(e): i for i, e in enumerate(self.layers[layer][0].tolist())}

    def to_json(self) -> dict:
        return {"source": self.source, "decode_tokens": int(self.decode_tokens),
                "prefill_tokens": int(self.prefill_tokens),
                "layers": {str(li): {"ranked": r.tolist(), "counts": c.tolist()}
                           for li, (r, c) in self.layers.items()}}


def load(path: str | os.PathLike) -> HotProfile:
    """Reads a profile file (the format above)."""
    with open(path) as f:
        obj = json.load(f)
    layers = {int(k): (np.asarray(v["ranked"], dtype=np.int64),
                       np.asarray(v["counts"], dtype=np.float64))
              for k, v in obj["layers"].items()}
    for li, (r, c) in layers.items():
        if r.shape != c.shape:
            raise ValueError(f"hot profile layer {li}: ranked and counts differ in length")
    return HotProfile(layers, str(obj.get("source", "")), int(obj.get("decode_tokens", 0)),
                      int(obj.get("prefill_tokens", 0)))


def save(profile: HotProfile, path: str | os.PathLike) -> None:
    with open(path, "w") as f:
        json.dump(profile.to_json(), f)


def build(counts: np.ndarray, layer_ids=None, source: str = "", top_k: int = 10,
          prefill_counts: np.ndarray | None = None) -> HotProfile:
    """counts [L, E] routings per (layer, expert) -> a profile: each layer's experts ranked by
    count, highest first, ties in expert order (a stable sort), with their counts.
    decode_tokens = total routings / (L * top_k), as the reference's writer records it.
    layer_ids names the rows (default 0..L-1)."""
    counts = np.asarray(counts)
    if counts.ndim != 2:
        raise ValueError("counts must be [layers, experts]")
    L = counts.shape[0]
    ids = list(range(L)) if layer_ids is None else [int(x) for x in layer_ids]
    if len(ids) != L:
        raise ValueError("one layer id per row of counts")
    layers = {}
    for row, li in enumerate(ids):
        c = counts[row]
        order = np.argsort(-c, kind="stable")
        layers[li] = (order.astype(np.int64), c[order].astype(np.float64))
    pre = 0 if prefill_counts is None else int(np.asarray(prefill_counts).sum() // (L * top_k))
    return HotProfile(layers, source, int(counts.sum() // (L * top_k)), pre)


def budget_experts(budget_gb: float, per_expert_bytes: int) -> int:
    """How many (layer, expert) pairs budget_gb of HBM holds."""
    if per_expert_bytes <= 0:
        raise ValueError("per_expert_bytes must be positive")
    return int(float(budget_gb) * 1e9) // int(per_expert_bytes)


def hot_sets(profile: HotProfile, per_expert_bytes: int,
             budget_gb: float) -> dict[int, list[int]]:
    """The global water-fill (r4d_mxfp4_moe.py.lru.diff:100-126): layer -> hot expert ids,
    ascending. Raises ValueError when a layer has no routings."""
    budget = budget_experts(budget_gb, per_expert_bytes)
    keep_layers, keep_ids = _water_fill(profile, budget)
    out: dict[int, list[int]] = {li: [] for li in profile.layers}
    for li, e in zip(keep_layers.tolist(), keep_ids.tolist()):
        out[li].append(e)
    return {li: sorted(v) for li, v in out.items()}


def coverage(profile: HotProfile, per_expert_bytes: int, budget_gb: float) -> float:
    """The profile-estimated routing coverage the reference logs with its split: the kept
    fractions summed over layers, divided by the number of layers."""
    frac = _fractions(profile)
    keep = np.argsort(-frac[2], kind="stable")[:budget_experts(budget_gb, per_expert_bytes)]
    return float(frac[2][keep].sum()) / len(profile.layers)


def _fractions(profile: HotProfile):
    layers, ranked, fracs = [], [], []
    for li, (r, c) in profile.layers.items():
        tot = c.sum()
        if tot <= 0:
            raise ValueError(f"hot profile layer {li} has no routing counts")
        layers.append(np.full(len(r), li))
        ranked.append(r)
        fracs.append(c / tot)
    return np.concatenate(layers), np.concatenate(ranked), np.concatenate(fracs)


def _water_fill(profile: HotProfile, budget: int):
    layers, ranked, fracs = _fractions(profile)
    keep = np.argsort(-fracs, kind="stable")[:max(budget, 0)]
    return layers[keep], ranked[keep]


# ---- the reference's environment-driven entry points ------------------------------------------
def hot_profile() -> HotProfile | None:
    """The profile named by VLLM_R4D_HOT_PROFILE, or None (r4d_mxfp4_moe.py.lru.diff:87-96)."""
    path = os.environ.get(ENV_PROFILE)
    return load(path) if path else None


def hot_ids_for_layer(layer_idx: int, per_expert_bytes: int) -> list[int] | None:
    """None when no profile is configured or the layer is not profiled
    (r4d_mxfp4_moe.py.lru.diff:129-133). Raises ValueError when a profile is set but
    VLLM_R4D_HOT_GB is not."""
    prof = hot_profile()
    if prof is None:
        return None
    gb = os.environ.get(ENV_GB)
    if gb is None:
        raise ValueError(f"{ENV_PROFILE} is set but {ENV_GB} is not")
    return hot_sets(prof, per_expert_bytes, float(gb)).get(layer_idx)


def profile_rank_for_layer(layer_idx: int) -> dict[int, int] | None:
    """expert id -> rank in this layer's profile (r4d_mxfp4_moe.py.lru.diff:136-141)."""
    prof = hot_profile()
    return None if prof is None else prof.rank(layer_idx)
