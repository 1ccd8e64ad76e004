"""Writes tests/golden/lru_c1.npz: the 64-step LRU workload (E=512, S=257, top-10, 5 rows,
seeded Zipf(1.1) trace with drift, profile warm start) and the full cache state plus both
align outputs after every step, from the numpy oracle (cross-checked here against the serial
C restatement before anything is written).

    python tests/golden/gen_golden.py
"""
import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

from lru_cases import c1_trace  # noqa: E402
from oracle import clru, lru  # noqa: E402

ALIGN = ("sorted_hot", "eids_hot", "npad_hot", "sorted_cold", "eids_cold", "npad_cold")


def main():
    ids, s = c1_trace()
    c = s.copy()
    out = {"ids": ids}
    for n, name in enumerate(lru.LruState.NAMES):
        out[f"init_{name}"] = getattr(s, name).copy()
    for n in range(ids.shape[0]):
        a = lru.fused(s, ids[n], 16)
        b = clru.fused(c, ids[n], 16)
        for x, y in zip(a, b):
            assert np.array_equal(x, y), f"oracles disagree at step {n}"
        for name in lru.LruState.NAMES:
            assert np.array_equal(getattr(s, name), getattr(c, name)), (n, name)
            out[f"{name}_{n}"] = getattr(s, name).copy()
        for name, x in zip(ALIGN, a):
            out[f"{name}_{n}"] = x
    path = pathlib.Path(__file__).with_name("lru_c1.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
