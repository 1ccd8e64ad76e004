"""ctypes binding of oracle/lru_oracle.c (serial C restatement; test infrastructure only).

``load()`` builds oracle/_build/liblru_oracle.so with gcc if it is missing (this is the
checker, not the product: the product library never falls back to it).
"""
from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

from .lru import LruState, align_sizes

_HERE = pathlib.Path(__file__).resolve().parent
_SO = _HERE / "_build" / "liblru_oracle.so"
_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int


def load():
    global _lib
    if _lib is None:
        src = _HERE / "lru_oracle.c"
        if not _SO.exists() or _SO.stat().st_mtime < src.stat().st_mtime:
            subprocess.run(["make", "-s", "-C", str(_HERE), "all"], check=True)
        lib = ctypes.CDLL(str(_SO))
        lib.oracle_lru_manage.restype = _I
        lib.oracle_lru_manage.argtypes = [_P] + [_I] * 5 + [_P] * 8
        lib.oracle_lru_fused.restype = _I
        lib.oracle_lru_fused.argtypes = [_P] + [_I] * 5 + [_P] * 8 + [_I] * 3 + [_P] * 7
        lib.oracle_lru_gather.restype = _I
        lib.oracle_lru_gather.argtypes = [_P, _P, ctypes.c_long] * 6 + [_P, _P]
        _lib = lib
    return _lib


def _p(a: np.ndarray):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(_P)


def _state_ptrs(s: LruState):
    return [_p(s.table), _p(s.map_cold), _p(s.slot_expert), _p(s.slot_stamp), _p(s.routed),
            _p(s.step), _p(s.miss), _p(s.n_miss)]


def manage(s: LruState, ids, max_distinct=None, max_inserts=None) -> int:
    ids = np.ascontiguousarray(np.asarray(ids, np.int32).reshape(-1))
    md = s.max_distinct if max_distinct is None else max_distinct
    mi = s.max_inserts if max_inserts is None else max_inserts
    rc = load().oracle_lru_manage(_p(ids), ids.size, s.E, s.S, md, mi, *_state_ptrs(s))
    if rc != 0:
        raise ValueError(f"oracle_lru_manage rc={rc}")
    return int(s.n_miss[0])


def fused(s: LruState, ids, bs, L=None, NB=None, max_distinct=None, max_inserts=None):
    ids = np.ascontiguousarray(np.asarray(ids, np.int32).reshape(-1))
    mk = ids.size
    if L is None or NB is None:
        L, NB = align_sizes(mk, s.E, bs)
    md = s.max_distinct if max_distinct is None else max_distinct
    mi = s.max_inserts if max_inserts is None else max_inserts
    out = [np.empty(L, np.int32), np.empty(NB, np.int32), np.empty(1, np.int32),
           np.empty(L, np.int32), np.empty(NB, np.int32), np.empty(1, np.int32)]
    scratch = np.empty(2 * mk + 4096, np.int32)
    rc = load().oracle_lru_fused(_p(ids), mk, s.E, s.S, md, mi, *_state_ptrs(s), bs, L, NB,
                                 *[_p(o) for o in out], _p(scratch))
    if rc != 0:
        raise ValueError(f"oracle_lru_fused rc={rc}")
    return tuple(out)
