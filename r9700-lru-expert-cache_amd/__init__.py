"""MI355X-native (gfx950) MoE decode hot path with a device-side LRU expert cache.

Drop-in for the librlu.so entry points and op wrappers of davetha/r9700-lru-expert-cache
(kernels/lru/r4d_lru.hip, patches/.../fused_moe/experts/r4d_mxfp4_moe.py.lru.diff). All device
work runs in lib/librlu.so (hand-written HIP for gfx950, C-ABI in include/rlu.h); this package
is the host side: ctypes bindings, the reference's op wrappers, and the per-layer state.
"""
from . import _lib  # noqa: F401
from ._lib import LIB_PATH, LibraryMissing, lib  # noqa: F401
from .lru import (LruCache, _align_sizes, _r4d_lru_fused, _r4d_lru_gather,  # noqa: F401
                  _r4d_lru_manage)
from . import ops  # noqa: F401
from . import hot_profile  # noqa: F401
from . import routecap  # noqa: F401
from . import traces  # noqa: F401
from . import w4  # noqa: F401
from .moe import ExpertWeights, LruMoELayer  # noqa: F401
