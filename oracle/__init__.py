"""CPU oracle for the MoE decode hot path (test infrastructure, not product).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import anything from this package, and only as the checker (or, for ``cpu_baseline``, as the
timed CPU restatement). The product path in ``r9700-lru-expert-cache_amd/`` never imports it
and fails loudly when its HIP library is missing.

Modules:
  lru     numpy restatement of the device LRU manager, the fused manager + align, the gather,
          and the warm start (kernels/lru/r4d_lru.hip, patches/.../r4d_mxfp4_moe.py.lru.diff)
  clru    ctypes binding of lru_oracle.c: an independent serial (argmin-per-insert) C
          restatement of the same functions, used to pin the numpy one
  fp8     bit-exact float32 <-> OCP e4m3fn conversion and the block / group / SiLU quantizers
  gemm    fp32-dequant grouped MoE GEMM and moe_sum
  w4      the int4 group-128 quantizer, this build's W4 layout, and the float64 W4 GEMV

Parity status of every function is listed in each module's header.
"""
