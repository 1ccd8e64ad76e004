"""Build librlu.so (all HIP kernels of this package) for gfx950, in-tree.

    python -m ... build     or     build.build()

Every csrc/*.hip is compiled to an object with hipcc, then linked into lib/librlu.so. The
library travels with the source tree; nothing is JIT-compiled at run time.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import subprocess

HERE = pathlib.Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIBDIR = HERE / "lib"
LIB = LIBDIR / "librlu.so"
INCLUDE = HERE.parent / "include"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-I", str(INCLUDE),
         "-I", str(CSRC),
         # packed fp32 VALU forms are kept out of every kernel of this library
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _compile(src: pathlib.Path, obj: pathlib.Path) -> None:
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr}")


def build(verbose: bool = False) -> pathlib.Path:
    objdir = HERE / "_build"
    objdir.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    objs = [objdir / (s.stem + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        list(ex.map(_compile, srcs, objs))
    tmp = LIB.with_suffix(".so.tmp")
    r = subprocess.run([HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", str(tmp),
                        *map(str, objs)], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {[s.name for s in srcs]}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
