"""Build block_lut_amd/liblutmoe.so for gfx950 with hipcc (in-tree).

    python -m block_lut_amd.csrc.build          # or build() from Python

Each .hip / .cpp translation unit is compiled to an object in parallel, then
linked into one shared library exporting the C ABI of include/lutmoe.h.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
LIB = os.path.join(PKG, "liblutmoe.so")
SOURCES = ["api.cpp", "dequant.hip", "gemv.hip", "decode.hip", "route.hip", "gemm.hip",
           "encode.hip", "noalloc.hip", "dense.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    p = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(p):
        raise RuntimeError("hipcc not found; cannot build liblutmoe.so")
    return p


def common_flags():
    return [
        f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
        "-I", os.path.join(ROOT, "include"),
        # packed-fp32 instructions stay off (hipcc's host pass warns that it
        # does not know the feature; that warning is expected)
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
    ]


def _compile(src: str, obj_dir: str) -> str:
    obj = os.path.join(obj_dir, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *common_flags(), "-c", os.path.join(HERE, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    obj_dir = os.path.join(PKG, "_build")
    os.makedirs(obj_dir, exist_ok=True)
    jobs = min(len(SOURCES), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, obj_dir), SOURCES))
    # the inline-asm LDS-DMA loads against the VALU-SGPR-write hazard (the
    # compiler does not guard inline asm): a library with one is not linked
    if HERE not in sys.path:
        sys.path.insert(0, HERE)
    import isa_check
    hazards = isa_check.check_objects(objs)
    if hazards:
        raise RuntimeError("LDS-DMA load reads an SGPR a VALU instruction wrote fewer than "
                           f"{isa_check.WAIT_STATES} wait states earlier:\n" +
                           "\n".join("  |  ".join(map(str, h)) for h in hazards))
    tmp = LIB + f".tmp{os.getpid()}"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
