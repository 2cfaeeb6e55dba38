"""Builds libsolvedelta_hip.so in-tree with hipcc for gfx950.

Usage: python -m solvedelta_amd.build   (or solvedelta_amd.build.build()).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libsolvedelta_hip.so")
# sd_fwd_noalloc and its static device array, in a library of their own so that
# only the processes that call it carry the array
NOALLOC_SRC = os.path.join(CSRC, "noalloc", "sd_noalloc.hip")
NOALLOC_LIB = os.path.join(HERE, "libsolvedelta_noalloc.so")
OBJ = os.path.join(HERE, "_obj")
ARCH = os.environ.get("SD_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # keep the compiler from emitting packed-fp32 VALU ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    # scheduler: relaxed occupancy targets and memory-clause grouping (the chunk
    # kernels run one latency-bound workgroup per CU): F+B 0.859 -> 0.854 ms
    "-mllvm", "-amdgpu-schedule-relaxed-occupancy",
    "-mllvm", "-amdgpu-sched-strategy=max-memory-clause",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src):
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr[-6000:]}")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
           "-Wl,-soname,libsolvedelta_hip.so"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-4000:]}")
    os.replace(tmp, LIB)
    nobj = _compile(NOALLOC_SRC)
    tmp = NOALLOC_LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, nobj,
           f"-L{HERE}", "-lsolvedelta_hip", "-Wl,-rpath,$ORIGIN"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-4000:]}")
    os.replace(tmp, NOALLOC_LIB)
    if verbose:
        print(f"built {LIB} and {NOALLOC_LIB}")
    return LIB


if __name__ == "__main__":
    build()
