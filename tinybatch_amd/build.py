"""Build libtinybatch_amd.so (gfx950) in-tree with hipcc.

Usage: python -m tinybatch_amd.build   (or tinybatch_amd.build.build()).
The library is a plain C-ABI shared object; Python reaches it via ctypes.
Each source compiles to its own object in parallel (tinybatch_amd/_build/),
then one link makes the library.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
OBJ_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libtinybatch_amd.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
SOURCES = ["tb_append.hip", "tb_attention.hip", "tb_copy.hip", "tb_fused.hip", "tb_linear.hip", "tb_decode.hip",
           "tb_prefill.hip", "tb_metadata.cpp"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # packed fp32 VALU forms are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(REPO_DIR, "include"),
]

# hipcc's host pass warns that it does not know the packed-fp32 feature: harmless
_NOISE = "'-packed-fp32-ops' is not a recognized feature for this target"


def _run(cmd: list[str]) -> tuple[int, str]:
    res = subprocess.run(cmd, capture_output=True, text=True)
    return res.returncode, "\n".join(l for l in res.stderr.splitlines() if _NOISE not in l)


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every HIP source into LIB_PATH; returns the library path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    jobs = jobs or min(len(SOURCES), max(1, min(os.cpu_count() or 1, 8)))
    cmds = []
    objs = []
    for s in SOURCES:
        obj = os.path.join(OBJ_DIR, os.path.splitext(s)[0] + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *FLAGS, "-c", os.path.join(CSRC, s), "-o", obj])
    if verbose:
        for c in cmds:
            print(" ".join(c), flush=True)
    with ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(_run, cmds))
    for (rc, err), s in zip(results, SOURCES):
        if rc != 0:
            raise RuntimeError(f"hipcc failed on {s} ({rc}):\n{err}")
        if err.strip() and verbose:
            print(err, file=sys.stderr)
    tmp = LIB_PATH + ".tmp"
    link = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(link), flush=True)
    rc, err = _run(link)
    if rc != 0:
        raise RuntimeError(f"link failed ({rc}):\n{err}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
