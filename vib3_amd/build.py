"""Build libvib3_hip.so for gfx950 with hipcc, in-tree (vib3_amd/libvib3_hip.so).

Each translation unit compiles to an object of its own (in parallel, under vib3_amd/_build/),
then one hipcc line links them into the shared library.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libvib3_hip.so")
SOURCES = ["api.hip", "int4_gemv.hip", "router.hip", "synth.hip", "mxfp4_moe.hip", "norm.hip",
           "vib3file.cpp", "fp4_fused.hip", "fp4_pages.hip"]
ARCH = os.environ.get("VIB3_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Wall", "-Wno-unused-function",
    # packed fp32 VALU ops are kept out of the generated code on this platform
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed: " + " ".join(cmd[-3:]))


def build(verbose: bool = False, extra_flags=(), sources=None, out: str = LIB,
          objdir: str = OBJ) -> str:
    """Compile `sources` (default SOURCES) and link them into `out`; returns `out`."""
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    sources = list(SOURCES if sources is None else sources)
    os.makedirs(objdir, exist_ok=True)
    objs = [os.path.join(objdir, os.path.splitext(s)[0] + ".o") for s in sources]
    cmds = [[hipcc, *HIPCC_FLAGS, *extra_flags, "-c", "-o", o, os.path.join(CSRC, s)]
            for s, o in zip(sources, objs)]
    jobs = min(len(cmds), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", out + ".tmp", *objs],
         verbose)
    os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
