"""Build libkmoe.so (HIP, gfx950) in-tree with hipcc.

    python -m kappa_amd.build            # compile every source, link kappa_amd/libkmoe.so

Sources are compiled in parallel to objects under kappa_amd/_build/ and linked
into one shared library next to this file: the HIP files with hipcc, the
host-only validation and layout (host.cpp) with the system C++ compiler. Every device compile disables the
packed-FP32 VALU forms (-packed-fp32-ops); hipcc's host pass warns that it does
not know that feature, which is harmless.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libkmoe.so")
SOURCES = ["api.hip", "route.hip", "expert.hip", "weights.hip", "block.hip", "host.cpp"]
ARCH = os.environ.get("KMOE_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for p in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if p and os.path.exists(p):
            return p
    return "hipcc"


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Wall",
        "-Wno-unused-command-line-argument",
        "-fhip-fp32-correctly-rounded-divide-sqrt",
        "-Xclang",
        "-target-feature",
        "-Xclang",
        "-packed-fp32-ops",
        "-I",
        os.path.join(ROOT, "include"),
        "-I",
        CSRC,
    ]


def host_flags() -> list[str]:
    """The host-only translation unit (host.cpp: validation and workspace layout)
    is plain C++ and builds with the system compiler."""
    return ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-I", os.path.join(ROOT, "include"), "-I", CSRC]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    if src.endswith(".cpp"):
        cmd = [os.environ.get("CXX", "g++"), *host_flags(), "-c", os.path.join(CSRC, src), "-o", obj]
    else:
        cmd = [hipcc(), *compile_flags(), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    """Compile and link libkmoe.so; returns its path. Always rebuilds."""
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
