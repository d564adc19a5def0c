"""Builds libw4a16.so in-tree with hipcc for gfx950 (no JIT, no cmake).

Usage: python -m ... or import and call build_library().  Each .hip source compiles to an
object in csrc/_build/, then all objects link into csrc/libw4a16.so.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(CSRC, "_build")
LIB_NAME = "libw4a16.so"
LIB_PATH = os.path.join(CSRC, LIB_NAME)
SOURCES = ("w4a16_format.hip", "w4a16_quant.hip", "w4a16_decode.hip", "w4a16_tile.hip", "w4a16_norm.hip",
           "w4a16_api.hip")
ARCH = "gfx950"

COMPILE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # no packed-FP32 instructions in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the W4A16 HIP library cannot be built")
    return path


def _compile(src: str, extra: list[str]) -> str:
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *COMPILE_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stderr}")
    return obj


def build_library(extra_flags: list[str] | None = None, jobs: int = 4) -> str:
    """Compile every HIP source for gfx950 and link libw4a16.so.  Returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    extra = list(extra_flags or [])
    with ThreadPoolExecutor(max_workers=max(1, min(jobs, len(SOURCES)))) as pool:
        objs = list(pool.map(lambda s: _compile(s, extra), SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link of {LIB_NAME} failed:\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


PROBE_SOURCE = "probe_read.hip"
PROBE_PATH = os.path.join(CSRC, "libw4a16_probe.so")


def build_probe() -> str:
    """Compile the benchmark's read probe (csrc/probe_read.hip) into libw4a16_probe.so, a
    measurement helper kept out of libw4a16.so.  Returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    tmp = PROBE_PATH + ".tmp"
    cmd = [hipcc(), *COMPILE_FLAGS, "-shared", os.path.join(CSRC, PROBE_SOURCE), "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {PROBE_SOURCE}:\n{proc.stderr}")
    os.replace(tmp, PROBE_PATH)
    return PROBE_PATH


if __name__ == "__main__":
    print(build_library())
    print(build_probe())
