"""Build the gfx950 HIP library ``mlc_decode_amd/lib/libmla_decode_amd.so`` in-tree.

One ``hipcc`` invocation compiles the split-KV kernel, the combine kernel, the schedule
kernel and the C ABI of ``include/mla_decode_amd.h`` into a shared library that
``mlc_decode_amd._lib`` loads with ctypes.  Runs without a GPU (hipcc cross-compiles).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libmla_decode_amd.so")
SOURCES = [os.path.join(CSRC, "mla_decode.hip")]
# bench.py's MFMA-rate and shader-clock probe (a measurement helper, not the decode's ABI)
PROBE_PATH = os.path.join(LIB_DIR, "libmla_probe.so")
PROBE_SOURCES = [os.path.join(CSRC, "mla_probe.hip")]
ARCH = "gfx950"


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the HIP toolchain (ROCm) is required to build")
    return path


def build(verbose: bool = False) -> str:
    """Compile the decode library and the probe library; return the decode library's path.
    Always recompiles."""
    _compile(SOURCES, LIB_PATH, verbose)
    _compile(PROBE_SOURCES, PROBE_PATH, verbose)
    return LIB_PATH


def _compile(sources, target: str, verbose: bool) -> None:
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = target + ".tmp"
    cmd = [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        # Packed-FP32 VALU ops are kept out of the generated code (see the repository notes
        # on gfx950 packed fp32); hipcc's host pass warns that it does not know the feature.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", INCLUDE,
        "-I", CSRC,
        "-o", tmp,
        *sources,
    ]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with exit code {proc.returncode}")
    if verbose:
        noise = "is not a recognized feature for this target"
        for line in (proc.stdout + proc.stderr).splitlines():
            if noise not in line and line.strip():
                print(line)
    os.replace(tmp, target)


if __name__ == "__main__":
    print(build(verbose=True))
