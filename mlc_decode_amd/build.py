"""Build the gfx950 HIP library ``mlc_decode_amd/lib/libmla_decode_amd.so`` in-tree.

``hipcc`` compiles the split-KV kernels, the combine kernel, the schedule kernel and the C ABI
of ``include/mla_decode_amd.h`` into a shared library that ``mlc_decode_amd._lib`` loads with
ctypes.  Runs without a GPU (hipcc cross-compiles).  ``csrc/mla_decode_ws.hip`` (the dense
wave-split kernel) is compiled with LLVM's iterative ILP machine scheduler, every other
translation unit with the default one.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libmla_decode_amd.so")
# (source, extra hipcc flags) per translation unit
SOURCES = [
    (os.path.join(CSRC, "mla_decode.hip"), []),
    (os.path.join(CSRC, "mla_decode_ws.hip"), ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"]),
]
# bench.py's MFMA-rate and shader-clock probe (a measurement helper, not the decode's ABI)
PROBE_PATH = os.path.join(LIB_DIR, "libmla_probe.so")
PROBE_SOURCES = [(os.path.join(CSRC, "mla_probe.hip"), [])]
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


def _check(returncode: int, out: str, verbose: bool) -> None:
    if returncode != 0:
        sys.stderr.write(out)
        raise RuntimeError(f"hipcc failed with exit code {returncode}")
    if verbose:
        noise = "is not a recognized feature for this target"
        for line in out.splitlines():
            if noise not in line and line.strip():
                print(line)


def _run(cmd, verbose: bool) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    _check(proc.returncode, proc.stdout + proc.stderr, verbose)


def _compile(sources, target: str, verbose: bool) -> None:
    """Compile each (source, flags) unit to an object, then link them into ``target``."""
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = target + ".tmp"
    common = [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        # Packed-FP32 VALU ops are kept out of the generated code (see the repository notes
        # on gfx950 packed fp32); hipcc's host pass warns that it does not know the feature.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # scalar kernel arguments arrive preloaded in SGPRs (gfx950 kernarg preloading; the
        # code object keeps a preamble that loads them where the firmware does not)
        "-mllvm", "-amdgpu-kernarg-preload-count=16",
        "-I", INCLUDE,
        "-I", CSRC,
    ]
    with tempfile.TemporaryDirectory(prefix="mla_build_") as obj_dir:
        objs, procs = [], []
        for i, (src, flags) in enumerate(sources):  # the units compile side by side
            obj = os.path.join(obj_dir, f"{i}_{os.path.splitext(os.path.basename(src))[0]}.o")
            procs.append(subprocess.Popen([hipcc(), *common, *flags, "-c", "-o", obj, src],
                                          stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True))
            objs.append(obj)
        results = [(p.communicate()[0], p.returncode) for p in procs]
        for out, rc in results:
            _check(rc, out, verbose)
        _run([hipcc(), f"--offload-arch={ARCH}", "-fPIC", "-shared", "-o", tmp, *objs], verbose)
    os.replace(tmp, target)


if __name__ == "__main__":
    print(build(verbose=True))
