"""Builds libadi_hip.so in-tree: every HIP source under adi_amd/csrc (and the
host-only .cpp sources, compiled as HIP for the shared headers) built for
gfx950 with hipcc and linked into one shared library exporting the C ABI
declared in include/adi_hip.h and include/adi_hip_gguf.h.

    python -m adi_amd.build          # or adi_amd.build.build()
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(HERE, "_build")
LIBRARY = os.path.join(HERE, "libadi_hip.so")
ARCH = "gfx950"

# Packed FP32 instructions are kept out of every device code object: hipcc
# forms them from ordinary float code on its own otherwise.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = [
    "-O3", "-std=c++20", "-fPIC", f"--offload-arch={ARCH}",
    "-Wall", "-Wno-unused-command-line-argument",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; ROCm is required to build the HIP library")
    return path


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def _compile(source: str) -> str:
    stem, ext = os.path.splitext(os.path.basename(source))
    obj = os.path.join(BUILD_DIR, stem + ".o")
    # host-only .cpp sources share the HIP headers of the library
    lang = ["-x", "hip"] if ext == ".cpp" else []
    cmd = [hipcc(), *COMMON_FLAGS, *DEVICE_FLAGS, *lang, "-c", source, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(jobs: int = 0, verbose: bool = False) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIBRARY + ".tmp"
    cmd = [hipcc(), "-shared", f"--offload-arch={ARCH}", "-o", tmp, *objs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
