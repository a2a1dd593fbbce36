"""Compile the gfx950 HIP sources into the in-tree C-ABI library.

    python -m nanoserve_amd._build

The library is a plain shared object linked only against libamdhip64 and
loaded with ctypes, so it does not depend on torch's C++ ABI.  It is built
in-tree (next to this file) so a snapshot of the repository carries it to a
GPU machine as is.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
LIB_NAME = "libnanoserve_paged.so"
LIB_PATH = PKG_DIR / LIB_NAME
SOURCES = ["paged_attention.hip", "decode_plan.hip", "reshape_and_cache.hip", "rope_cache.hip",
           "int4_linear.hip", "argmax.hip", "generic_attention.hip"]
# The benchmark's measurement probe (an empty launch and a plain streaming
# read) is a library of its own: nothing in the product loads or declares it.
FLOORS_SOURCES = ["floors.hip"]
FLOORS_LIB_PATH = PKG_DIR / "libnanoserve_floors.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Keep the compiler from forming packed-fp32 VALU instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the softmax rescales them every step, and
    # AGPR accumulators would cost a read and a write per element each time.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    # Single-lane atomics stay single-lane: the atomic optimizer turns them
    # into a wave-wide pattern that reads the result back at once, which
    # makes the issuing wave wait for every load it has in flight.
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-Wall",
]


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise FileNotFoundError("hipcc not found (set HIPCC or install ROCm)")


def build(verbose: bool = False) -> Path:
    """Compile the product's HIP sources into LIB_PATH; always recompiles."""
    return _compile(SOURCES, LIB_PATH, verbose)


def build_floors(verbose: bool = False) -> Path:
    """Compile the benchmark's measurement probe into FLOORS_LIB_PATH."""
    return _compile(FLOORS_SOURCES, FLOORS_LIB_PATH, verbose)


def _compile(sources: list[str], lib_path: Path, verbose: bool) -> Path:
    tmp = lib_path.with_suffix(".so.tmp")
    cmd = [hipcc_path(), *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-o", str(tmp)]
    cmd += [str(CSRC / s) for s in sources]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that
    # line is expected and is filtered out of anything we print.
    noise = "is not a recognized feature for this target"
    log = "\n".join(l for l in (proc.stdout + proc.stderr).splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{' '.join(cmd)}\n{log}")
    if verbose and log.strip():
        print(log, file=sys.stderr)
    os.replace(tmp, lib_path)
    return lib_path


if __name__ == "__main__":
    print(build(verbose=True))
    print(build_floors(verbose=True))
