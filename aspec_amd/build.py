"""Builds libaspec_amd.so (all HIP kernels + the C ABI) for gfx950 with hipcc, in-tree.

Every `csrc/*.hip` file compiles to an object under `_build/` (in parallel), host-only
`csrc/*.cpp` files compile with the host C++ compiler, then one link step produces
`aspec_amd/libaspec_amd.so`, which travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC = PACKAGE_DIR / "csrc"
BUILD_DIR = PACKAGE_DIR.parent / "_build"
LIBRARY = PACKAGE_DIR / "libaspec_amd.so"
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed FP32 (v_pk_*_f32) stays off: scalar fp32 code only.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Run LLVM's machine verifier on the device code: an instruction selected with an operand of
    # the wrong register class fails the build instead of being encoded silently.
    "-mllvm", "-verify-machineinstrs",
]
# The loss and sampled-L1 kernels must evaluate draft and teacher probabilities (and the
# forward's and backward's) with identical instruction sequences; contraction into FMAs stays off.
PER_FILE_FLAGS = {"loss.hip": ["-ffp-contract=off"], "sampling.hip": ["-ffp-contract=off"]}


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the aspec_amd HIP library cannot be built")
    return path


HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall"]


def host_cxx() -> str:
    path = shutil.which("g++") or shutil.which("c++")
    if path is None:
        raise RuntimeError("no host C++ compiler found for the host-only sources")
    return path


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    if src.suffix == ".cpp":
        cmd = [host_cxx(), *HOST_FLAGS, "-c", str(src), "-o", str(obj)]
    else:
        cmd = [hipcc(), *COMMON_FLAGS, *PER_FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"{Path(cmd[0]).name} failed for {src.name}:\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link libaspec_amd.so. Always rebuilds."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(lambda s: _compile(s, verbose), sources))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
