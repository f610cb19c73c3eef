"""Build the gfx950 shared library `nacho_amd/libnacho_hip.so` from `nacho_amd/csrc/*.hip`
(device code, hipcc for gfx950 only) and `nacho_amd/csrc/*.cpp` (host-only code, g++).

Every source is compiled in parallel, then linked into one
shared library exporting the C ABI declared in `include/nacho_hip.h`.  The library is built
in-tree so that it travels with the repository to the GPU machine.

    python -m nacho_amd.build          # rebuild

The HIP code generator for the GPU target (`nacho_amd/codegen`, host C++) is built beside it
as `nacho_amd/codegen/nacho_hipgen` by `build_codegen()`.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
CSRC_DIR = PACKAGE_DIR / "csrc"
BUILD_DIR = PACKAGE_DIR / "_build"
LIBRARY = PACKAGE_DIR / "libnacho_hip.so"
CODEGEN_DIR = PACKAGE_DIR / "codegen"
CODEGEN_EXE = CODEGEN_DIR / "nacho_hipgen"

ARCH = "gfx950"

# -packed-fp32-ops: keep hipcc from forming packed FP32 instructions.
# -ffp-contract=off: no FMA contraction, so every value is the single IEEE operation the
# reference performs (add and multiply must be bit-exact).
HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Keep single-lane atomics (tile tickets) plain: the wave-level atomic optimizer consumes
    # their result right away, which stalls on every load issued before them.
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
    f"-I{REPO_DIR / 'include'}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the gfx950 backend cannot be built")
    return path


# Host-only sources (no device code): compiled by the host C++ compiler.
HOST_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Wall", f"-I{REPO_DIR / 'include'}"]


def sources() -> list[Path]:
    return sorted(CSRC_DIR.glob("*.hip")) + sorted(CSRC_DIR.glob("*.cpp"))


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    if src.suffix == ".cpp":
        cxx = shutil.which("g++") or shutil.which("c++")
        if cxx is None:
            raise RuntimeError("no host C++ compiler (g++) for the host-only sources")
        cmd = [cxx, *HOST_FLAGS, "-c", str(src), "-o", str(obj)]
    else:
        cmd = [hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed on {src.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source for gfx950 and link libnacho_hip.so.  Always recompiles."""
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY} from {len(srcs)} sources", file=sys.stderr)
    return LIBRARY


def build_codegen(verbose: bool = False) -> Path:
    """Compile the code generator's command line, nacho_hipgen (host C++17, g++)."""
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        raise RuntimeError("no host C++ compiler (g++) for the code generator")
    tmp = CODEGEN_EXE.with_name(CODEGEN_EXE.name + ".tmp")
    cmd = [cxx, "-O2", "-std=c++17", "-Wall", "-Wextra", *map(str, sorted(CODEGEN_DIR.glob("*.cpp"))),
           "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"code generator build failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, CODEGEN_EXE)
    if verbose:
        print(f"built {CODEGEN_EXE}", file=sys.stderr)
    return CODEGEN_EXE


if __name__ == "__main__":
    build(verbose=True)
    build_codegen(verbose=True)
