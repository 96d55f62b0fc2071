"""Build recipe for libunikern_hip.so (gfx950 only).

Host C++ (front end, solver, inputs, self-check) is compiled with g++; HIP sources (kernels and
the C ABI) with hipcc --offload-arch=gfx950. Objects go to unikern_amd/_build/ and the shared
library to unikern_amd/libunikern_hip.so, in-tree, so it travels with the repository snapshot.

Usage: python3 unikern_amd/build.py

Run it by path: `python -m unikern_amd.build` imports the package first, and the package loads
the library this script builds, so it fails whenever that library is missing or stale.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libunikern_hip.so"
CLI = PKG / "unikern"
ROOT = PKG.parent

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
ARCH = "gfx950"

COMMON = ["-O3", "-std=c++20", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter", f"-I{ROOT / 'include'}", f"-I{CSRC}"]
# Packed-FP32 instructions are disabled for all device code (a hipcc flag; the host pass warns
# that it does not know the feature, which is harmless).
HIP_FLAGS = COMMON + [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                      "-Wno-unused-result"]
CXX_FLAGS = COMMON + ["-ffp-contract=off"]


def _sources():
    host = sorted((CSRC / "host").glob("*.cpp"))
    hip = sorted((CSRC / "kernels").glob("*.hip")) + [CSRC / "capi.hip"]
    return host, hip


def _compile(src: Path) -> Path:
    rel = src.relative_to(CSRC)
    obj = OBJ / (str(rel).replace("/", "__") + ".o")
    if src.suffix == ".hip":
        cmd = [HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    else:
        cmd = [CXX, *CXX_FLAGS, "-c", str(src), "-o", str(obj)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{p.stdout}\n{p.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every source and link libunikern_hip.so. Always rebuilds."""
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    OBJ.mkdir(exist_ok=True)
    host, hip = _sources()
    srcs = hip + host  # the long HIP compiles first
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs), "-lpthread", "-ldl"]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{p.stdout}\n{p.stderr}")
    os.replace(tmp, LIB)
    # The command-line front door, over the C ABI only; finds the library next to itself.
    cli_tmp = CLI.with_suffix(".tmp")
    cmd = [CXX, "-O2", "-std=c++20", "-Wall", f"-I{ROOT / 'include'}", str(CSRC / "cli" / "unikern.cpp"), "-o",
           str(cli_tmp), f"-L{PKG}", "-lunikern_hip", "-Wl,-rpath,$ORIGIN", "-Wl,-rpath-link,/opt/rocm/lib"]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"CLI build failed: {' '.join(cmd)}\n{p.stdout}\n{p.stderr}")
    os.replace(cli_tmp, CLI)
    if verbose:
        print(f"built {LIB} from {len(objs)} objects, and {CLI}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
