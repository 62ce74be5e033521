"""Build libplastic_infer_amd.so for gfx950 with hipcc.

Every ``*.hip`` file in this directory is compiled to an object under ``<pkgroot>/_build`` and
linked into ``<pkgroot>/plastic_infer/_lib/libplastic_infer_amd.so`` (in-tree, so the library
travels with the source tree). Compilation always runs (no staleness check): callers that want
the build call this, callers that only want to load the library use ``plastic_infer._native``.

Usage:  python plastic-infer_amd/csrc/build.py [-v]
"""

from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

CSRC = pathlib.Path(__file__).resolve().parent
PKG_ROOT = CSRC.parent
REPO_ROOT = PKG_ROOT.parent
INCLUDE = REPO_ROOT / "include"
BUILD_DIR = PKG_ROOT / "_build"
LIB_DIR = PKG_ROOT / "plastic_infer" / "_lib"
LIB_NAME = "libplastic_infer_amd.so"
ARCH = "gfx950"

# Packed-FP32 VALU forms are disabled for all device code (they are only a throughput
# optimisation and some of their encodings are unreliable on this target).
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-result",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]

# Per-file flags (none at present).
FILE_FLAGS: dict[str, list[str]] = {}


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not pathlib.Path(exe).exists():
        raise RuntimeError("hipcc not found (ROCm toolchain required to build the HIP library)")
    return exe


def _compile(src: pathlib.Path, verbose: bool) -> pathlib.Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [_hipcc(), *COMMON_FLAGS, *DEVICE_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src),
           "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the device-only feature flag: drop that noise.
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    return obj


def build_library(verbose: bool = False) -> pathlib.Path:
    """Compile every HIP source and link the shared library. Returns the library path."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(lambda s: _compile(s, verbose), sources))
    out = LIB_DIR / LIB_NAME
    tmp = out.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    path = build_library(verbose="-v" in sys.argv)
    print(path)
