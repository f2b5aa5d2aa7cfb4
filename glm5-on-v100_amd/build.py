"""Builds libmi355_dsa.so (all HIP kernels + the C ABI) for gfx950, in-tree.

Usage: python glm5-on-v100_amd/build.py   (or __graft_entry__.build())

Each csrc/*.hip is compiled to an object in _build/ (in parallel), then the
objects are linked into <package>/libmi355_dsa.so.  hipcc cross-compiles
gfx950 code without a GPU.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libmi355_dsa.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ARCH = "gfx950"


def hipcc() -> str:
    p = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(p):
        raise RuntimeError("hipcc not found; the HIP toolchain is required")
    return p


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Wall",
        "-Wno-unused-function",
        # packed fp32 VALU forms are kept out of generated code on purpose
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", os.path.join(PKG_DIR, "..", "include"),
    ]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src).replace(".hip", ".o"))
    cmd = [hipcc(), *compile_flags(), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


TESTKIT_SRC = os.path.join(PKG_DIR, "..", "tests", "hip", "quant_exhaustive.hip")
TESTKIT_LIB = os.path.join(PKG_DIR, "..", "tests", "hip", "libdsa_testkit.so")


def build_testkit(verbose: bool = True) -> str:
    """Builds the test-only kernels (tests/hip/*.hip) into
    tests/hip/libdsa_testkit.so; the product library does not contain them."""
    tmp = TESTKIT_LIB + ".tmp"
    cmd = [hipcc(), *compile_flags(), "-shared", TESTKIT_SRC, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {TESTKIT_SRC}:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, TESTKIT_LIB)
    if verbose:
        print(f"built {os.path.normpath(TESTKIT_LIB)}", flush=True)
    return TESTKIT_LIB


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError("no HIP sources found")
    jobs = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources", flush=True)
    return LIB_PATH


if __name__ == "__main__":
    build()
    build_testkit()
    sys.exit(0)
