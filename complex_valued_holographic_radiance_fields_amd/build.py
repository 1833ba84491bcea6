"""Build the gfx950 HIP library ``lib/libhrf.so`` in-tree with hipcc.

Run as a script (``python complex_valued_holographic_radiance_fields_amd/build.py``)
or through ``__graft_entry__.build()``; it imports nothing from the package,
whose ``__init__`` loads the library this file builds.

Every source under ``csrc/`` is compiled separately (in parallel) and linked
into one shared library exposing the C ABI of ``include/hrf.h``.  Flags:

* ``--offload-arch=gfx950`` only (MI355X);
* ``-ffp-contract=off`` so expressions that must match the reference bit for
  bit are evaluated in source order (FMAs are written out explicitly);
* ``-fhip-fp32-correctly-rounded-divide-sqrt`` (IEEE division and sqrt);
* ``-Xclang -target-feature -Xclang -packed-fp32-ops`` disables packed FP32
  (v_pk_*_f32) code generation.
"""
from __future__ import annotations

import concurrent.futures as _cf
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libhrf.so")
OBJ_DIR = os.path.join(REPO_DIR, "_build", "obj")

SOURCES = [
    "raster_geom.hip",
    "geom_ops.hip",
    "raster_sort.hip",
    "raster_render.hip",
    "asm_prop.hip",
    "asm_fft.hip",
    "hrf_capi.hip",
    "preprocess.hip",
    "optim.hip",
    "recon.hip",
    "ssim.hip",
    "hrf_trace.hip",
]

COMMON_FLAGS = [
    "-std=c++17",
    "-O3",
    "-fPIC",
    "--offload-arch=gfx950",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    "-I", INCLUDE,
    "-I", CSRC,
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [_hipcc(), *COMMON_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
    if verbose and res.stderr.strip():
        print(res.stderr, file=sys.stderr)
    return obj


def build_library(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile all HIP sources and link ``lib/libhrf.so``; returns its path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    jobs = jobs or min(len(SOURCES), max(1, (os.cpu_count() or 2)))
    with _cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), "-shared", "-fPIC", "--offload-arch=gfx950", *objs,
           "-L/opt/rocm/lib", "-lhipfft", "-Wl,-rpath,/opt/rocm/lib", "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


TEST_SRC = os.path.join(REPO_DIR, "tests", "hip", "wave_reduce_test.hip")
TEST_LIB = os.path.join(REPO_DIR, "tests", "hip", "libwave_test.so")


def build_test_library(verbose: bool = False) -> str:
    """Compile the GPU unit-test kernels of tests/hip (wave reductions)."""
    cmd = [_hipcc(), *COMMON_FLAGS, "-shared", TEST_SRC, "-o", TEST_LIB + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {TEST_SRC}:\n{res.stdout}\n{res.stderr}")
    os.replace(TEST_LIB + ".tmp", TEST_LIB)
    return TEST_LIB


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv))
    print(build_test_library(verbose="-v" in sys.argv))
