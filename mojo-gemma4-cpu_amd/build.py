"""Build libbq.so (the gfx950 butterquant library) in-tree with hipcc.

    python mojo-gemma4-cpu_amd/build.py

Each csrc/*.hip is compiled to an object in parallel, then linked into
mojo-gemma4-cpu_amd/libbq.so; calib/*.hip (the benchmark's streaming-read and
MFMA measurement kernels, no part of the API) into libbq_calib.so.  Flags:
  -ffp-contract=off   the epilogues restate the reference's f32 op order and
                      use fmaf only where the reference calls .fma
  -Xclang -target-feature -Xclang -packed-fp32-ops
                      no packed-FP32 VALU ops (the host pass warns that it does
                      not know the feature; the device pass takes it)
  -Xarch_device -mllvm=-amdgpu-kernarg-preload-count=16
                      the first 16 dwords of every kernel's scalar arguments
                      arrive preloaded in SGPRs at dispatch, so no argument
                      load precedes the first address (a one-token norm-quant
                      4.22 -> 4.02 us); the compiler keeps a loading prologue
                      for a dispatcher that does not preload
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libbq.so")
CALIB = os.path.join(HERE, "calib")
CALIB_LIB = os.path.join(HERE, "libbq_calib.so")
ARCH = os.environ.get("BQ_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Xarch_device", "-mllvm=-amdgpu-kernarg-preload-count=16",
    "-Wall", "-Wno-unused-function", "-I", os.path.join(HERE, "..", "include"),
]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.basename(os.path.dirname(src)) + "_" +
                       os.path.basename(src) + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in (r.stderr or "").splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def _link(objs, lib: str) -> None:
    tmp = lib + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, lib)


def build(verbose: bool = True) -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    csrcs = sorted(glob.glob(os.path.join(CALIB, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs) + len(csrcs))) as ex:
        objs = list(ex.map(_compile, srcs + csrcs))
    _link(objs[: len(srcs)], LIB)
    _link(objs[len(srcs):], CALIB_LIB)
    if verbose:
        print(f"built {LIB}, {CALIB_LIB}")
    return LIB


if __name__ == "__main__":
    build()
