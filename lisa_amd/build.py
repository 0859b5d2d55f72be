"""Builds liblisaq.so (all HIP kernels + the C ABI) in-tree for gfx950.

Each source is compiled to an object in parallel with hipcc, then linked into
``lisa_amd/liblisaq.so``.  Compilation always runs (the driver's "does it
build" check); tests and the bench only load what is built.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
ROOT = os.path.dirname(HERE)
OUT = os.path.join(HERE, "liblisaq.so")
OBJ = os.path.join(ROOT, "_build", "lisaq")
SOURCES = ["qmv.hip", "qmv16.hip", "qmvt.hip", "qmvd.hip", "qmvp.hip", "qmvw.hip", "qmvs.hip", "qmm.hip", "qmm_k4_p.hip", "qmm_k4_s.hip", "qmm_k2_p.hip", "qmm_k2_s.hip", "qmm_gu.hip", "quant.hip", "qtyped.hip", "addnorm.hip", "diag.hip", "moe.hip", "moe_decode.hip", "api.cpp"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    "-Wno-unused-function",
    # packed FP32 instructions stay off: the compiler must not form
    # v_pk_{add,mul,fma}_f32 from scalar or float2 code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l and "--hip-link" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", OUT + ".tmp", *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(OUT + ".tmp", OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build(verbose=True)
