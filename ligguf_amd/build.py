"""Build the native libraries in-tree.

* ``libligguf_hip.so``   -- the gfx950 kernels + C-ABI (include/ligguf_hip.h),
  compiled with hipcc for gfx950 only.
* ``libligguf_encode.so`` -- host-side weight encoders (include/ligguf_encode.h).

Run ``python -m ligguf_amd.build``.  Every call recompiles.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
HIP_SO = os.path.join(PKG, "libligguf_hip.so")
ENC_SO = os.path.join(PKG, "libligguf_encode.so")

HIP_SOURCES = ["lg_fused.hip", "lg_fused_p1.hip", "lg_fused_p2.hip", "lg_fused_p3.hip", "lg_prefill.hip", "lg_engine.hip",
               "lg_persist.hip", "lg_attn.hip", "lg_bert.hip", "lg_sample.hip", "lg_kernels.hip", "lg_matvec.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
    # packed fp32 ops stay off: hipcc -O3 would otherwise form v_pk_{add,mul,fma}_f32 from
    # ordinary float code, and some forms of those have returned wrong values on MI355X
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


def build_hip(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    objs = []

    def one(src):
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        _run([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        return obj

    with cf.ThreadPoolExecutor(max_workers=min(8, len(HIP_SOURCES))) as ex:
        objs = list(ex.map(one, HIP_SOURCES))
    tmp = HIP_SO + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, HIP_SO)
    if verbose:
        print("built", HIP_SO)
    return HIP_SO


def build_encode(verbose: bool = False) -> str:
    cc = shutil.which("gcc") or "cc"
    tmp = ENC_SO + ".tmp"
    _run([cc, "-O2", "-fPIC", "-fopenmp", "-shared", "-std=gnu11", "-Wall", "-Wextra", "-o", tmp,
          os.path.join(CSRC, "lg_encode.c"), "-lm"])
    os.replace(tmp, ENC_SO)
    if verbose:
        print("built", ENC_SO)
    return ENC_SO


def build_all(verbose: bool = False) -> None:
    build_encode(verbose)
    build_hip(verbose)


if __name__ == "__main__":
    build_all(verbose=True)
    sys.exit(0)
