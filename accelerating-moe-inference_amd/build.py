"""Builds libmoe_amd.so (the HIP kernels + C ABI) for gfx950 with hipcc.

    python accelerating-moe-inference_amd/build.py

Every HIP source is compiled with explicit floating-point contraction
(-ffp-contract=off: the kernels fuse only where __builtin_fmaf is written),
IEEE fp32 division, and packed-fp32 instructions disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmoe_amd.so")
HIP_SOURCES = ["gemm.hip", "route.hip", "elementwise.hip", "norm.hip", "attention.hip",
               "flash.hip", "capi.hip"]
DROPIN_LIB = os.path.join(HERE, "libmoe_dropin.so")
DROPIN_SOURCES = ["device.cpp", "tensor.cpp", "model_loader.cpp", "layer.cpp", "model.cpp",
                  "driver.cpp"]
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-result",
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    # MOE_HIPCC_DEFINES: extra -D flags for tile-configuration tuning builds
    extra = os.environ.get("MOE_HIPCC_DEFINES", "").split()
    cmd = [HIPCC, *HIP_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def _run(cmd, what):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{what} failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")


def build_dropin() -> str:
    """The C++ drop-in of the reference host API (Tensor, tensor_ops, Linear,
    PhiMLP, PhiMoE, ModelLoader): host code over the C ABI, built with g++."""
    srcs = [os.path.join(HERE, "host", f) for f in DROPIN_SOURCES]
    tmp = DROPIN_LIB + ".tmp"
    _run(["g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra",
          "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", *srcs, "-o", tmp,
          f"-L{HERE}", "-lmoe_amd", f"-L{ROCM}/lib", "-lamdhip64",
          "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{ROCM}/lib"], "drop-in build")
    os.replace(tmp, DROPIN_LIB)
    return DROPIN_LIB


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=len(HIP_SOURCES)) as ex:
        objs = list(ex.map(_compile, HIP_SOURCES))
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs], "link")
    os.replace(tmp, LIB)
    build_dropin()
    if verbose:
        print(f"built {LIB}\nbuilt {DROPIN_LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
