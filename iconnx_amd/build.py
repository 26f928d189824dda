"""Ahead-of-time build of libiconnx_hip.so for gfx950 (hipcc; no JIT, no torch extension).

    python -m iconnx_amd.build        # or iconnx_amd.build.build()

Objects go to iconnx_amd/_build/ (git-ignored); the shared library is written in-tree as
iconnx_amd/libiconnx_hip.so so it travels with the source tree.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libiconnx_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -ffp-contract=off: every f32 op of the epilogue rounds once (no FMA contraction), as the
#   reference's separate ONNX nodes do.
# -fhip-fp32-correctly-rounded-divide-sqrt: IEEE f32 division in the Div epilogue op.
# -packed-fp32-ops disabled: no v_pk_*_f32 generation.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# host-only C++ (the graph executor) goes through hipcc for the HIP runtime headers
HOST_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Wall"]
SOURCES = ["dql.hip", "gemm.hip", "elementwise.hip", "encoder.hip", "layout.hip", "executor.cpp", "memory.cpp"]


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    flags = HIP_FLAGS if src.endswith(".hip") else HOST_FLAGS
    cmd = [HIPCC, *flags, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed for %s:\n%s\n%s" % (src, " ".join(cmd), r.stderr))
    return obj


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=4) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n%s\n%s" % (" ".join(cmd), r.stderr))
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
