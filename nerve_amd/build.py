"""Builds libnerve_hip.so for gfx950 with hipcc (in-tree, no JIT cache).

Usage: python -m nerve_amd.build
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libnerve_hip.so")
SOURCES = ["context.hip", "mxfp4_moe.hip", "routing.hip", "int4.hip", "fp8_head.hip", "rms_quant.hip", "int4_moe.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-fPIC",
    "-std=c++17",
    # Packed-FP32 VALU forms are kept out of generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-fast-math",
    "-ffp-contract=off",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-result",
]


def _compile(src: str) -> str:
    out = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", out]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return out


# Read-only HBM calibration kernels for bench.py's hbm_read workload: a
# library of their own, so the hot-path library carries no measurement code.
CALIB_SOURCES = ["hbm_calib.hip"]
CALIB_LIB = os.path.join(HERE, "libnerve_calib.so")


def _link(objs, out):
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", out, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")


def build() -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = [s for s in SOURCES + CALIB_SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = dict(zip(srcs, ex.map(_compile, srcs)))
    _link([objs[s] for s in SOURCES if s in objs], LIB)
    _link([objs[s] for s in CALIB_SOURCES if s in objs], CALIB_LIB)
    return LIB


if __name__ == "__main__":
    print(build())
