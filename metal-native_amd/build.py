"""Build libmetal_native_amd.so (the C-ABI HIP library) in-tree for gfx950.

Each source under csrc/ is compiled with hipcc and the objects are linked
against the HIP runtime that PyTorch-ROCm ships, so one process holds one HIP
runtime and torch's stream handles are valid in this library.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "metal_native")
LIB_NAME = "libmetal_native_amd.so"
BUILD_DIR = os.path.join(HERE, "_build")

SOURCES = ["mq_capi.cpp", "mq_gemv.hip", "mq_rows.hip", "mq_rstream.hip", "mq_gemmw.hip", "mq_gemm16.hip", "mq_tiled.hip", "mq_misc.hip", "mq_quant.hip", "mq_glue.hip", "mq_vecmat32.hip"]

HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
    "-ffp-contract=off",
    "-fvisibility=hidden",
    # keep the compiler from forming packed-fp32 VALU ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _hipcc() -> str:
    for cand in ("/opt/rocm/bin/hipcc", shutil.which("hipcc") or ""):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _torch_lib_dir() -> str:
    import torch  # noqa: PLC0415

    d = os.path.join(os.path.dirname(torch.__file__), "lib")
    if not os.path.exists(os.path.join(d, "libamdhip64.so")):
        raise RuntimeError(f"torch's libamdhip64.so not found under {d}")
    return d


def _compile(src: str, hipcc: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc, *HIP_FLAGS, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    hipcc = _hipcc()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(lambda s: _compile(s, hipcc), SOURCES))
    tlib = _torch_lib_dir()
    out = os.path.join(OUT_DIR, LIB_NAME)
    tmp = out + ".tmp"
    cmd = ["g++", "-shared", "-o", tmp, *objs, f"-L{tlib}", "-lamdhip64", f"-Wl,-rpath,{tlib}",
           "-Wl,--no-undefined", "-Wl,-z,defs"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
