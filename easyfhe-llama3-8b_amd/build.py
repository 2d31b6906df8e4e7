"""Build the gfx950 backend library (easyfhe/_lib/libckks_mi355x.so) with hipcc.

Every HIP source is compiled for gfx950 only, with packed-FP32 instruction
selection disabled and floating-point contraction off (the encoder is
bit-exact with its CPU statement only without FMA contraction).
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "csrc"
OUT_DIR = HERE / "easyfhe" / "_lib"
LIB = OUT_DIR / "libckks_mi355x.so"
BUILD = HERE / "csrc" / "build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]
SOURCES = ["ckks_kernels.hip", "ckks_api.hip"]
# per-source flags: the int8 matrix-core conversion keeps its accumulators in
# ordinary VGPRs (the AGPR form moves every accumulator through v_accvgpr
# reads and writes, which the VALU pays for); fully unrolled loops stay
# unrolled up to a larger body (below it the tile-resident conversion's row
# loop was left rolled, and its per-row register arrays went to scratch
# memory)
EXTRA = {"ckks_kernels.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form",
                              "-mllvm", "-pragma-unroll-threshold=40000"]}


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    OUT_DIR.mkdir(parents=True, exist_ok=True)

    def compile_one(name: str) -> Path:
        obj = BUILD / (Path(name).stem + ".o")
        cmd = [HIPCC, *FLAGS, *EXTRA.get(name, []), "-c", str(SRC / name), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        return obj

    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
