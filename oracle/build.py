"""Build recipe for the CPU oracle (test infrastructure): oracle/liboracle.so.

The oracle is the CPU restatement tests/, smoke() and bench.py's cpu_baseline compare
against. It is built with g++ with floating-point contraction disabled, so its
single-precision operation sequence matches the GPU kernels that share
threedgaussiansplatting.jl_amd/csrc/tdgs_math.hpp.

The reference's only native component (deps/cub_sort_pairs/cub_sort_pairs_wrapper.cu)
needs nvcc and CUB, which this image does not have, so no reference build exists here.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
SRC = [os.path.join(HERE, "tdgs_oracle.cpp")]
HEADERS = [
    os.path.join(HERE, "..", "threedgaussiansplatting.jl_amd", "csrc", "tdgs_math.hpp"),
    os.path.join(HERE, "..", "include", "tdgs.h"),
]


def build(force: bool = True) -> str:
    if not force and os.path.exists(LIB):
        newest = max(os.path.getmtime(p) for p in SRC + HEADERS)
        if os.path.getmtime(LIB) >= newest:
            return LIB
    tmp = LIB + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off", "-pthread",
           *SRC, "-o", tmp]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(force="--if-stale" not in sys.argv))
