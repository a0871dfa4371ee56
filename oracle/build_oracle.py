"""Build the CPU oracle (test infrastructure) into oracle/build/liboracle.so.

The oracle is plain C compiled with gcc; -ffp-contract=off keeps every
multiply-add in the synthetic-input generator separately rounded unless the
source asks for fmaf(), so it produces the same bits as the GPU generator.

The reference's own kernels (CUDA + LibTorch + NCCL) cannot be compiled in this
image, so there is no oracle/_ref build.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "build")
LIB = os.path.join(OUT_DIR, "liboracle.so")


def build(verbose=False):
    os.makedirs(OUT_DIR, exist_ok=True)
    src = os.path.join(HERE, "fp8lin_oracle.c")
    tmp = LIB + ".tmp"
    cmd = ["gcc", "-O2", "-march=x86-64-v3", "-ffp-contract=off", "-fno-fast-math",
           "-fopenmp", "-std=c11", "-Wall", "-Wextra", "-shared", "-fPIC",
           "-o", tmp, src, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
