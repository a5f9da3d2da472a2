"""Build recipe for the oracle's C restatement (test infrastructure only).

Compiles oracle/cpu_ref.c into oracle/libcpuref.so with the float semantics
of Go's default amd64 code generation: no contraction of a*b+c into a fused
multiply-add (-ffp-contract=off) and no fast-math.

The reference itself is Go (no Go toolchain in this image) and its only C
source, inference_core.c, holds no KV-cache or attention arithmetic, so no
build of the reference goes into oracle/_ref.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "cpu_ref.c")
OUT = os.path.join(HERE, "libcpuref.so")


def build(verbose=False):
    cmd = ["gcc", "-std=c11", "-O2", "-ffp-contract=off", "-fno-fast-math",
           "-fPIC", "-shared", "-pthread", "-Wall", "-Wextra", "-o", OUT + ".tmp", SRC, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
