"""Build recipe for the CPU oracle (test infrastructure: the checker, never the product).

Compiles oracle/kk_oracle.c into oracle/libkk_oracle.so with gcc.  -ffp-contract=off keeps every
multiply and add separately rounded, so the only fused multiply-adds are the explicit fmaf() calls
that restate the reference's own fmaf() (kernels/kokoro.cu:214-222, 239-248).
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "kk_oracle.c")
OUT = os.path.join(HERE, "libkk_oracle.so")

CFLAGS = ["-O3", "-std=gnu11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
          "-fno-math-errno", "-march=x86-64-v3", "-Wall", "-Wno-unused-function", "-Wno-format-truncation"]


def build(verbose=False):
    cmd = ["gcc", *CFLAGS, SRC, "-o", OUT + ".tmp", "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
