"""Build recipe for the oracle (test infrastructure only).

Compiles oracle/fakref.c into oracle/_build/liboracle.so with the flags that reproduce amd64 Go
float semantics for the restated loops: no FP contraction (every product is rounded before it is
added), no fast-math reassociation. Vectorisation is left on: the four accumulators are
independent lanes, so any SIMD form gcc chooses computes the same per-lane sequence.

The reference itself (Go) cannot be built in this image (no Go toolchain), so there is no
oracle/_ref build.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "liboracle.so")
CFLAGS = ["-O3", "-ffp-contract=off", "-fno-fast-math", "-fno-math-errno", "-std=c11",
          "-fPIC", "-shared", "-pthread", "-Wall", "-Wextra"]


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    src = os.path.join(HERE, "fakref.c")
    tmp = LIB + ".tmp%d" % os.getpid()
    cmd = ["gcc", *CFLAGS, src, "-o", tmp, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
