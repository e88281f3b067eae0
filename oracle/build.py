"""Build recipe for the CPU oracle (test infrastructure; see oracle.c's header).

Compiles oracle.c into oracle/_build/liboracle.so.  x86-64-v3 (AVX2 + FMA) keeps the
library runnable on the GPU box's host CPU, which need not match this machine's.
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "liboracle.so")


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    cmd = [
        "gcc", "-O3", "-march=x86-64-v3", "-ffp-contract=off", "-fno-fast-math",
        "-fopenmp", "-shared", "-fPIC", "-o", LIB + ".tmp",
        os.path.join(HERE, "oracle.c"), "-lm",
    ]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
