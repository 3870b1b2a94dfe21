"""Build recipe for the CPU oracle library (test infrastructure only).

    python oracle/build.py

compiles oracle/hc_oracle.c into oracle/lib/libhc_oracle.so with gcc.  The
reference's own path for this GEMM is Python (its NumPy simulator), so there
is no reference C source to compile into oracle/_ref.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "hc_oracle.c")
OUT_DIR = os.path.join(HERE, "lib")
OUT = os.path.join(OUT_DIR, "libhc_oracle.so")

# x86-64-v3 (AVX2) runs on both the build container and the GPU hosts; no
# fast-math and no contraction, so the C code rounds exactly as written.
CFLAGS = [
    "-O3",
    "-march=x86-64-v3",
    "-fno-fast-math",
    "-ffp-contract=off",
    "-fopenmp",
    "-fPIC",
    "-shared",
    "-std=c11",
    "-Wall",
]


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    tmp = OUT + ".tmp"
    cmd = ["gcc", *CFLAGS, SRC, "-o", tmp, "-lm"]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
