"""Build the oracle's C pieces (test infrastructure only): oracle/_build/liboracle.so.

gcc -O2 -ffp-contract=off keeps every floating-point step of the C
specification a separate IEEE operation (no fused multiply-add contraction
beyond the explicit fmaf calls).
"""
from __future__ import annotations

import glob
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "_build", "liboracle.so")


def build() -> str:
    srcs = sorted(glob.glob(os.path.join(HERE, "csrc", "*.c")))
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    cmd = ["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared",
           *srcs, "-lm", "-o", OUT + ".tmp"]
    subprocess.run(cmd, check=True)
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build())
