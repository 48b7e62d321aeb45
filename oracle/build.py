"""Build the oracle shared library (test infrastructure only).

    python oracle/build.py

gcc, -O3, -ffp-contract=off (the reference never contracts a*b+c; its NEON
fmas are written out as fmaf), OpenMP over independent rows.  -march is a
portable x86-64-v3 so the library built here also runs on the GPU box's host.
"""
from __future__ import annotations

import os
import platform
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"


def build() -> Path:
    march = ["-march=x86-64-v3"] if platform.machine() == "x86_64" else []
    tmp = LIB.with_suffix(".so.tmp")
    cmd = ["gcc", "-O3", *march, "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-fPIC", "-shared",
           "-std=c11", "-Wall", "-o", str(tmp), str(HERE / "oracle.c"), str(HERE / "head.c"), str(HERE / "attn.c"), "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
