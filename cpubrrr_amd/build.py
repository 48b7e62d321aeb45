"""Build the HIP library (libcpb_moe.so, gfx950) in-tree.

    python -m cpubrrr_amd.build          # or cpubrrr_amd.build.build()

Each translation unit is compiled with hipcc for gfx950 only, then linked into
cpubrrr_amd/libcpb_moe.so.  The oracle (test infrastructure) is built by
oracle/build.py, not here.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libcpb_moe.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # IEEE fp32: no a*b+c contraction, correctly rounded divide/sqrt
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    # packed fp32 VALU ops disabled (device code)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
    "-Wno-unused-command-line-argument",
]

SOURCES = ["route.hip", "moe_mx.hip", "moe_kq.hip", "moe_grouped.hip", "moe_grouped_kq.hip", "head.hip", "attn.hip", "api.hip"]
HOST_SOURCES = ["synth.cpp", "gguf.cpp"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l and "not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")


def build(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link libcpb_moe.so (always rebuilds)."""
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found")
    BUILD.mkdir(exist_ok=True)
    jobs = []
    for s in SOURCES:
        jobs.append([HIPCC, *COMMON, "-c", str(CSRC / s), "-o", str(BUILD / (s + ".o"))])
    for s in HOST_SOURCES:
        jobs.append(["g++", "-O3", "-std=c++17", "-fPIC", "-Wall", f"-I{ROOT / 'include'}", f"-I{CSRC}", "-c", str(CSRC / s),
                     "-o", str(BUILD / (s + ".o"))])
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        for f in [ex.submit(_run, j) for j in jobs]:
            f.result()
    objs = [str(BUILD / (s + ".o")) for s in SOURCES + HOST_SOURCES]
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objs, "-lpthread"])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
