"""Build the test-only HIP kernels under tests/hip/ into libtest_kernels.so
(gfx950), next to this file.  Test infrastructure: nothing in myelin_amd
loads it."""

from __future__ import annotations

import os
import pathlib
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
LIB = HERE / "libtest_kernels.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-shared", "-std=c++17", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def build() -> pathlib.Path:
    sources = sorted(str(p) for p in HERE.glob("*.hip"))
    tmp = LIB.with_suffix(".so.tmp")
    proc = subprocess.run([HIPCC, *FLAGS, *sources, "-o", str(tmp)], capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError("building tests/hip failed")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
