"""Build ``myelin_amd/libmyelin_hip.so`` from ``myelin_amd/csrc/*.hip`` for gfx950.

Run ``python -m myelin_amd.build``.  Every source is compiled with hipcc
(``--offload-arch=gfx950``) into ``myelin_amd/_build/`` and linked into one
shared library next to this file.  Extra ``-D`` defines (kernel tuning
knobs) can be passed with ``MYELIN_HIPCC_DEFINES="-DNAME=VALUE ..."`` and the
output path with ``MYELIN_LIB_OUT``.
"""

from __future__ import annotations

import os
import pathlib
import shlex
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = pathlib.Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libmyelin_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-fPIC",
    "-std=c++17",
    # every multiply and add rounded separately, like the separate ATen ops
    "-ffp-contract=off",
    # no packed-FP32 instructions in generated code
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-result",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}")
    noise = "packed-fp32-ops"
    for line in (proc.stdout + proc.stderr).splitlines():
        if line.strip() and noise not in line and "warning: argument unused" not in line:
            sys.stderr.write(line + "\n")


def build(out: pathlib.Path | None = None, defines: list[str] | None = None) -> pathlib.Path:
    out = pathlib.Path(os.environ.get("MYELIN_LIB_OUT", out or LIB))
    defines = list(defines or []) + shlex.split(os.environ.get("MYELIN_HIPCC_DEFINES", ""))
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    tag = out.stem
    objs = [BUILD / f"{tag}.{src.stem}.o" for src in sources]
    jobs = [
        [HIPCC, *FLAGS, *defines, "-c", str(src), "-o", str(obj)]
        for src, obj in zip(sources, objs)
    ]
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as pool:
        list(pool.map(_run, jobs))
    tmp = out.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build())
