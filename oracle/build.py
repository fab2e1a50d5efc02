"""Build the C part of the CPU oracle (test infrastructure only).

Compiles ``raster_ref.c`` twice (float and double arithmetic) with gcc into
``oracle/_build/liboracle.so``.  The reference's own rasterizer is CUDA
(gsplat/cuda/csrc/*.cu) and cannot be compiled in this image, so there is no
``oracle/_ref`` build.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
BUILD = HERE / "_build"
LIB = BUILD / "liboracle.so"


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    objs = []
    for real, suffix in (("float", "f32"), ("double", "f64")):
        obj = BUILD / f"raster_ref_{suffix}.o"
        cmd = ["gcc", "-O2", "-fPIC", "-std=c11", "-ffp-contract=off",
               f"-DREAL={real}", f"-DSUFFIX={suffix}", "-c", str(HERE / "raster_ref.c"),
               "-o", str(obj)]
        subprocess.run(cmd, check=True)
        objs.append(str(obj))
    tmp = LIB.with_suffix(".so.tmp")
    subprocess.run(["gcc", "-shared", "-o", str(tmp), *objs, "-lm"], check=True)
    tmp.replace(LIB)
    if verbose:
        print(f"[oracle.build] -> {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
