"""gcc recipe for the C oracle (TEST INFRASTRUCTURE ONLY).

    python oracle/build.py      ->  oracle/_build/libgdn_oracle.so

Built for x86-64-v3 (AVX2 + FMA) so the library built here also runs on the
GPU box's host CPU.  The reference repository has no gated-delta-rule source
to compile, so there is no ``oracle/_ref`` build.
"""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "gdn_cpu.c"
OUT = HERE / "_build" / "libgdn_oracle.so"
CFLAGS = ["-O3", "-march=x86-64-v3", "-fopenmp", "-fPIC", "-shared", "-std=c11",
          "-Wall", "-Wextra", "-Wno-unused-parameter"]


def build(verbose: bool = False) -> Path:
    OUT.parent.mkdir(exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    cmd = ["gcc", *CFLAGS, str(SRC), "-o", str(tmp), "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"gcc failed:\n{proc.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
