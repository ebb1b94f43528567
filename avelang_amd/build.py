"""Build ``avelang_amd/libgdn.so`` (gfx950 only) from ``avelang_amd/csrc``.

    python -m avelang_amd.build            # or: python avelang_amd/build.py

One ``hipcc`` invocation compiles every ``csrc/*.hip`` for gfx950 into the
in-tree shared library that ``avelang_amd._native`` loads with ctypes.
Packed-fp32 VALU ops are disabled (``-packed-fp32-ops``) for every device
pass; hipcc's host pass prints a harmless "not a recognized feature" note.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libgdn.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in ordinary VGPRs: the kernels feed every accumulator to
    # VALU code, and AGPR results would each need a v_accvgpr_read first.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    return str(cand) if cand.exists() else "hipcc"


def sources():
    return sorted(str(p) for p in CSRC.glob("*.hip"))


def build(verbose: bool = False) -> Path:
    """Compile every HIP source into LIB (always recompiles)."""
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, *sources(), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
