"""Compile the sampler's HIP sources into ``vinfer_amd/libvsampler.so`` (gfx950 only).

Run as ``python -m vinfer_amd.csrc.build``. The build is in-tree so the library travels with
the source tree; there is no JIT cache.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parents[1]
ROOT = PKG.parent
LIB = PKG / "libvsampler.so"
SOURCES = [PKG / "csrc" / "capi.hip"]

# -ffp-contract=off: the penalty arithmetic rounds every operation on its own.
# -fhip-fp32-correctly-rounded-divide-sqrt: x / T is IEEE division, as on the CPU.
# -packed-fp32-ops is disabled for every kernel (no v_pk_*_f32 code).
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and Path(c).exists():
            return c
    raise RuntimeError("hipcc not found (ROCm is required to build the sampler library)")


def build(verbose: bool = False) -> Path:
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *FLAGS, f"-I{ROOT / 'include'}", "-o", str(tmp), *map(str, SOURCES)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        line
        for line in (proc.stdout + proc.stderr).splitlines()
        if "packed-fp32-ops" not in line  # the host pass does not know the feature: harmless
    )
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{out}")
    if verbose and out.strip():
        print(out)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(LIB)
