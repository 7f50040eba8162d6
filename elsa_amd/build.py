"""Build libelsa_hip.so (gfx950) in-tree with hipcc.

``python -m elsa_amd.build`` or ``elsa_amd.build.build_library()``.  Objects are
compiled in parallel and linked into ``elsa_amd/libelsa_hip.so``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libelsa_hip.so"
SOURCES = ("elsa_fwd.hip", "elsa_bwd.hip", "elsa_api.hip")
ARCH = "gfx950"

# Packed fp32 VALU forms are disabled for all device code (only scalar / packed-16-bit VALU).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # scores and p are never NaN by construction (masking uses -inf), so min/max
    # need no NaN-quieting canonicalisation of their inputs
    "-fno-honor-nans",
    "-Wno-unused-result",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libelsa_hip.so)")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    lines = [ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln]
    if proc.returncode != 0:
        raise RuntimeError("command failed: " + " ".join(cmd) + "\n" + "\n".join(lines))


def build_library(verbose: bool = False) -> Path:
    hipcc = _hipcc()
    obj_dir = ROOT / "_build"
    obj_dir.mkdir(exist_ok=True)
    inc = ["-I", str(ROOT / "include"), "-I", str(CSRC)]
    objs = []
    cmds = []
    for src in SOURCES:
        obj = obj_dir / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([hipcc, *HIP_FLAGS, *inc, "-c", str(CSRC / src), "-o", str(obj)])
    with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        for cmd, _ in zip(cmds, ex.map(_run, cmds)):
            if verbose:
                print(" ".join(cmd), flush=True)
    tmp = LIB.with_suffix(".so.tmp")
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    _run(link)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", flush=True)
    return LIB


if __name__ == "__main__":
    build_library(verbose="-q" not in sys.argv)
