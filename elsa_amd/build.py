"""Build libelsa_hip.so (gfx950) in-tree with hipcc, and the C++ autograd module.

``python -m elsa_amd.build`` or ``elsa_amd.build.build_library()``.  Objects are
compiled in parallel and linked into ``elsa_amd/libelsa_hip.so``;
``build_torch_module()`` then compiles ``csrc/elsa_torch.cpp`` (host C++ against
PyTorch's headers, linked to libelsa_hip.so) into ``elsa_amd/_elsa_torch.so``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libelsa_hip.so"
TORCH_MODULE = PKG / "_elsa_torch.so"
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
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-soname,libelsa_hip.so", "-o", str(tmp),
            *map(str, objs)]
    _run(link)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", flush=True)
    return LIB


def build_torch_module(verbose: bool = False) -> Path:
    """Compile csrc/elsa_torch.cpp into elsa_amd/_elsa_torch.so (host code: g++ with PyTorch's
    include paths, C++ ABI flag and libraries, plus ROCm's headers for the HIP stream API).
    It links libelsa_hip.so from its own directory (rpath $ORIGIN)."""
    import torch
    import torch.utils.cpp_extension as ce

    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared",
        "-DTORCH_EXTENSION_NAME=_elsa_torch", "-DTORCH_API_INCLUDE_EXTENSION_H",
        # ROCm's HIP headers select the AMD platform by this macro when a host compiler reads them
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
        *(f"-I{p}" for p in ce.include_paths()),
        f"-I{sysconfig.get_paths()['include']}", "-I/opt/rocm/include", "-I", str(ROOT / "include"),
        str(CSRC / "elsa_torch.cpp"), "-o", str(TORCH_MODULE.with_suffix(".so.tmp")),
        f"-L{torch_lib}", "-lc10", "-ltorch_cpu", "-ltorch", "-ltorch_python", "-lc10_hip", "-ltorch_hip",
        f"-L{PKG}", "-lelsa_hip", "-Wl,-rpath,$ORIGIN",
    ]
    _run(cmd)
    os.replace(TORCH_MODULE.with_suffix(".so.tmp"), TORCH_MODULE)
    if verbose:
        print(f"built {TORCH_MODULE}", flush=True)
    return TORCH_MODULE


if __name__ == "__main__":
    build_library(verbose="-q" not in sys.argv)
    build_torch_module(verbose="-q" not in sys.argv)
