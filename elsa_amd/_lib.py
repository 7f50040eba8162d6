"""ctypes binding of libelsa_hip.so (the C ABI declared in include/elsa_hip.h).

The library is built in-tree by ``elsa_amd.build`` (``__graft_entry__.build()``).
There is no fallback: if the library is missing or fails to load, every call
raises ``RuntimeError``.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path
from typing import Optional

import torch

LIB_PATH = Path(__file__).resolve().parent / "libelsa_hip.so"
TORCH_MODULE_PATH = Path(__file__).resolve().parent / "_elsa_torch.so"

ELSA_F16, ELSA_BF16, ELSA_F32 = 0, 1, 2
ELSA_OK, ELSA_ERR_INVALID, ELSA_ERR_WORKSPACE, ELSA_ERR_LAUNCH, ELSA_ERR_UNSUPPORTED = 0, -1, -2, -3, -4

_DTYPE_CODE = {torch.float16: ELSA_F16, torch.bfloat16: ELSA_BF16, torch.float32: ELSA_F32}

EXPORTED_SYMBOLS = (
    "elsa_abi_version",
    "elsa_last_error",
    "elsa_struct_size",
    "elsa_fwd_plan_get",
    "elsa_fwd",
    "elsa_fwd_noalloc",
    "elsa_phase1",
    "elsa_phase2",
    "elsa_bwd_workspace_bytes",
    "elsa_bwd",
    "elsa_bwd_stage",
    "elsa_row_stats",
    "elsa_dbias",
    "elsa_dbias_workspace_bytes",
    "elsa_bwd_dbias",
    "elsa_bwd_dbias_workspace_bytes",
    "elsa_debug_mfma",
    "elsa_debug_mfma_rate",
)


class BiasDesc(ctypes.Structure):
    _fields_ = [
        ("ptr", c_void_p),
        ("dtype", c_int32),
        ("_pad", c_int32),
        ("stride_b", c_int64),
        ("stride_h", c_int64),
        ("stride_q", c_int64),
        ("stride_k", c_int64),
    ]


class Layout(ctypes.Structure):
    """elsa_layout: element strides (batch, head, row) of a [B,H,N,D] operand; zeros = dense."""

    _fields_ = [("batch", c_int64), ("head", c_int64), ("row", c_int64)]


def layout_of(t) -> "Layout":
    """Strides of a [B,H,N,D] tensor with a contiguous last dim, as an elsa_layout."""
    sb, sh, sn, sd = t.stride()
    assert sd == 1
    return Layout(sb, sh, sn)


class FwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", c_void_p),
        ("k", c_void_p),
        ("v", c_void_p),
        ("out", c_void_p),
        ("row_m", c_void_p),
        ("row_z", c_void_p),
        ("bias", BiasDesc),
        ("batch", c_int32),
        ("heads", c_int32),
        ("seq_len", c_int32),
        ("head_dim", c_int32),
        ("dtype", c_int32),
        ("summary_dtype", c_int32),
        ("is_causal", c_int32),
        ("partition_len", c_int32),
        ("q_chunk", c_int32),
        ("scale", c_float),
        ("workspace", c_void_p),
        ("workspace_bytes", c_size_t),
        ("q_layout", Layout),
        ("k_layout", Layout),
        ("v_layout", Layout),
        ("out_layout", Layout),
        ("exact_row_max", c_int32),
    ]


class FwdPlan(ctypes.Structure):
    _fields_ = [
        ("partitions", c_int32),
        ("partition_len", c_int32),
        ("q_chunk", c_int32),
        ("block_m", c_int32),
        ("key_tile", c_int32),
        ("_pad", c_int32),
        ("workspace_bytes", c_size_t),
    ]


class BwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", c_void_p),
        ("k", c_void_p),
        ("v", c_void_p),
        ("out", c_void_p),
        ("dout", c_void_p),
        ("row_m", c_void_p),
        ("row_z", c_void_p),
        ("dq", c_void_p),
        ("dk", c_void_p),
        ("dv", c_void_p),
        ("bias", BiasDesc),
        ("batch", c_int32),
        ("heads", c_int32),
        ("seq_len", c_int32),
        ("head_dim", c_int32),
        ("dtype", c_int32),
        ("is_causal", c_int32),
        ("scale", c_float),
        ("_pad", c_int32),
        ("workspace", c_void_p),
        ("workspace_bytes", c_size_t),
        ("q_layout", Layout),
        ("k_layout", Layout),
        ("v_layout", Layout),
        ("out_layout", Layout),
        ("dout_layout", Layout),
        ("dq_layout", Layout),
        ("dk_layout", Layout),
        ("dv_layout", Layout),
    ]


_STRUCTS = {0: FwdArgs, 1: FwdPlan, 2: BwdArgs, 3: BiasDesc, 4: Layout}
ABI_VERSION = 4
_lib: Optional[ctypes.CDLL] = None


def load() -> ctypes.CDLL:
    """Load libelsa_hip.so once; raise RuntimeError if it is missing or mismatched."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -m elsa_amd.build` (or __graft_entry__.build()) first"
        )
    lib = ctypes.CDLL(os.fspath(LIB_PATH))
    lib.elsa_abi_version.restype = c_int32
    lib.elsa_last_error.restype = ctypes.c_char_p
    lib.elsa_struct_size.restype = c_size_t
    lib.elsa_struct_size.argtypes = [c_int32]
    lib.elsa_fwd_plan_get.argtypes = [ctypes.POINTER(FwdArgs), ctypes.POINTER(FwdPlan)]
    lib.elsa_fwd.argtypes = [ctypes.POINTER(FwdArgs), c_void_p]
    lib.elsa_fwd_noalloc.argtypes = [ctypes.POINTER(FwdArgs), c_void_p]
    lib.elsa_phase1.argtypes = [ctypes.POINTER(FwdArgs), c_int32, c_int32, c_void_p]
    lib.elsa_phase2.argtypes = [ctypes.POINTER(FwdArgs), c_int32, c_int32, c_void_p]
    lib.elsa_bwd_workspace_bytes.restype = c_size_t
    lib.elsa_bwd_workspace_bytes.argtypes = [ctypes.POINTER(BwdArgs)]
    lib.elsa_bwd.argtypes = [ctypes.POINTER(BwdArgs), c_void_p]
    lib.elsa_bwd_stage.argtypes = [ctypes.POINTER(BwdArgs), c_int32, c_void_p]
    lib.elsa_row_stats.argtypes = [ctypes.POINTER(BwdArgs), c_void_p, c_void_p, c_void_p]
    lib.elsa_dbias.argtypes = [ctypes.POINTER(BwdArgs), c_void_p, c_int32, c_int32, c_void_p]
    lib.elsa_dbias_workspace_bytes.restype = c_size_t
    lib.elsa_dbias_workspace_bytes.argtypes = [ctypes.POINTER(BwdArgs), c_int32, c_int32]
    lib.elsa_bwd_dbias_workspace_bytes.restype = c_size_t
    lib.elsa_bwd_dbias_workspace_bytes.argtypes = [ctypes.POINTER(BwdArgs), c_int32, c_int32]
    lib.elsa_bwd_dbias.argtypes = [ctypes.POINTER(BwdArgs), c_void_p, c_int32, c_int32, c_void_p]
    lib.elsa_debug_mfma.argtypes = [c_int32, c_void_p, c_void_p, c_void_p, c_void_p]
    lib.elsa_debug_mfma_rate.argtypes = [c_int32, c_void_p, c_void_p, c_int32, c_int32, c_void_p]
    for fn in ("elsa_fwd_plan_get", "elsa_fwd", "elsa_fwd_noalloc", "elsa_phase1", "elsa_phase2", "elsa_bwd", "elsa_bwd_stage", "elsa_row_stats",
               "elsa_dbias", "elsa_bwd_dbias", "elsa_debug_mfma", "elsa_debug_mfma_rate"):
        getattr(lib, fn).restype = c_int32
    if lib.elsa_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH}: ABI version {lib.elsa_abi_version()} != {ABI_VERSION}")
    for which, st in _STRUCTS.items():
        if lib.elsa_struct_size(which) != ctypes.sizeof(st):
            raise RuntimeError(f"{LIB_PATH}: struct {st.__name__} size mismatch "
                               f"({lib.elsa_struct_size(which)} != {ctypes.sizeof(st)})")
    _lib = lib
    return lib


_torch_module = None


def torch_module():
    """The C++ autograd module (_elsa_torch.so, built by elsa_amd.build next to libelsa_hip.so).

    Loads libelsa_hip.so first, so both share that one copy of the library (its SONAME)."""
    global _torch_module
    if _torch_module is None:
        import importlib.util

        load()
        if not TORCH_MODULE_PATH.exists():
            raise RuntimeError(f"{TORCH_MODULE_PATH} is missing: run `python -m elsa_amd.build` (or "
                               "__graft_entry__.build()) to compile it")
        spec = importlib.util.spec_from_file_location("elsa_amd._elsa_torch", TORCH_MODULE_PATH)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        if mod.abi_version() != ABI_VERSION:
            raise RuntimeError(f"{TORCH_MODULE_PATH}: ABI version {mod.abi_version()} != {ABI_VERSION}")
        _torch_module = mod
    return _torch_module


def check(status: int, what: str) -> None:
    if status != ELSA_OK:
        msg = load().elsa_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {status}): {msg}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise ValueError("supported dtypes are fp16, bf16, and fp32") from None


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def bias_desc(view: Optional[torch.Tensor], strides=(0, 0, 0, 0)) -> BiasDesc:
    b = BiasDesc()
    if view is None:
        b.ptr = None
        b.dtype = ELSA_F32
        return b
    b.ptr = view.data_ptr()
    b.dtype = dtype_code(view.dtype)
    b.stride_b, b.stride_h, b.stride_q, b.stride_k = (int(s) for s in strides)
    return b
