"""Helpers shared by the GPU parity tests (inputs are drawn on the CPU so every
device sees identical values; the oracle is the checker)."""
from __future__ import annotations

import numpy as np
import torch

TORCH_DT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}
# north-star parity bars versus the reference path (forward, gradients)
FWD_TOL = {"fp32": 1e-6, "fp16": 1e-3, "bf16": 1e-2}
GRAD_TOL = {"fp32": 1e-6, "fp16": 5e-5, "bf16": 5e-4}


def dev(x, dtype: str) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(np.asarray(x, dtype=np.float32))).to("cuda").to(TORCH_DT[dtype])


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def max_abs(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    assert a.shape == b.shape, (a.shape, b.shape)
    return float(np.abs(a - b).max()) if a.size else 0.0


def describe(msg: str) -> None:
    print(msg, flush=True)
