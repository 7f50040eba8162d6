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


def assert_parity(got, exact, ref, tol: float, what: str = "") -> dict:
    """The parity bar of this build.

    ``ref`` is the oracle at the reference's rounding points (the stand-in for the
    reference's own output), ``exact`` the fp64 closed form.  Asserts
      1. max|got - ref| <= tol                      (the north-star bar versus the reference path);
      2. max|got - exact| <= max(tol, 1.25 * max|ref - exact|)
         (never less accurate than the reference beyond the bar: on short causal rows
         and 49-token windows the reference's own fp16 rounding of p / dS / out already
         exceeds the bar against the exact value).
    """
    got = np.asarray(got, np.float64)
    e_ref = max_abs(ref, exact)
    d_ref = max_abs(got, ref)
    e_got = max_abs(got, exact)
    info = {"vs_ref": d_ref, "vs_exact": e_got, "ref_vs_exact": e_ref}
    assert d_ref <= tol, (what, info)
    assert e_got <= max(tol, 1.25 * e_ref), (what, info)
    return info
