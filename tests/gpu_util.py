"""Helpers shared by the GPU parity tests (inputs are drawn on the CPU so every
device sees identical values; the oracle is the checker)."""
from __future__ import annotations

import json
import os

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


def ulp(x, dtype: str) -> np.ndarray:
    """Spacing of the output dtype at |x| (elementwise)."""
    a = np.abs(np.asarray(x, np.float64))
    if dtype == "fp16":
        return np.spacing(a.astype(np.float16)).astype(np.float64)
    if dtype == "bf16":
        e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
        return 2.0 ** (e - 7)
    return np.spacing(a.astype(np.float32)).astype(np.float64)


def parity_record(rec: dict) -> None:
    """Append one parity record (a JSON line) to $ELSA_PARITY_LOG when that is set."""
    path = os.environ.get("ELSA_PARITY_LOG")
    if not path:
        return
    # PYTEST_CURRENT_TEST is "<node id> (<phase>)"; node ids can hold spaces
    rec = dict(rec, test=os.environ.get("PYTEST_CURRENT_TEST", "").rsplit(" (", 1)[0])
    with open(path, "a") as f:
        f.write(json.dumps(rec) + "\n")


# Factor on the reference's own error in the bar against the exact value: a different but
# equally accurate evaluation lands within about that multiple of it.  16-bit outputs keep
# 1.25; fp32 gradients of order 1 and fp32 dbias sums (two float32 summation orders, each a
# few ulps of 1e-6 scale) take 2.
EXACT_FACTOR = {"fp16": 1.25, "bf16": 1.25, "fp32": 2.0}


def assert_parity(got, exact, ref, tol: float, what: str = "", dtype: str = "fp16", plain: bool = False) -> dict:
    """The parity bar of this build.

    ``ref`` is the oracle at the reference's rounding points (the stand-in for the
    reference's own output), ``exact`` the fp64 closed form, ``dtype`` the storage
    type of ``got``.  An output stored in ``dtype`` cannot agree with another one
    better than one ulp of that format, so the bar is applied beyond it:
      1. max(|got - ref| - ulp(ref)) <= max(tol, 2 * e_ref)   (the north-star bar versus the
         reference path; e_ref = max|ref - exact| is the reference's own error, and where
         it exceeds tol/2 two independent roundings can differ by up to twice it);
      2. max(|got - exact| - ulp(exact)/2) <= max(tol, EXACT_FACTOR[dtype] * e_ref)
         (in the reference's accuracy class beyond the bar: on short causal rows and
         49-token windows the reference's own fp16 rounding of p / dS / out already exceeds
         the bar against the exact value).
    ``plain=True`` applies the north-star bar alone (tol, with no e_ref term) to both.
    The returned dict says under "bound" whether the plain bar held for both criteria
    ("plain") or the e_ref term was needed ("e_ref").
    """
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    exact = np.asarray(exact, np.float64)
    assert got.shape == ref.shape == exact.shape
    e_ref = max_abs(ref, exact)
    d_ref = float((np.abs(got - ref) - ulp(ref, dtype)).max()) if got.size else 0.0
    e_got = float((np.abs(got - exact) - 0.5 * ulp(exact, dtype)).max()) if got.size else 0.0
    bar_ref = tol if plain else max(tol, 2.0 * e_ref)
    bar_exact = tol if plain else max(tol, EXACT_FACTOR[dtype] * e_ref)
    info = {"vs_ref_beyond_ulp": d_ref, "vs_exact_beyond_half_ulp": e_got, "ref_vs_exact": e_ref,
            "vs_ref_raw": max_abs(got, ref), "tol": tol,
            "bound": "plain" if (d_ref <= tol and e_got <= tol) else "e_ref"}
    parity_record(dict(info, what=what, dtype=dtype, plain=plain, n=int(got.size)))
    assert d_ref <= bar_ref, (what, info)
    assert e_got <= bar_exact, (what, info)
    return info
