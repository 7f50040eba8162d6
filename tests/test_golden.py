"""The committed golden vectors (``tests/golden/*.npz``, written by
``tests/golden/make_fixtures.py``).

CPU: the fixtures' closed-form fields agree with PyTorch's math SDPA in float64 and its
autograd (an independent routine), the reference-rounding fields sit within the
reference's published error of it (README.md:31, 78-79), the seeded inputs regenerate
bit for bit, and the oracle still reproduces the stored outputs.
GPU: the HIP path on the stored inputs meets the parity bar against the stored
outputs.
"""
from __future__ import annotations

import glob
import json
import os

import numpy as np
import pytest
import torch

from oracle import elsa_oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FILES = sorted(glob.glob(os.path.join(GOLDEN, "*.npz")))
IDS = [os.path.basename(f)[:-4] for f in FILES]


def _load(path):
    with np.load(path, allow_pickle=False) as z:
        rec = {key: z[key] for key in z.files}
    rec["meta"] = json.loads(str(rec["meta"]))
    return rec


def _sdpa_fp64(rec):
    """out, dq, dk, dv and d(scores) from torch's math SDPA in float64 with autograd."""
    q, k, v, do = (torch.from_numpy(np.asarray(rec[x], np.float64)) for x in ("q", "k", "v", "dout"))
    q.requires_grad_(True)
    k.requires_grad_(True)
    v.requires_grad_(True)
    mask = None
    if "bias" in rec:
        mask = torch.from_numpy(np.asarray(rec["bias"], np.float64)).requires_grad_(True)
    out = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask,
                                                           is_causal=rec["meta"]["causal"])
    out.backward(do)
    grads = [t.grad.numpy() for t in (q, k, v)]
    db = mask.grad.numpy() if mask is not None else None
    return out.detach().numpy(), grads, db


def test_golden_files_present():
    assert len(FILES) == 6, FILES


@pytest.mark.parametrize("path", FILES, ids=IDS)
def test_inputs_regenerate_from_their_seed(path):
    rec = _load(path)
    meta = rec["meta"]
    q, k, v, do = O.make_inputs(tuple(meta["shape"]), seed=meta["seed"], dtype=meta["dtype"],
                                with_dout=True, dout_scale=meta["dout_scale"])
    for name, x in (("q", q), ("k", k), ("v", v), ("dout", do)):
        assert rec[name].dtype == x.dtype and np.array_equal(rec[name], x), name


@pytest.mark.parametrize("path", FILES, ids=IDS)
def test_closed_form_fields_match_math_sdpa(path):
    rec = _load(path)
    out, (dq, dk, dv), db = _sdpa_fp64(rec)
    tol = 1e-12 if rec["meta"]["dtype"] == "fp32" else 1e-6  # float64 / float32 storage of the fields
    for name, want in (("out_exact", out), ("dq_exact", dq), ("dk_exact", dk), ("dv_exact", dv)):
        np.testing.assert_allclose(rec[name], want, rtol=tol, atol=tol, err_msg=name)
    if db is not None:
        np.testing.assert_allclose(rec["dbias_exact"], db, rtol=tol, atol=tol)
    # base-2 row state: row_m = max(s * log2 e), row_z = sum 2^(s log2 e - row_m)
    meta = rec["meta"]
    b, h, n, d = meta["shape"]
    s = np.einsum("bhid,bhjd->bhij", rec["q"].astype(np.float64), rec["k"].astype(np.float64)) / np.sqrt(d)
    if "bias" in rec:
        s = s + rec["bias"].astype(np.float64)
    if meta["causal"]:
        s = np.where(np.tril(np.ones((n, n), bool)), s, -np.inf)
    s2 = (s * np.log2(np.e)).reshape(b * h, n, n)
    m = s2.max(-1)
    np.testing.assert_allclose(rec["row_m_exact"], m, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(rec["row_z_exact"], np.exp2(s2 - m[..., None]).sum(-1), rtol=1e-12)


# the reference's published error against math SDPA (README.md:31, 78-79): fp32 ~5e-7 forward,
# ~1e-7 gradients; fp16 ~4-5e-4 forward, ~1.5e-5 gradients.  Its gradient figures are measured
# with dO scaled by 0.1 (benchmarks/bwd_grad_correctness.py:24); these fixtures draw dO ~ N(0,1),
# so the gradient errors are ten times larger.  49-token windows and short causal rows sit above
# the long-sequence figures because each fp16 rounding of p / dS weighs more.
REF_ERR = {"fp32": (1e-6, 2e-6), "fp16": (2e-3, 1e-3), "bf16": (2e-2, 1e-2)}


@pytest.mark.parametrize("path", FILES, ids=IDS)
def test_reference_rounding_fields_within_published_error(path):
    rec = _load(path)
    fwd, grad = REF_ERR[rec["meta"]["dtype"]]
    assert np.abs(rec["out"] - rec["out_exact"]).max() <= fwd
    for g in ("dq", "dk", "dv"):
        assert np.abs(rec[g] - rec[g + "_exact"]).max() <= grad, g
    fin = np.isfinite(rec["row_m_exact"])
    assert np.abs(rec["row_m"][fin] - rec["row_m_exact"][fin]).max() <= 2e-3
    np.testing.assert_allclose(rec["row_z"], rec["row_z_exact"], rtol=5e-3)


@pytest.mark.parametrize("path", FILES, ids=IDS)
def test_oracle_reproduces_the_fixture(path):
    rec = _load(path)
    meta = rec["meta"]
    dt = meta["dtype"]
    bias = rec.get("bias")
    out, rm, rz = O.forward(rec["q"], rec["k"], rec["v"], bias=bias, is_causal=meta["causal"],
                            part_len=meta["part_len"], dtype=dt, mode="ref")
    dq, dk, dv = O.backward(rec["q"], rec["k"], rec["v"], out, rec["dout"], rm, rz, bias=bias,
                            is_causal=meta["causal"], dtype=dt, mode="ref")
    # BLAS summation order may move the last fp32 bit; the rounded output by at most one ulp
    one_ulp = np.spacing(np.abs(rec["out"]).astype(np.float16 if dt == "fp16" else np.float32))
    if dt == "bf16":
        one_ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(rec["out"]), 2.0 ** -126))) - 7)
    assert (np.abs(out - rec["out"]) <= one_ulp).all()
    for name, got in (("row_m", rm), ("row_z", rz), ("dq", dq), ("dk", dk), ("dv", dv)):
        np.testing.assert_allclose(got, rec[name], rtol=1e-5, atol=1e-7, err_msg=name)


@pytest.mark.gpu
@pytest.mark.parametrize("path", FILES, ids=IDS)
def test_hip_path_meets_the_bar_on_the_golden_vectors(path):
    import elsa_amd
    from tests.gpu_util import FWD_TOL, GRAD_TOL, assert_parity, describe, dev, host

    rec = _load(path)
    meta = rec["meta"]
    dt = meta["dtype"]
    describe(f"golden {os.path.basename(path)}")
    kw = dict(is_causal=meta["causal"], block_n=meta["part_len"])
    qt, kt, vt = (dev(rec[x], dt).requires_grad_(True) for x in ("q", "k", "v"))
    bt = None
    if "bias" in rec:
        bt = dev(rec["bias"], "fp32").requires_grad_(True)
        kw["bias"] = bt
    out = elsa_amd.twopass_attention_train(qt, kt, vt, **kw)
    out.backward(dev(rec["dout"], dt))
    with torch.no_grad():
        _, row_m, row_z = elsa_amd.twopass_attention_with_state(qt.detach(), kt.detach(), vt.detach(), **kw)
    torch.cuda.synchronize()
    describe(str(assert_parity(host(out), rec["out_exact"], rec["out"], FWD_TOL[dt], "out", dt)))
    for name, t in (("dq", qt), ("dk", kt), ("dv", vt)):
        describe(str(assert_parity(host(t.grad), rec[name + "_exact"], rec[name], GRAD_TOL[dt], name, dt)))
    fin = np.isfinite(rec["row_m_exact"])
    assert np.array_equal(np.isneginf(host(row_m)), np.isneginf(rec["row_m_exact"]))
    assert np.abs(host(row_m)[fin] - rec["row_m"][fin]).max() <= 1e-4 * max(1.0, np.abs(rec["row_m"][fin]).max())
    np.testing.assert_allclose(host(row_z), rec["row_z"], rtol=2e-3 if dt != "fp32" else 1e-5)
    if bt is not None:
        # each entry of this [B, H, N, N] bias is one (b, h) pair's dS: the gradient bar applies
        describe(str(assert_parity(host(bt.grad), rec["dbias_exact"], rec["dbias"], GRAD_TOL[dt], "dbias",
                                   "fp32")))
