"""CPU pins of the pure-PyTorch restatement (oracle/torch_scan.py) against the numpy
oracle (oracle/elsa_oracle.py), which tests/test_oracle.py and
tests/test_oracle_rounding.py pin against closed forms, finite differences and the
reference's rounding points.

fp64 mode and the closed forms must agree to float64 rounding.  In ``ref`` mode the two
restatements round at the same points but accumulate float32 sums in different orders,
so an fp16 rounding occasionally lands on the other side of a boundary: fp16 outputs are
bit-equal almost everywhere and at most a few ulps apart elsewhere, and the float32
gradients agree to float32 noise plus those flips.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import elsa_oracle as O
from oracle import torch_scan as T

CASES = [
    # shape, dtype, causal, part_len, micro, bias shape
    ((1, 2, 197, 64), "fp16", False, 64, 64, None),
    ((1, 2, 197, 64), "fp16", True, 128, 128, None),
    ((2, 2, 130, 32), "bf16", False, 64, 64, (2, 130, 130)),
    ((1, 2, 300, 64), "fp32", False, 128, 64, None),
    ((1, 2, 100, 64), "fp16", False, None, 64, None),
    ((1, 1, 77, 16), "fp32", True, 32, 32, (77, 77)),
    ((2, 1, 49, 32), "fp16", False, 49, 49, (2, 1, 49, 49)),
]


def _ids(c):
    return f"{c[0]}-{c[1]}-{'causal' if c[2] else 'full'}-p{c[3]}-bias{c[5] is not None}"


def _np(x):
    return x.numpy() if hasattr(x, "numpy") else np.asarray(x)


def _same_inf(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    assert np.array_equal(np.isneginf(a), np.isneginf(b))
    fin = np.isfinite(b)
    return a[fin], b[fin]


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_fp64_mode_equals_numpy_oracle(case):
    shape, dt, causal, part, micro, bshape = case
    q, k, v, do = O.make_inputs(shape, seed=sum(shape), dtype=dt, with_dout=True)
    bias = None if bshape is None else np.random.default_rng(1).standard_normal(bshape) * 0.5
    o1, m1, z1 = O.forward(q, k, v, bias=bias, is_causal=causal, part_len=part, micro=micro, dtype=dt, mode="fp64")
    o2, m2, z2 = T.forward(q, k, v, bias=bias, is_causal=causal, part_len=part, micro=micro, dtype=dt, mode="fp64",
                           row_chunk=61)
    np.testing.assert_allclose(_np(o2), o1, atol=1e-12)
    np.testing.assert_allclose(*_same_inf(_np(m2), m1), atol=1e-12)
    np.testing.assert_allclose(_np(z2), z1, rtol=1e-12)
    g1 = O.backward(q, k, v, o1, do, m1, z1, bias=bias, is_causal=causal, dtype=dt, mode="fp64")
    g2 = T.backward(q, k, v, o1, do, m1, z1, bias=bias, is_causal=causal, dtype=dt, mode="fp64", row_chunk=45)
    for a, b in zip(g2, g1):
        np.testing.assert_allclose(_np(a), b, atol=1e-12)


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_ref_mode_agrees_with_numpy_oracle(case):
    shape, dt, causal, part, micro, bshape = case
    q, k, v, do = O.make_inputs(shape, seed=sum(shape) + 1, dtype=dt, with_dout=True)
    bias = None if bshape is None else (np.random.default_rng(2).standard_normal(bshape) * 0.5).astype(np.float32)
    o1, m1, z1 = O.forward(q, k, v, bias=bias, is_causal=causal, part_len=part, micro=micro, dtype=dt, mode="ref")
    o2, m2, z2 = T.forward(q, k, v, bias=bias, is_causal=causal, part_len=part, micro=micro, dtype=dt, mode="ref")
    o1, o2 = np.asarray(o1, np.float64), _np(o2).astype(np.float64)
    if dt == "fp32":
        np.testing.assert_allclose(o2, o1, atol=2e-6 * np.abs(o1).max())
    else:
        # a flipped fp16/bf16 rounding of a partition summary moves out by that summary's ulp
        # over z, which at small |out| is several ulps of out: bound it by the largest output
        assert np.mean(o1 == o2) >= 0.97
        eps = 2.0 ** -10 if dt == "fp16" else 2.0 ** -7
        assert np.abs(o1 - o2).max() <= eps * np.abs(o1).max()
    a, b = _same_inf(_np(m2), m1)
    np.testing.assert_allclose(a, b, atol=1e-5)
    np.testing.assert_allclose(_np(z2), z1, rtol=1e-5)
    g1 = O.backward(q, k, v, o1, do, m1, z1, bias=bias, is_causal=causal, dtype=dt, mode="ref")
    g2 = T.backward(q, k, v, o1, do, m1, z1, bias=bias, is_causal=causal, dtype=dt, mode="ref", row_chunk=50)
    for a, b in zip(g2, g1):
        a, b = _np(a).astype(np.float64), np.asarray(b, np.float64)
        rms = np.sqrt(np.mean((a - b) ** 2)) / np.sqrt(np.mean(b ** 2))
        assert rms <= (1e-6 if dt == "fp32" else 2e-4), rms


@pytest.mark.parametrize("causal", [False, True])
def test_exact_forms_equal_numpy_closed_forms_on_row_and_key_subsets(causal):
    q, k, v, do = O.make_inputs((2, 2, 93, 16), seed=5, with_dout=True)
    bias = np.random.default_rng(5).standard_normal((2, 93, 93)) * 0.3
    eo, em, ez = O.exact_forward(q, k, v, bias=bias, is_causal=causal)
    eq, ek, ev, _ = O.exact_backward(q, k, v, do, bias=bias, is_causal=causal)
    rows = np.array([0, 5, 40, 92])
    keys = np.array([0, 1, 47, 92])
    to, tm, tz = T.exact_forward(q, k, v, bias=bias, is_causal=causal, rows=rows, row_chunk=3)
    np.testing.assert_allclose(_np(to), eo[:, :, rows], atol=1e-13)
    np.testing.assert_allclose(_np(tm), em[:, rows], atol=1e-13)
    np.testing.assert_allclose(_np(tz), ez[:, rows], rtol=1e-13)
    tq, tk, tv = T.exact_backward(q, k, v, do, bias=bias, is_causal=causal, rows=rows, keys=keys, row_chunk=17)
    np.testing.assert_allclose(_np(tq), eq[:, :, rows], atol=1e-13)
    np.testing.assert_allclose(_np(tk), ek[:, :, keys], atol=1e-13)
    np.testing.assert_allclose(_np(tv), ev[:, :, keys], atol=1e-13)


def test_backward_row_subset_is_the_row_restricted_recompute():
    q, k, v, do = O.make_inputs((1, 2, 140, 64), seed=8, dtype="fp16", with_dout=True)
    out, rm, rz = O.forward(q, k, v, part_len=64, dtype="fp16", mode="ref")
    rows = np.array([3, 64, 139])
    dq_all, _, _ = T.backward(q, k, v, out, do, rm, rz, dtype="fp16", row_chunk=32)
    dq_rows, dk, dv = T.backward(q, k, v, out, do, rm, rz, dtype="fp16", rows=rows, need_kv=False)
    assert dk is None and dv is None
    np.testing.assert_array_equal(_np(dq_rows), _np(dq_all)[:, :, rows])
    # the numpy oracle's row-restricted form gives the same rows
    rq, _, _ = O.backward(q[:, :, rows], k, v, out[:, :, rows], do[:, :, rows], rm[:, rows], rz[:, rows],
                          dtype="fp16", rows=rows)
    a, b = _np(dq_rows).astype(np.float64), np.asarray(rq, np.float64)
    assert np.sqrt(np.mean((a - b) ** 2)) / np.sqrt(np.mean(b ** 2)) <= 2e-4


def test_reference_routing_table():
    # attention.py:175-226 and attention_bwd.py:130-158
    assert O.reference_routing(16384, 64, "fp16") == (2048, 64)
    assert O.reference_routing(16384, 64, "fp16", training=True) == (256, 256)
    assert O.reference_routing(4096, 64, "fp16") == (256, 256)
    assert O.reference_routing(1025, 64, "fp32") == (1088, 64)
    assert O.reference_routing(300, 64, "fp32") == (256, 256)
    assert O.reference_routing(65536, 64, "fp32", training=True) == (2048, 64)
    assert O.reference_routing(8192, 64, "fp16", is_causal=True) == (2048, 2048)
    assert O.reference_routing(8192, 64, "fp16", training=True, is_causal=True) == (256, 256)
    assert O.reference_routing(197, 128, "bf16") == (64, 64)
    assert O.reference_routing(49, 32, "fp16", has_bias=True) == (256, 256)


@pytest.mark.parametrize("causal,bias", [(False, False), (True, True)])
def test_key_columns_are_the_full_backward_restricted(causal, bias):
    q, k, v, do = O.make_inputs((1, 2, 150, 64), seed=9, dtype="fp16", with_dout=True)
    b = (np.random.default_rng(9).standard_normal((2, 150, 150)) * 0.4).astype(np.float32) if bias else None
    out, rm, rz = T.forward(q, k, v, bias=b, is_causal=causal, part_len=64, dtype="fp16")
    _, dk, dv = T.backward(q, k, v, out, do, rm, rz, bias=b, is_causal=causal, dtype="fp16", row_chunk=40)
    keys = np.array([0, 63, 64, 149])
    kk, vv = T.backward_key_columns(q, k, v, out, do, rm, rz, keys, bias=b, is_causal=causal, dtype="fp16",
                                    row_chunk=33)
    np.testing.assert_allclose(_np(kk), _np(dk)[:, :, keys], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(_np(vv), _np(dv)[:, :, keys], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("causal", [False, True])
def test_fp32_summaries_agree_with_numpy_oracle(causal):
    """fp16 inputs with summary_dtype=fp32 (p @ v from the fp32 p in both restatements)."""
    q, k, v = O.make_inputs((1, 2, 197, 64), seed=91, dtype="fp16")
    o1, m1, z1 = O.forward(q, k, v, is_causal=causal, part_len=64, dtype="fp16", mode="ref", summary_dtype="fp32")
    o2, m2, z2 = T.forward(q, k, v, is_causal=causal, part_len=64, dtype="fp16", mode="ref", summary_dtype="fp32")
    o1, o2 = np.asarray(o1, np.float64), _np(o2).astype(np.float64)
    assert np.mean(o1 == o2) >= 0.99
    assert np.abs(o1 - o2).max() <= 2.0 ** -10 * np.abs(o1).max()
    np.testing.assert_allclose(*_same_inf(_np(m2), m1), atol=1e-5)
    np.testing.assert_allclose(_np(z2), z1, rtol=1e-5)
    # and both differ from the 16-bit-summary fold, whose p @ v rounds p
    o3, _, _ = T.forward(q, k, v, is_causal=causal, part_len=64, dtype="fp16", mode="ref", summary_dtype="fp16")
    assert np.mean(_np(o3).astype(np.float64) == o2) < 0.9
