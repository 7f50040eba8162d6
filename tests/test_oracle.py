"""CPU checks that pin the oracle (the numpy restatement) before it is trusted.

The reference ships no golden vectors (its tests compare against SDPA at run time,
reference tests/test_attention.py:16-25), so the oracle is pinned by: independent fp64
closed forms, the reference's published error magnitudes (README.md:31, 78-79), monoid
laws, partition/merge-order invariance, finite differences and brute force on tiny
inputs.  Each check is chosen so that a plausible slip in the restatement (a dropped
alpha/beta, a wrong log2e, a transposed operand, an unguarded -inf) fails one of them.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

from oracle import elsa_oracle as O


def _rand_summary(rng, rows, d, empty_frac=0.2):
    m = rng.standard_normal(rows) * 4
    z = rng.uniform(0.5, 20, rows)
    s = rng.standard_normal((rows, d)) * z[:, None]
    empty = rng.uniform(size=rows) < empty_frac
    m = np.where(empty, -np.inf, m)
    z = np.where(empty, 0.0, z)
    s = np.where(empty[:, None], 0.0, s)
    return m, z, s


def _close(a, b, tol=1e-12):
    for x, y in zip(a, b):
        assert np.array_equal(np.isneginf(x), np.isneginf(y))
        xf = np.where(np.isneginf(x), 0, x)
        yf = np.where(np.isneginf(y), 0, y)
        np.testing.assert_allclose(xf, yf, rtol=tol, atol=tol)


# ----------------------------------------------------------------------- monoid
@settings(max_examples=60, deadline=None)
@given(seed=st.integers(0, 2**31 - 1), rows=st.integers(1, 9), d=st.sampled_from([1, 4, 8]))
def test_merge_associative(seed, rows, d):
    rng = np.random.default_rng(seed)
    a, b, c = (_rand_summary(rng, rows, d) for _ in range(3))
    left = O.merge(O.merge(a, b), c)
    right = O.merge(a, O.merge(b, c))
    # compare the represented quantities s/z and log2(z)+m (the canonical form)
    _close(O.finalize(left), O.finalize(right), 1e-12)


@settings(max_examples=40, deadline=None)
@given(seed=st.integers(0, 2**31 - 1), rows=st.integers(1, 9))
def test_identity_is_neutral(seed, rows):
    rng = np.random.default_rng(seed)
    a = _rand_summary(rng, rows, 4)
    e = O.identity((rows,), 4)
    _close(O.merge(e, a), a)
    _close(O.merge(a, e), a)
    # identity with itself stays the identity (no NaN from -inf - -inf)
    m, z, s = O.merge(e, e)
    assert np.all(np.isneginf(m)) and np.all(z == 0) and np.all(s == 0)


def test_merge_matches_direct_softmax_sum():
    # merging the summaries of two key sets equals the summary of their union
    rng = np.random.default_rng(7)
    x = rng.standard_normal(37) * 3
    vals = rng.standard_normal((37, 5))

    def summ(idx):
        m = x[idx].max()
        w = np.exp2(x[idx] - m)
        return np.array([m]), np.array([w.sum()]), (w[:, None] * vals[idx]).sum(0)[None]

    a, b = summ(np.arange(0, 20)), summ(np.arange(20, 37))
    _close(O.merge(a, b), summ(np.arange(37)), 1e-12)


@pytest.mark.parametrize("p", [1, 2, 3, 5, 8, 13])
def test_tree_flat_scan_agree(p):
    rng = np.random.default_rng(p)
    parts = [_rand_summary(rng, 6, 3) for _ in range(p)]
    tree = O.merge_tree(parts)
    flat = O.merge_flat(parts)
    scan = O.scan_hillis_steele(parts)
    _close(O.finalize(tree), O.finalize(flat), 1e-12)
    _close(O.finalize(scan[-1]), O.finalize(flat), 1e-12)
    # every inclusive prefix equals the sequential fold of its prefix
    acc = parts[0]
    _close(O.finalize(scan[0]), O.finalize(acc), 1e-12)
    for j in range(1, p):
        acc = O.merge(acc, parts[j])
        _close(O.finalize(scan[j]), O.finalize(acc), 1e-12)


# ----------------------------------------------------------------------- forward
@pytest.mark.parametrize("n", [1, 5, 64, 97, 197])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("part_len", [64, 128, 100000])
def test_fp64_forward_equals_closed_form(n, causal, part_len):
    q, k, v = O.make_inputs((1, 2, n, 16), seed=n)
    for kind in ("tree", "flat", "scan"):
        out, rm, rz = O.forward(q, k, v, is_causal=causal, part_len=part_len, mode="fp64", merge_kind=kind)
        eo, em, ez = O.exact_forward(q, k, v, is_causal=causal)
        np.testing.assert_allclose(out, eo, rtol=0, atol=1e-12)
        np.testing.assert_allclose(rm, em, rtol=0, atol=1e-12)
        np.testing.assert_allclose(rz, ez, rtol=1e-12, atol=0)


def test_fp64_forward_bias_and_micro_tile():
    q, k, v = O.make_inputs((2, 3, 49, 32), seed=3)
    bias = np.random.default_rng(3).standard_normal((1, 3, 49, 49)) * 0.5
    for micro in (16, 64):
        out, rm, rz = O.forward(q, k, v, bias=bias, part_len=32, micro=micro, mode="fp64")
        eo, em, ez = O.exact_forward(q, k, v, bias=bias)
        np.testing.assert_allclose(out, eo, atol=1e-12)
        np.testing.assert_allclose(rm, em, atol=1e-12)
        np.testing.assert_allclose(rz, ez, rtol=1e-12)


def test_fully_masked_rows_give_zero_and_identity_state():
    # a -inf bias row masks every key of that row: out=0, row_m=-inf, row_z=0
    # (attention_parallel_scan.py:410, paper_scan_d64_kernel.cu:73-74, :93)
    q, k, v = O.make_inputs((1, 1, 10, 8), seed=1)
    bias = np.zeros((10, 10))
    bias[3, :] = -np.inf
    out, rm, rz = O.forward(q, k, v, bias=bias, part_len=4, mode="fp64")
    assert np.all(out[0, 0, 3] == 0) and np.isneginf(rm[0, 3]) and rz[0, 3] == 0
    eo, _, _ = O.exact_forward(q, k, v, bias=bias)
    np.testing.assert_allclose(out, eo, atol=1e-12)


def test_state_is_base2():
    # row_m = max(s*log2e) and row_z = sum exp2(s*log2e - row_m) (attention_bwd.py:224)
    q, k, v = O.make_inputs((1, 1, 7, 4), seed=2)
    _, rm, rz = O.forward(q, k, v, mode="fp64")
    s = (q[0, 0].astype(np.float64) @ k[0, 0].T.astype(np.float64)) / 2.0
    np.testing.assert_allclose(rm[0], s.max(1) * O.LOG2E, atol=1e-13)
    np.testing.assert_allclose(rz[0], np.exp2(s * O.LOG2E - (s.max(1) * O.LOG2E)[:, None]).sum(1), rtol=1e-13)


@pytest.mark.parametrize("dtype,tol", [("fp32", 2e-6), ("fp16", 2e-3), ("bf16", 2e-2)])
@pytest.mark.parametrize("n,causal", [(197, False), (256, False), (129, True)])
def test_ref_rounding_mode_error_matches_published_magnitude(dtype, tol, n, causal):
    # README.md:31,78: fp32 error ~5e-7, fp16 ~4e-4..5e-4 versus math SDPA
    q, k, v = O.make_inputs((1, 2, n, 64), seed=11, dtype=dtype)
    out, rm, rz = O.forward(q, k, v, is_causal=causal, part_len=64, dtype=dtype, mode="ref")
    eo, em, ez = O.exact_forward(np.asarray(q, np.float32), np.asarray(k, np.float32), np.asarray(v, np.float32),
                                 is_causal=causal)
    err = np.abs(out.astype(np.float64) - eo).max()
    assert err < tol, err
    assert err > 0  # the ref mode really rounds
    np.testing.assert_allclose(rm, em, atol=tol * 8)


def test_round_helpers():
    x = np.array([1.0, 1.0 + 2**-11, 1.0 + 3 * 2**-11, 65504.0, 1e-8], np.float32)
    np.testing.assert_array_equal(O.round_fp16(x), x.astype(np.float16).astype(np.float32))
    b = O.round_bf16(np.array([1.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8, -2.5], np.float32))
    np.testing.assert_array_equal(b, np.array([1.0, 1.0, 1.0 + 2**-6, -2.5], np.float32))


# ----------------------------------------------------------------------- backward
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("with_bias", [False, True])
def test_fp64_backward_equals_closed_form(causal, with_bias):
    q, k, v, do = O.make_inputs((1, 2, 33, 16), seed=5, with_dout=True)
    bias = np.random.default_rng(5).standard_normal((2, 33, 33)) * 0.3 if with_bias else None
    out, rm, rz = O.forward(q, k, v, bias=bias, is_causal=causal, part_len=16, mode="fp64")
    dq, dk, dv = O.backward(q, k, v, out, do, rm, rz, bias=bias, is_causal=causal, mode="fp64")
    eq, ek, ev, _ = O.exact_backward(q, k, v, do, bias=bias, is_causal=causal)
    np.testing.assert_allclose(dq, eq, atol=1e-12)
    np.testing.assert_allclose(dk, ek, atol=1e-12)
    np.testing.assert_allclose(dv, ev, atol=1e-12)


def test_closed_form_backward_matches_finite_differences():
    q, k, v, do = O.make_inputs((1, 1, 6, 4), seed=9, with_dout=True)
    q, k, v, do = (x.astype(np.float64) for x in (q, k, v, do))
    bias = np.random.default_rng(9).standard_normal((6, 6)) * 0.4
    eq, ek, ev, ds = O.exact_backward(q, k, v, do, bias=bias, is_causal=True)
    h = 1e-6

    def loss(qq, kk, vv, bb):
        return float((O.exact_forward(qq, kk, vv, bias=bb, is_causal=True)[0] * do).sum())

    for name, arr, grad in (("q", q, eq), ("k", k, ek), ("v", v, ev)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            a1, a2 = arr.copy(), arr.copy()
            a1[idx] += h
            a2[idx] -= h
            args = {"q": (a1, k, v), "k": (q, a1, v), "v": (q, k, a1)}[name]
            args2 = {"q": (a2, k, v), "k": (q, a2, v), "v": (q, k, a2)}[name]
            num[idx] = (loss(*args, bias) - loss(*args2, bias)) / (2 * h)
        np.testing.assert_allclose(grad, num, atol=1e-7)
    # dbias = dscores summed over broadcast dims
    numb = np.zeros_like(bias)
    for idx in np.ndindex(bias.shape):
        b1, b2 = bias.copy(), bias.copy()
        b1[idx] += h
        b2[idx] -= h
        numb[idx] = (loss(q, k, v, b1) - loss(q, k, v, b2)) / (2 * h)
    out, rm, rz = O.exact_forward(q, k, v, bias=bias, is_causal=True)
    db = O.dbias(q, k, v, out, do, rm, rz, bias=bias, is_causal=True)
    np.testing.assert_allclose(db, numb, atol=1e-7)


@pytest.mark.parametrize("shape", [(2, 3, 9, 9), (1, 3, 9, 9), (2, 1, 9, 9), (1, 1, 9, 9), (3, 9, 9), (9, 9)])
def test_dbias_broadcast_reduction(shape):
    q, k, v, do = O.make_inputs((2, 3, 9, 8), seed=4, with_dout=True)
    bias = np.random.default_rng(4).standard_normal(shape) * 0.2
    out, rm, rz = O.exact_forward(q, k, v, bias=bias)
    db = O.dbias(q, k, v, out, do, rm, rz, bias=bias)
    assert db.shape == tuple(shape)
    _, _, _, ds = O.exact_backward(q, k, v, do, bias=bias)
    full = ds
    if len(shape) == 4:
        if shape[0] == 1:
            full = full.sum(0, keepdims=True)
        if shape[1] == 1:
            full = full.sum(1, keepdims=True)
    elif len(shape) == 3:
        full = full.sum(0)
    else:
        full = full.sum((0, 1))
    np.testing.assert_allclose(db, full, atol=1e-12)


@pytest.mark.parametrize("dtype,tol", [("fp32", 1e-5), ("fp16", 2e-3)])
def test_ref_backward_error_magnitude(dtype, tol):
    # README.md:79 gradient error fp32 ~1e-7, fp16 ~1.5e-5 (with their dO scaling)
    q, k, v, do = O.make_inputs((1, 2, 128, 64), seed=2026, dtype=dtype, with_dout=True, dout_scale=0.1)
    out, rm, rz = O.forward(q, k, v, part_len=64, dtype=dtype, mode="ref")
    dq, dk, dv = O.backward(q, k, v, out, do, rm, rz, dtype=dtype, mode="ref")
    eq, ek, ev, _ = O.exact_backward(*(np.asarray(x, np.float32) for x in (q, k, v, do)))
    for a, b in ((dq, eq), (dk, ek), (dv, ev)):
        err = np.abs(a - b).max()
        assert err < tol, err


def test_row_stats_matches_forward_state():
    q, k, v = O.make_inputs((1, 2, 40, 8), seed=8)
    m, z = O.row_stats(q, k, is_causal=True)
    _, em, ez = O.exact_forward(q, k, v, is_causal=True)
    np.testing.assert_allclose(m, em, atol=1e-12)
    np.testing.assert_allclose(z, ez, rtol=1e-12)


def test_canonical_bias_errors():
    with pytest.raises(ValueError, match="last dims"):
        O.canonical_bias(np.zeros((3, 4)), 1, 1, 3)
    with pytest.raises(ValueError, match="3D bias"):
        O.canonical_bias(np.zeros((2, 3, 3)), 1, 3, 3)
    with pytest.raises(ValueError, match="4D bias"):
        O.canonical_bias(np.zeros((2, 2, 3, 3)), 3, 2, 3)


@pytest.mark.parametrize("shape", [(2, 3, 9, 9), (1, 3, 9, 9), (2, 1, 9, 9), (3, 9, 9), (9, 9)])
@pytest.mark.parametrize("causal", [False, True])
def test_dbias_ref_mode_is_the_fp32_evaluation(shape, causal):
    """dbias in the reference kernel's float32 arithmetic (attention_bwd.py:596-614) is the float64
    form up to float32 rounding, on every broadcast rank; its float32 evaluation shows (it is not
    the float64 value rounded once)."""
    q, k, v, do = O.make_inputs((2, 3, 9, 8), seed=40, with_dout=True)
    bias = (np.random.default_rng(40).standard_normal(shape) * 0.3).astype(np.float32)
    out, rm, rz = O.exact_forward(q, k, v, bias=bias, is_causal=causal)
    exact = O.dbias(q, k, v, out, do, rm, rz, bias=bias, is_causal=causal)
    ref = O.dbias(q, k, v, out, do, rm, rz, bias=bias, is_causal=causal, mode="ref")
    assert ref.dtype == np.float32 and ref.shape == exact.shape
    err = np.abs(ref - exact).max()
    assert err <= 2e-6 * max(1.0, np.abs(exact).max()), err
    assert err > np.abs(exact.astype(np.float32) - exact).max()


def test_tf32x3_dot_drops_only_the_tail_product():
    """matmul_tf32x3 against its definition on single products: exact when one operand is a TF32
    value (its tail is zero), and off by exactly the dropped tail*tail term otherwise; its error
    on a random dot sits near 2^-22 relative, between TF32 (2^-11) and fp32 (2^-24)."""
    rng = np.random.default_rng(3)
    a = rng.standard_normal((5, 7)).astype(np.float32)
    b = rng.standard_normal((7, 4)).astype(np.float32)
    np.testing.assert_array_equal(O.matmul_tf32x3(O.round_tf32(a), O.round_tf32(b)),
                                  (O.round_tf32(a).astype(np.float64) @ O.round_tf32(b).astype(np.float64))
                                  .astype(np.float32))
    x = np.float32(1.0 + 2 ** -12 + 2 ** -20)  # head 1, tail 2^-12 + 2^-20 (both TF32-exact)
    hx = O.round_tf32(np.array([x]))[0]
    assert hx == np.float32(1.0)
    got = O.matmul_tf32x3(np.array([[x]]), np.array([[x]]))[0, 0]
    tail = float(x) - 1.0
    assert got == np.float32(float(x) * float(x) - tail * tail)
    assert O.round_tf32(np.array([1.0 + 2 ** -11], np.float32))[0] == np.float32(1.0 + 2 ** -10)  # ties away
    big_a = rng.standard_normal((64, 256)).astype(np.float32)
    big_b = rng.standard_normal((256, 64)).astype(np.float32)
    exact = big_a.astype(np.float64) @ big_b.astype(np.float64)
    rel = np.abs(O.matmul_tf32x3(big_a, big_b) - exact).max() / np.abs(exact).max()
    assert 2 ** -26 < rel < 2 ** -19, rel
