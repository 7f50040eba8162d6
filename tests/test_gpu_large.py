"""GPU parity at BASELINE.json's own configurations, with the upstream gradient dO ~ N(0,1).

Each case runs the benchmarked calls (``twopass_attention_with_state`` then
``twopass_attention_backward``, or ``twopass_attention`` for the inference forward) at the
configuration's full size, and checks what the CPU can afford to restate:

* full tensors (every row, every head) where that is seconds of CPU work: B1 H8 at 1K-4K,
  causal 2K and 4097, and the reference's own gradient-check shapes B8 H3 N in
  {1025, 2305, 4097} and B1 H8 N4096 (benchmarks/bwd_grad_correctness.py:11-16,
  scripts/spot_check.py:39-51);
* at 8K-64K: sampled query rows of every head (out, row state, dq), and either two full
  heads (dq, dk, dv, at 8K-16K) or sampled key columns of one head's dk/dv (32K-64K).

The reference-rounded values come from oracle/torch_scan.py (the pure-PyTorch restatement,
pinned against the numpy oracle) laid out as the reference lays out that call
(``reference_routing``), and the exact values from its float64 closed forms.  The bar is
tests/gpu_util.py's ``assert_parity`` (forward 1e-3 fp16 / 1e-6 fp32,
gradients 5e-5 fp16 / 1e-6 fp32, relaxed only where the reference's own rounding exceeds
them); every check prints its raw max_abs.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import elsa_amd
from elsa_amd.attention import forward_plan
from oracle import elsa_oracle as O
from oracle import torch_scan as T
from tests.gpu_util import FWD_TOL, GRAD_TOL, TORCH_DT, assert_parity, describe

pytestmark = pytest.mark.gpu


def _draw(shape, dt, seed):
    """q, k, v, dO ~ N(0,1) from one CPU generator, in that order, cast to dt."""
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(shape, generator=g).to(TORCH_DT[dt]) for _ in range(4)]


def _rows(n, count, seed, extra=()):
    rng = np.random.default_rng(seed)
    pick = set(rng.choice(n, min(n, count), replace=False).tolist()) | {0, 1, n - 1}
    pick |= {r for r in extra if 0 <= r < n}
    return np.array(sorted(pick))


def _train_on_gpu(q, k, v, do, causal):
    qd, kd, vd, dod = (x.cuda() for x in (q, k, v, do))
    out, rm, rz = elsa_amd.twopass_attention_with_state(qd, kd, vd, is_causal=causal)
    dq, dk, dv = elsa_amd.twopass_attention_backward(qd, kd, vd, out, dod, is_causal=causal, row_m=rm, row_z=rz)
    torch.cuda.synchronize()
    return [t.float().cpu() for t in (out, rm, rz, dq, dk, dv)]


def _np(t):
    return t.double().numpy() if isinstance(t, torch.Tensor) else np.asarray(t, np.float64)


def _check_state(rm, rz, em, ez, what):
    m, em = _np(rm), _np(em)
    assert np.array_equal(np.isneginf(m), np.isneginf(em)), what
    fin = np.isfinite(em)
    # the fp16 fast path scores q rounded after scaling (attention_parallel_scan.py:257-259),
    # which moves the row max by up to ~1e-3 from the exact one, in the reference as here
    assert np.abs(m[fin] - em[fin]).max() <= 2e-3 * max(1.0, np.abs(em[fin]).max()), what
    np.testing.assert_allclose(_np(rz), _np(ez), rtol=3e-3, err_msg=what)


def _check_sampled_rows(q, k, v, do, got, dt, causal, rows, part, micro):
    """out, row state and dq of the sampled rows of every head against the reference
    restatement and the closed form."""
    out, rm, rz, dq = got[0], got[1], got[2], got[3]
    b, h, n, d = q.shape
    ro, rrm, rrz = T.forward(q, k, v, is_causal=causal, part_len=part, micro=micro, dtype=dt, rows=rows)
    eo, em, ez = T.exact_forward(q, k, v, is_causal=causal, rows=rows)
    describe(f"  out rows {assert_parity(_np(out[:, :, rows]), _np(eo), _np(ro), FWD_TOL[dt], 'out', dt)}")
    _check_state(rm[:, rows], rz[:, rows], em, ez, "row state")
    # the reference's dq of those rows from its own out and row state
    full_o = torch.zeros((b, h, n, d))
    full_o[:, :, rows] = ro.float()
    full_m = torch.full((b * h, n), float("-inf"))
    full_z = torch.zeros((b * h, n))
    full_m[:, rows] = rrm.float()
    full_z[:, rows] = rrz.float()
    rq, _, _ = T.backward(q, k, v, full_o, do, full_m, full_z, is_causal=causal, dtype=dt, rows=rows, need_kv=False)
    eq, _, _ = T.exact_backward(q, k, v, do, is_causal=causal, rows=rows, keys=[])
    describe(f"  dq rows {assert_parity(_np(dq[:, :, rows]), _np(eq), _np(rq), GRAD_TOL[dt], 'dq', dt)}")


def _check_full_heads(q, k, v, do, got, dt, causal, heads, part, micro):
    """Every row and key of the given heads (indices into the flattened B*H axis): out, dq,
    dk, dv against the reference restatement and the closed form."""
    b, h, n, d = q.shape
    hs = list(heads)
    flat = lambda x: x.reshape(1, b * h, n, d)[:, hs]  # noqa: E731
    qh, kh, vh, doh = (flat(x) for x in (q, k, v, do))
    out, dq, dk, dv = (flat(x) for x in (got[0], got[3], got[4], got[5]))
    ro, rm_, rz_ = T.forward(qh, kh, vh, is_causal=causal, part_len=part, micro=micro, dtype=dt)
    eo, _, _ = T.exact_forward(qh, kh, vh, is_causal=causal, row_chunk=512)
    describe(f"  heads {hs[0]}..{hs[-1]} out {assert_parity(_np(out), _np(eo), _np(ro), FWD_TOL[dt], 'out', dt)}")
    grads_ref = T.backward(qh, kh, vh, ro, doh, rm_, rz_, is_causal=causal, dtype=dt, row_chunk=512)
    grads_exact = T.exact_backward(qh, kh, vh, doh, is_causal=causal, row_chunk=512)
    for name, g, e, r in zip(("dq", "dk", "dv"), (dq, dk, dv), grads_exact, grads_ref):
        info = assert_parity(_np(g), _np(e), _np(r), GRAD_TOL[dt], name, dt)
        describe(f"  heads {hs[0]}..{hs[-1]} {name} {info}")


def _check_key_columns(q, k, v, do, got, dt, causal, head, keys, part, micro):
    """dk, dv of sampled key columns of one head, every query row contributing: against the
    reference restatement (its fold over every row of the head, then the key columns) and
    the closed form."""
    dk, dv = got[4], got[5]
    sl = slice(head, head + 1)
    qh, kh, vh, doh = (x[:, sl] for x in (q, k, v, do))
    ro, rm_, rz_ = T.forward(qh, kh, vh, is_causal=causal, part_len=part, micro=micro, dtype=dt)
    rk, rv = T.backward_key_columns(qh, kh, vh, ro, doh, rm_, rz_, keys, is_causal=causal, dtype=dt)
    _, ek, ev = T.exact_backward(qh, kh, vh, doh, is_causal=causal, rows=[], keys=keys)
    for name, g, e, r in (("dk", dk, ek, rk), ("dv", dv, ev, rv)):
        info = assert_parity(_np(g[:, sl][:, :, keys]), _np(e), _np(r), GRAD_TOL[dt], name, dt)
        describe(f"  head {head} {name} key columns {info}")


# (B, H, N, D), dtype, causal -- every row and head checked
FULL = [
    ((1, 8, 1024, 64), "fp16", False),
    ((1, 8, 1024, 64), "fp32", False),
    ((1, 8, 4096, 64), "fp16", False),
    ((1, 8, 4096, 64), "fp32", False),   # spot_check C1 / bwd_grad_correctness divisible control
    ((8, 3, 1025, 64), "fp32", False),   # bwd_grad_correctness.py:11-16 (ViT odd lengths)
    ((8, 3, 2305, 64), "fp32", False),
    ((8, 3, 4097, 64), "fp32", False),
    ((8, 3, 1025, 64), "fp16", False),
    ((8, 3, 2305, 64), "fp16", False),
    ((1, 8, 2048, 64), "fp16", True),    # causal config: N=2048 forward and backward
    ((1, 8, 4097, 64), "fp16", True),    # causal NEEDS_MASK length
    ((4, 32, 1024, 64), "fp16", False),  # the two-tile dq kernel in 256 8-wave work-groups of 512 rows
    ((2, 16, 4160, 64), "bf16", False),  # the same with a partial last work-group (64 of its 512 rows)
    ((2, 64, 1024, 64), "bf16", False),
    ((4, 32, 1024, 64), "fp16", True),   # causal: the 8-wave dq and dK/dV work-groups
    ((1, 8, 2048, 64), "bf16", False),   # the split backward (four key / row ranges, fp32 partials)
    ((2, 4, 2048, 32), "fp16", True),    # the same at d = 32, causal
]


@pytest.mark.parametrize("case", FULL, ids=[f"{c[0]}-{c[1]}-{'causal' if c[2] else 'full'}" for c in FULL])
def test_train_full_tensors(case):
    shape, dt, causal = case
    b, h, n, d = shape
    describe(f"train full tensors {shape} {dt} causal={causal}")
    q, k, v, do = _draw(shape, dt, seed=2026)
    got = _train_on_gpu(q, k, v, do, causal)
    part, micro = O.reference_routing(n, d, dt, training=True, is_causal=causal)
    _check_full_heads(q, k, v, do, got, dt, causal, range(b * h), part, micro)
    _, em, ez = T.exact_forward(q, k, v, is_causal=causal, row_chunk=512)
    _check_state(got[1], got[2], em, ez, "row state")


# (B, H, N, D), dtype, causal, how dk/dv are checked
BIG = [
    ((1, 8, 16384, 64), "fp16", False, "heads"),   # the north star
    ((1, 8, 16384, 64), "fp32", False, "heads"),
    ((1, 8, 8192, 64), "fp16", True, "heads"),
    ((1, 8, 32768, 64), "fp16", True, "keys"),
    ((1, 8, 65536, 64), "fp16", False, "keys"),
    ((1, 8, 65536, 64), "fp32", False, "keys"),
]


@pytest.mark.parametrize("case", BIG, ids=[f"{c[0]}-{c[1]}-{'causal' if c[2] else 'full'}" for c in BIG])
def test_train_at_benchmark_sizes(case):
    shape, dt, causal, how = case
    b, h, n, d = shape
    describe(f"train {shape} {dt} causal={causal}: sampled rows, dk/dv by {how}")
    q, k, v, do = _draw(shape, dt, seed=2026)
    got = _train_on_gpu(q, k, v, do, causal)
    part, micro = O.reference_routing(n, d, dt, training=True, is_causal=causal)
    # partition boundaries of this build's plan and of the reference's layout
    plan = forward_plan(q, is_causal=causal)  # reads only the shape and dtype
    edges = [j * plan["partition_len"] + o for j in range(1, plan["partitions"]) for o in (-1, 0)]
    edges += [part - 1, part, n // 2]
    rows = _rows(n, 40, seed=n, extra=edges)
    _check_sampled_rows(q, k, v, do, got, dt, causal, rows, part, micro)
    if how == "heads":
        _check_full_heads(q, k, v, do, got, dt, causal, [0, h - 1], part, micro)
    else:
        keys = _rows(n, 20, seed=n + 1, extra=edges)
        _check_key_columns(q, k, v, do, got, dt, causal, 0, keys, part, micro)


# inference forward (twopass_attention): the north star's forward and the reference's
# forward spot check (scripts/spot_check.py:39-51: fp32 within 1e-5 and fp16 within 5e-3 of SDPA)
FWD = [
    ((1, 8, 16384, 64), "fp16", False, 1234),
    ((1, 8, 65536, 64), "fp16", False, 1234),
    ((8, 3, 1025, 64), "fp32", False, 0),
    ((8, 3, 2305, 64), "fp16", False, 0),
    ((1, 8, 4096, 64), "fp32", False, 0),
    ((1, 8, 32768, 64), "fp16", True, 1234),
]


@pytest.mark.parametrize("case", FWD, ids=[f"{c[0]}-{c[1]}-{'causal' if c[2] else 'full'}" for c in FWD])
def test_inference_forward(case):
    shape, dt, causal, seed = case
    b, h, n, d = shape
    describe(f"inference forward {shape} {dt} causal={causal}")
    q, k, v, _ = _draw(shape, dt, seed)
    out = elsa_amd.twopass_attention(q.cuda(), k.cuda(), v.cuda(), is_causal=causal).float().cpu()
    part, micro = O.reference_routing(n, d, dt, training=False, is_causal=causal)
    rows = _rows(n, 48 if n > 8192 else 1 << 20, seed=seed + n, extra=[part - 1, part, n // 2])
    ro, _, _ = T.forward(q, k, v, is_causal=causal, part_len=part, micro=micro, dtype=dt, rows=rows)
    eo, _, _ = T.exact_forward(q, k, v, is_causal=causal, rows=rows)
    info = assert_parity(_np(out[:, :, rows]), _np(eo), _np(ro), FWD_TOL[dt], "out", dt)
    describe(f"  out {info}")
    if n <= 8192 and not causal:  # the spot check's own bars against the exact output
        assert info["vs_exact_beyond_half_ulp"] <= (1e-5 if dt == "fp32" else 5e-3)


# The training entry point (twopass_attention_train, the call the reference's benchmarks/bench_bwd.py
# times): its forward keeps a relaxed row state wherever the ping-pong fold runs (fp16/bf16, d64,
# non-causal, unbiased, partitions of at least 1024 keys): a reference m at most 8 below the row
# maximum and z relative to it, the same log-sum-exp.  "spikes" scales two late keys so that their
# stages must raise the reference (the fold's rare path) long after the first stage.
TRAIN = [
    ((1, 8, 16384, 64), "fp16", None, None),   # the north star's step (2 partitions of 8192 keys)
    ((1, 8, 8192, 64), "fp16", None, None),
    ((1, 4, 4096, 64), "fp16", "spikes", 1024),
    ((2, 8, 4097, 64), "fp16", None, 2048),    # ragged: a last partition of one key, its stage masked
    ((2, 16, 2048, 64), "bf16", None, 1024),
]


@pytest.mark.parametrize("case", TRAIN, ids=[f"{c[0]}-{c[1]}-{c[2] or 'randn'}-bn{c[3]}" for c in TRAIN])
def test_train_entry_point_relaxed_state(case):
    from elsa_amd.attention_bwd import _with_state

    shape, dt, fill, bn = case
    b, h, n, d = shape
    describe(f"twopass_attention_train {shape} {dt} {fill or 'randn'} block_n={bn}")
    q, k, v, do = _draw(shape, dt, seed=2027)
    if fill == "spikes":
        k[:, :, n - 700] *= 8
        k[:, :, n - 90] *= 12
    plan = forward_plan(q, is_causal=False, block_n=bn)
    assert plan["partition_len"] >= 1024 and plan["block_m"] == 256, plan  # the ping-pong fold's routing
    qd, kd, vd = (x.cuda().requires_grad_() for x in (q, k, v))
    out = elsa_amd.twopass_attention_train(qd, kd, vd, block_n=bn)
    dq, dk, dv = torch.autograd.grad(out, (qd, kd, vd), do.cuda())
    # the relaxed state against the exact one on the same inputs and plan
    with torch.no_grad():
        _, m_e, z_e = elsa_amd.twopass_attention_with_state(qd, kd, vd, block_n=bn)
        _, m_r, z_r = _with_state(qd, kd, vd, block_n=bn, exact_row_max=False)
    torch.cuda.synchronize()
    m_e, z_e, m_r, z_r = (_np(t.cpu()) for t in (m_e, z_e, m_r, z_r))
    assert np.isfinite(m_r).all() and (z_r > 0).all()
    assert (m_r <= m_e + 1e-5 * np.maximum(1.0, np.abs(m_e))).all() and (m_r >= m_e - 8.0 - 1e-5).all()
    lse_e, lse_r = m_e + np.log2(z_e), m_r + np.log2(z_r)
    err = np.abs(lse_r - lse_e).max()
    describe(f"  relaxed state: max |LSE relaxed - LSE exact| = {err:.3e}, "
             f"m below the maximum by up to {np.max(m_e - m_r):.3f}")
    assert err <= 2e-5 * max(1.0, np.abs(lse_e).max())
    got = [out.detach().float().cpu(), None, None] + [t.float().cpu() for t in (dq, dk, dv)]
    part, micro = O.reference_routing(n, d, dt, training=True, is_causal=False)
    heads = range(b * h) if b * h * n * n <= 8 * 4096 * 4096 else [0, b * h - 1]
    _check_full_heads(q, k, v, do, got, dt, False, heads, part, micro)
