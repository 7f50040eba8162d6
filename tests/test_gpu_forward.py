"""GPU parity of the two-pass forward (Phase 1 on MFMA + Phase 2 merge) through the
C ABI, against the oracle (reference rounding points) and the fp64 closed form.

Shapes cover the reference's own tests (tests/test_attention.py:28-103: seeds,
shapes, q-chunking, bias, causal), the NEEDS_MASK lengths of the causal config
{197, 1025, 4097}, multi-partition routing, head dims 8..128 and fully masked rows.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import elsa_amd
from elsa_amd.attention import forward_plan, two_pass_explicit
from oracle import elsa_oracle as O
from tests.gpu_util import FWD_TOL, TORCH_DT, assert_parity, describe, dev, host, max_abs

pytestmark = pytest.mark.gpu

# (B, H, N, D), dtype, causal, block_n, q_chunk
CASES = [
    ((1, 2, 64, 32), "fp32", False, None, None),
    ((1, 2, 64, 32), "fp16", False, None, None),
    ((1, 3, 196, 64), "fp32", False, None, None),
    ((1, 3, 196, 64), "fp16", False, None, None),
    ((2, 4, 257, 32), "fp32", False, None, None),
    ((2, 4, 257, 32), "fp16", False, None, None),
    ((1, 2, 513, 64), "fp32", False, None, 128),
    ((1, 2, 513, 64), "fp16", False, None, 128),
    ((1, 2, 129, 32), "fp32", True, None, None),
    ((1, 2, 129, 32), "fp16", True, None, None),
    ((1, 2, 197, 64), "fp16", True, 64, None),
    ((1, 2, 1025, 64), "fp16", True, 256, None),
    ((1, 2, 1025, 64), "fp16", False, 256, None),
    ((1, 2, 4097, 64), "fp16", True, None, None),
    ((1, 2, 4097, 64), "fp16", False, 1024, None),
    ((1, 2, 4096, 64), "fp16", False, 4096, None),  # the ping-pong fold over one partition, finalize fused
    ((1, 2, 4097, 64), "bf16", False, 4097, None),
    ((1, 2, 2048, 64), "fp16", True, None, None),
    ((1, 3, 777, 64), "fp16", True, 256, 256),   # causal q-chunks: the row-block order without longest first
    ((1, 2, 1000, 64), "bf16", True, 200, None),  # causal partitions not a multiple of the row block
    ((1, 2, 1024, 64), "fp32", False, 256, None),
    ((1, 2, 1024, 64), "fp32", True, 256, None),
    ((1, 3, 197, 64), "bf16", False, None, None),
    ((1, 2, 300, 128), "fp16", False, 128, None),
    ((1, 2, 300, 128), "fp32", True, 128, None),
    ((1, 2, 100, 8), "fp16", False, None, None),
    ((1, 2, 100, 48), "fp32", False, None, None),
    ((1, 2, 77, 20), "fp32", True, None, None),
]


def _ids(case):
    (b, h, n, d), dt, causal, bn, qc = case
    return f"{b}x{h}x{n}x{d}-{dt}-{'causal' if causal else 'full'}-bn{bn}-qc{qc}"


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_forward_matches_oracle_and_closed_form(case):
    shape, dt, causal, bn, qc = case
    describe(f"forward {_ids(case)}")
    q, k, v = O.make_inputs(shape, seed=sum(shape), dtype=dt)
    out, row_m, row_z = elsa_amd.twopass_attention_with_state(
        dev(q, dt), dev(k, dt), dev(v, dt), is_causal=causal, block_n=bn, q_chunk_size=qc
    )
    torch.cuda.synchronize()
    qf, kf, vf = (np.asarray(x, np.float32) for x in (q, k, v))
    eo, em, ez = O.exact_forward(qf, kf, vf, is_causal=causal)
    ro, rm, _ = O.forward(q, k, v, is_causal=causal, part_len=bn, dtype=dt, mode="ref")
    describe(str(assert_parity(host(out), eo, ro, FWD_TOL[dt], "out", dt)))
    m = host(row_m)
    assert np.array_equal(np.isneginf(m), np.isneginf(em))
    fin = np.isfinite(em)
    # the reference's fp16 d64 fold scores q rounded to fp16 after scaling
    # (attention_parallel_scan.py:257-259), which moves its row max off the exact one by up
    # to ~1e-3; the row max must match the reference path and stay within twice its error
    mbar = 1e-4 * max(1.0, np.abs(em[fin]).max())
    assert np.abs(m[fin] - rm[fin]).max() <= mbar
    assert np.abs(m[fin] - em[fin]).max() <= max(mbar, 2 * np.abs(rm[fin] - em[fin]).max())
    np.testing.assert_allclose(host(row_z), ez, rtol=2e-3 if dt != "fp32" else 1e-5)


@pytest.mark.parametrize("dt", ["fp32", "fp16"])
@pytest.mark.parametrize("bias_shape", [(1, 3, 128, 128), (2, 3, 128, 128), (128, 128), (3, 128, 128)])
def test_forward_bias(dt, bias_shape):
    describe(f"forward bias {bias_shape} {dt}")
    shape = (2, 3, 128, 32)
    q, k, v = O.make_inputs(shape, seed=1, dtype=dt)
    bias = (np.random.default_rng(1).standard_normal(bias_shape) * 0.05).astype(np.float32)
    out = elsa_amd.twopass_attention(dev(q, dt), dev(k, dt), dev(v, dt), bias=dev(bias, "fp32"))
    eo, _, _ = O.exact_forward(np.float32(q), np.float32(k), np.float32(v), bias=bias)
    ro, _, _ = O.forward(q, k, v, bias=bias, dtype=dt, mode="ref")
    assert_parity(host(out), eo, ro, FWD_TOL[dt], "out", dt)


@pytest.mark.parametrize("dt", ["fp32", "fp16"])
def test_forward_swin_window_bias_and_shift_mask(dt):
    # Swin-T stage-1 geometry: 49-token windows, d=32, rel-pos bias + -100 shift mask
    describe(f"forward swin window {dt}")
    b_win, h, n, d = 16, 3, 49, 32
    q, k, v = O.make_inputs((b_win, h, n, d), seed=7, dtype=dt)
    rng = np.random.default_rng(7)
    bias = (rng.standard_normal((b_win, h, n, n)) * 0.5).astype(np.float32)
    bias[1::2, :, :, 30:] -= 100.0
    out = elsa_amd.twopass_attention(dev(q, dt), dev(k, dt), dev(v, dt), bias=dev(bias, "fp32"))
    eo, _, _ = O.exact_forward(np.float32(q), np.float32(k), np.float32(v), bias=bias)
    ro, _, _ = O.forward(q, k, v, bias=bias, dtype=dt, mode="ref")
    describe(str(assert_parity(host(out), eo, ro, FWD_TOL[dt], "out", dt)))


def test_fully_masked_rows_return_zero_and_identity_state():
    describe("forward fully-masked rows")
    q, k, v = O.make_inputs((1, 2, 70, 32), seed=3, dtype="fp32")
    bias = np.zeros((70, 70), np.float32)
    bias[5, :] = -np.inf
    bias[69, :] = -np.inf
    out, rm, rz = elsa_amd.twopass_attention_with_state(dev(q, "fp32"), dev(k, "fp32"), dev(v, "fp32"),
                                                        bias=dev(bias, "fp32"), block_n=32)
    o = host(out)
    assert np.all(o[:, :, [5, 69]] == 0)
    assert np.all(np.isneginf(host(rm)[:, [5, 69]])) and np.all(host(rz)[:, [5, 69]] == 0)
    eo, _, _ = O.exact_forward(q, k, v, bias=bias)
    assert max_abs(o, eo) <= 1e-6


def test_reference_test_shapes_against_sdpa():
    # the reference's own oracle (tests/test_attention.py:16-25): fp32 SDPA cast back to dtype
    for dt, tol in (("fp32", 2e-4), ("fp16", 3e-2)):
        for shape in [(1, 2, 64, 32), (1, 3, 196, 64), (2, 4, 257, 32)]:
            torch.manual_seed(0)
            dtype = torch.float32 if dt == "fp32" else torch.float16
            q = torch.randn(shape, device="cuda", dtype=dtype)
            k = torch.randn(shape, device="cuda", dtype=dtype)
            v = torch.randn(shape, device="cuda", dtype=dtype)
            out = elsa_amd.twopass_attention(q, k, v)
            ref = torch.nn.functional.scaled_dot_product_attention(
                q.float().cpu(), k.float().cpu(), v.float().cpu(), scale=1.0 / math.sqrt(shape[-1])).to(dtype)
            torch.testing.assert_close(out.cpu(), ref, atol=tol, rtol=tol)


def test_algorithm_rejected_on_device():
    q = torch.randn((1, 2, 128, 32), device="cuda", dtype=torch.float16)
    with pytest.raises(ValueError, match="paper_scan"):
        elsa_amd.twopass_attention(q, q, q, algorithm="not_available")


def test_summary_dtypes_agree():
    describe("forward summary dtypes")
    q, k, v = O.make_inputs((1, 3, 196, 64), seed=3, dtype="fp16")
    eo, _, _ = O.exact_forward(np.float32(q), np.float32(k), np.float32(v))
    for sd in (torch.float16, torch.float32, torch.bfloat16):
        out = elsa_amd.twopass_attention(dev(q, "fp16"), dev(k, "fp16"), dev(v, "fp16"), summary_dtype=sd,
                                         block_n=64)
        assert max_abs(host(out), eo) <= (3e-3 if sd == torch.bfloat16 else 1e-3)


# fp16 inputs with summary_dtype=fp32: the reference's summary kernel runs with SUMMARY_DOT_FP32
# (attention_parallel_scan.py:701, :902) and forms p @ v from the fp32 p (attention.py:96-99);
# the fold keeps p to ~22 bits there (a hi/lo fp16 split of p), so the plain bar applies.
F32SUM = [
    ((1, 2, 1025, 64), False, 256),
    ((1, 2, 1025, 64), True, 256),
    ((1, 3, 4096, 64), False, None),   # planner routing (1024-key partitions, the 4-wave fold)
    ((2, 2, 300, 32), False, 128),
]


@pytest.mark.parametrize("case", F32SUM, ids=[f"{c[0]}-{'causal' if c[1] else 'full'}-bn{c[2]}" for c in F32SUM])
def test_fp16_inputs_with_fp32_summaries(case):
    shape, causal, bn = case
    describe(f"fp16 inputs, fp32 summaries {shape} causal={causal} block_n={bn}")
    q, k, v = O.make_inputs(shape, seed=21, dtype="fp16")
    plan = forward_plan(dev(q, "fp16"), is_causal=causal, block_n=bn, summary_dtype=torch.float32)
    assert plan["partitions"] >= 2, plan
    out = elsa_amd.twopass_attention(dev(q, "fp16"), dev(k, "fp16"), dev(v, "fp16"), is_causal=causal, block_n=bn,
                                     summary_dtype=torch.float32)
    eo, _, _ = O.exact_forward(np.float32(q), np.float32(k), np.float32(v), is_causal=causal)
    part = plan["partition_len"]
    ro, _, _ = O.forward(q, k, v, is_causal=causal, part_len=part, dtype="fp16", mode="ref", summary_dtype="fp32")
    describe(str(assert_parity(host(out), eo, ro, FWD_TOL["fp16"], "out", "fp16", plain=True)))
    # and nearer to the reference's fp32-summary result than to its fp16-summary one
    r16, _, _ = O.forward(q, k, v, is_causal=causal, part_len=part, dtype="fp16", mode="ref")
    got = host(out)
    assert np.mean(got == np.asarray(ro, np.float64)) > np.mean(got == np.asarray(r16, np.float64))


@pytest.mark.parametrize("causal", [False, True])
def test_two_pass_structure(causal):
    """Phase 1 writes P>1 summaries per row to HBM; Phase 2 alone turns them into the output
    (the reference's scripts/verify_2pass.py)."""
    describe(f"two-pass structure causal={causal}")
    shape = (1, 2, 1000, 64)
    q, k, v = O.make_inputs(shape, seed=5, dtype="fp16")
    out, rm, rz, m_buf, z_buf, s_buf, plan = two_pass_explicit(dev(q, "fp16"), dev(k, "fp16"), dev(v, "fp16"),
                                                                 is_causal=causal, block_n=256)
    assert plan["partitions"] == 4 and tuple(s_buf.shape) == (4, 2, 1000, 64)
    # every partition summary equals the oracle's fold of that partition at the reference's
    # rounding points (non-causal fp16 d64: q rounded after scaling, attention_parallel_scan.py:257-259)
    qf = np.float32(q).reshape(2, 1000, 64)
    for kb in range(4):
        rows = np.arange(1000) if not causal else np.arange(kb * 256, 1000)
        pm, pz, ps = O.phase1_partition(qf[:, rows], np.float32(k).reshape(2, 1000, 64),
                                        np.float32(v).reshape(2, 1000, 64), row_idx=rows, k_begin=kb * 256,
                                        k_end=min(1000, kb * 256 + 256), n_ctx=1000, is_causal=causal, bias=None,
                                        dtype="fp16", mode="ref")
        hm = host(m_buf[kb])[:, rows]
        assert np.abs(hm - pm).max() < 1e-4
        np.testing.assert_allclose(host(z_buf[kb])[:, rows], pz, rtol=2e-3)
        np.testing.assert_allclose(host(s_buf[kb])[:, rows], ps, rtol=3e-3, atol=3e-3 * np.abs(ps).max())
    ref = elsa_amd.twopass_attention(dev(q, "fp16"), dev(k, "fp16"), dev(v, "fp16"), is_causal=causal, block_n=256)
    assert torch.equal(out, ref)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("parts", [2, 3, 4, 5, 7, 8, 9, 17])
def test_phase2_every_partition_count(parts, causal):
    """Phase 2 over P partitions: the fixed-leaf kernel up to 8 (all leaves live, or a causal
    row's leading ones), the generic one beyond; both against the oracle's Blelloch up-sweep
    and the closed form."""
    n = 1000
    bn = -(-n // parts)
    describe(f"phase2 P={parts} block_n={bn} causal={causal}")
    q, k, v = O.make_inputs((1, 2, n, 64), seed=40 + parts, dtype="fp16")
    out, rm, rz, *_, plan = two_pass_explicit(dev(q, "fp16"), dev(k, "fp16"), dev(v, "fp16"), is_causal=causal,
                                              block_n=bn)
    torch.cuda.synchronize()
    assert plan["partitions"] == parts
    eo, em, ez = O.exact_forward(np.float32(q), np.float32(k), np.float32(v), is_causal=causal)
    ro, rmo, _ = O.forward(q, k, v, is_causal=causal, part_len=bn, dtype="fp16", mode="ref", merge_kind="tree")
    assert_parity(host(out), eo, ro, FWD_TOL["fp16"], "out", "fp16")
    assert np.abs(host(rm) - rmo).max() <= 1e-4 * max(1.0, np.abs(rmo).max())
    np.testing.assert_allclose(host(rz), ez, rtol=2e-3)


def test_north_star_shape_properties():
    """B1 H8 d64 N16384 fp16: closed form on sampled rows, a permutation of the keys leaves
    the output unchanged (monoid order invariance) and partitions 2/8 agree."""
    describe("forward north-star properties")
    shape = (1, 8, 16384, 64)
    g = torch.Generator().manual_seed(1234)
    q = torch.randn(shape, generator=g).half()
    k = torch.randn(shape, generator=g).half()
    v = torch.randn(shape, generator=g).half()
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    plan = forward_plan(qd)
    assert plan["partitions"] >= 2
    out = elsa_amd.twopass_attention(qd, kd, vd)
    out8 = elsa_amd.twopass_attention(qd, kd, vd, block_n=2048)
    perm = torch.randperm(16384, generator=g)
    outp = elsa_amd.twopass_attention(qd, kd[:, :, perm].contiguous(), vd[:, :, perm].contiguous())
    torch.cuda.synchronize()
    rows = np.random.default_rng(0).choice(16384, 64, replace=False)
    qs = q.float().numpy()[:, :, rows]
    sc = np.einsum("bhid,bhjd->bhij", qs.astype(np.float64), k.float().numpy().astype(np.float64)) / 8.0
    sc -= sc.max(-1, keepdims=True)
    p = np.exp(sc)
    p /= p.sum(-1, keepdims=True)
    eo = np.einsum("bhij,bhjd->bhid", p, v.float().numpy().astype(np.float64))
    assert max_abs(host(out)[:, :, rows], eo) <= 1e-3
    assert max_abs(host(out), host(out8)) <= 1e-3
    assert max_abs(host(out), host(outp)) <= 1e-3


@pytest.mark.parametrize("shape,dt,causal,bias", [((8, 3, 197, 64), "fp16", False, False),
                                                  ((2, 2, 300, 128), "bf16", True, False),
                                                  ((4, 3, 49, 32), "fp32", False, True)])
def test_single_partition_fused_finalize_matches_two_launches(shape, dt, causal, bias):
    """With one K partition the forward applies Phase 2's finalize inside Phase 1; the result
    must equal, bit for bit, the explicit Phase 1 + Phase 2 launches on the same plan."""
    describe(f"fused finalize {shape} {dt} causal={causal} bias={bias}")
    q, k, v = O.make_inputs(shape, seed=31, dtype=dt)
    qd, kd, vd = dev(q, dt), dev(k, dt), dev(v, dt)
    plan = forward_plan(qd, is_causal=causal)
    assert plan["partitions"] == 1
    if bias:
        b = dev((np.random.default_rng(31).standard_normal((shape[1], shape[2], shape[2])) * 0.5)
                .astype(np.float32), "fp32")
        out, rm, rz = elsa_amd.twopass_attention_with_state(qd, kd, vd, bias=b, is_causal=causal)
        o2, m2, z2 = elsa_amd.twopass_attention_with_state(qd, kd, vd, bias=b, is_causal=causal,
                                                           q_chunk_size=shape[2] // 2 + 1)
        assert torch.equal(out, o2) and torch.equal(rm, m2) and torch.equal(rz, z2)
        return
    out, rm, rz = elsa_amd.twopass_attention_with_state(qd, kd, vd, is_causal=causal)
    o2, m2, z2, *_ = two_pass_explicit(qd, kd, vd, is_causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(out, o2)
    assert torch.equal(rm, m2) and torch.equal(rz, z2)


@pytest.mark.parametrize("dt,n,causal", [("fp16", 197, False), ("bf16", 4097, True), ("fp32", 300, False),
                                         ("fp16", 16384, False)])
def test_strided_operands_read_in_place(dt, n, causal):
    """q/k/v as views of a fused [B, N, 3, H, D] projection (and a head-broadcast k) and an
    output written as [B, N, H, D] memory give the same bits as dense operands."""
    from elsa_amd.attention import _twopass_attention

    describe(f"strided {dt} n={n} causal={causal}")
    b, h, d = 2, 3, 64
    g = torch.Generator().manual_seed(n)
    qkv = torch.randn((b, n, 3, h, d), generator=g).to(TORCH_DT[dt]).cuda()
    q, k, v = qkv.permute(2, 0, 3, 1, 4).unbind(0)
    assert not q.is_contiguous()
    dense = elsa_amd.twopass_attention(q.contiguous(), k.contiguous(), v.contiguous(), is_causal=causal)
    strided = elsa_amd.twopass_attention(q, k, v, is_causal=causal)
    kw = dict(bias=None, is_causal=causal, block_m=None, block_n=None, q_chunk_size=None, summary_dtype=None,
              phase1_warps=None, phase2_warps=None, phase1_stages=None, phase2_stages=None,
              input_precision="auto", algorithm="auto")
    bnhd = _twopass_attention(q, k, v, out_bnhd=True, **kw)
    assert bnhd.transpose(1, 2).is_contiguous()
    torch.cuda.synchronize()
    assert torch.equal(strided, dense) and torch.equal(bnhd, dense)
    # a key/value shared by all heads (stride 0 over heads)
    k1 = k[:, :1].expand(b, h, n, d)
    v1 = v[:, :1].expand(b, h, n, d)
    shared = elsa_amd.twopass_attention(q, k1, v1, is_causal=causal)
    ref = elsa_amd.twopass_attention(q.contiguous(), k1.contiguous(), v1.contiguous(), is_causal=causal)
    assert torch.equal(shared, ref)


@pytest.mark.parametrize("dt,shape,causal,bias,kw", [
    ("fp16", (8, 3, 197, 64), False, False, {}),
    ("fp16", (1, 8, 2048, 64), True, False, {}),
    ("bf16", (2, 3, 1025, 32), False, True, {}),
    ("fp32", (1, 2, 300, 128), True, False, {}),
    ("fp16", (1, 4, 4096, 64), False, False, {"block_n": 1024, "q_chunk_size": 1000}),
    ("fp16", (1, 2, 777, 64), False, False, {"summary_dtype": torch.float32}),
])
def test_cpp_and_python_inference_forwards_agree(dt, shape, causal, bias, kw):
    """twopass_attention on operands read in place runs the C++ host side (attention_forward in
    elsa_torch.cpp); _elsa_forward is its Python twin over the same C ABI: the same bits."""
    from elsa_amd import _lib
    from elsa_amd.attention import _elsa_forward, _resolve_forward_options

    describe(f"C++ and Python inference forward {dt} {shape} causal={causal} bias={bias} {kw}")
    g = torch.Generator().manual_seed(41)
    q, k, v = (torch.randn(shape, generator=g).to(TORCH_DT[dt]).cuda() for _ in range(3))
    b = torch.randn(shape[2], shape[2], generator=g).to(TORCH_DT[dt]).cuda() if bias else None
    calls = []
    real = _lib.torch_module().attention_forward

    def spy(*a):
        calls.append(1)
        return real(*a)

    mod = _lib.torch_module()
    mod.attention_forward = spy
    try:
        got = elsa_amd.twopass_attention(q, k, v, bias=b, is_causal=causal, **kw)
    finally:
        mod.attention_forward = real
    assert calls, "twopass_attention did not take the C++ host path"
    part, qc, sdt = _resolve_forward_options(
        q, block_m=None, block_n=kw.get("block_n"), q_chunk_size=kw.get("q_chunk_size"),
        summary_dtype=kw.get("summary_dtype"), phase1_warps=None, phase2_warps=None, phase1_stages=None,
        phase2_stages=None, input_precision="auto")
    want, *_ = _elsa_forward(q, k, v, bias=b, is_causal=causal, summary_dtype=sdt, partition_len=part, q_chunk=qc,
                             want_state=False)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
