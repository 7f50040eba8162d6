"""GPU parity of biased attention at lengths with several K partitions.

16-bit biases (fp16 and bf16) reach the Phase-1 fold in two ways: rows whose stride is a
multiple of 8 elements are read as 16-byte vectors (a row-padded view, as the Swin
drop-in builds it), other rows element by element (a dense [.., 1025, 1025] bias).  Each
case runs N = 1025 with 512-key partitions (3 partitions, so the merge and the
partition-boundary masking both run), causal and not, through the training call, and
checks out, row state, dq, dk, dv and dbias against the reference restatement (the
reference's generic kernel, attention.py:22-106, with that block_n) and the closed form.
The bias gradient is reduced over the broadcast dimensions as the reference's dense
fallback does (attention_bwd.py:973-1000).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import elsa_amd
from oracle import elsa_oracle as O
from oracle import torch_scan as T
from tests.gpu_util import FWD_TOL, GRAD_TOL, TORCH_DT, assert_parity, describe

pytestmark = pytest.mark.gpu

N = 1025
PART = 512

# q/k/v dtype, bias dtype, bias layout, causal, bias shape[, q/k/v shape (default B2 H2)]
CASES = [
    ("fp16", "fp16", "padded", False, (2, N, N)),
    ("fp16", "fp16", "dense", True, (2, N, N)),
    ("bf16", "bf16", "padded", True, (2, 2, N, N)),
    ("bf16", "bf16", "dense", False, (1, 2, N, N)),
    ("fp16", "bf16", "padded", False, (N, N)),
    ("bf16", "fp16", "dense", True, (2, 1, N, N)),
    # B4 H32: enough 256-row blocks for the 8-wave dq and dK/dV work-groups
    ("fp16", "fp16", "padded", True, (32, N, N), (4, 32, N, 64)),
    # the same kernels without the causal mask: 9 stages of 128 rows in dK/dV, the last one ragged
    ("bf16", "bf16", "dense", False, (1, 32, N, N), (4, 32, N, 64)),
]


def _ids(c):
    tail = f"-B{c[5][0]}H{c[5][1]}" if len(c) > 5 else ""
    return f"{c[0]}-bias{c[1]}-{c[2]}-{'causal' if c[3] else 'full'}-{'x'.join(map(str, c[4][:-2])) or 'nn'}{tail}"


def _bias_leaf(values: torch.Tensor, layout: str):
    """(leaf that collects the gradient, the view handed to the API)."""
    if layout == "dense":
        leaf = values.clone().cuda().requires_grad_(True)
        return leaf, leaf
    pad = (N + 7) // 8 * 8 + 8  # a row stride that is a multiple of 8 elements, 16-byte rows
    store = torch.zeros(values.shape[:-1] + (pad,), dtype=values.dtype)
    store[..., :N] = values
    leaf = store.cuda().requires_grad_(True)
    return leaf, leaf[..., :N]


def _np(t):
    return t.double().numpy() if isinstance(t, torch.Tensor) else np.asarray(t, np.float64)


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_biased_forward_and_backward_several_partitions(case):
    dt, bdt, layout, causal, bshape = case[:5]
    describe(f"biased fwd+bwd {_ids(case)}")
    shape = case[5] if len(case) > 5 else (2, 2, N, 64)
    g = torch.Generator().manual_seed(600 + len(bshape))
    q, k, v, do = (torch.randn(shape, generator=g).to(TORCH_DT[dt]) for _ in range(4))
    bias = (torch.randn(bshape, generator=g) * 0.5).to(TORCH_DT[bdt])
    leaf, view = _bias_leaf(bias, layout)
    if layout == "padded":
        assert view.stride(-2) % 8 == 0 and view.stride(-1) == 1 and view.data_ptr() % 16 == 0
    else:
        assert view.is_contiguous() and view.stride(-2) % 8 != 0
    qd, kd, vd = (x.cuda().requires_grad_(True) for x in (q, k, v))
    out = elsa_amd.twopass_attention_train(qd, kd, vd, bias=view, is_causal=causal, block_n=PART)
    out.backward(do.cuda())
    with torch.no_grad():
        _, rm, rz = elsa_amd.twopass_attention_with_state(qd.detach(), kd.detach(), vd.detach(), bias=view.detach(),
                                                         is_causal=causal, block_n=PART)
    torch.cuda.synchronize()
    got = {"out": out.detach().float().cpu(), "dq": qd.grad.float().cpu(), "dk": kd.grad.float().cpu(),
           "dv": vd.grad.float().cpu()}
    dbias = leaf.grad.float().cpu()
    if layout == "padded":
        assert torch.count_nonzero(dbias[..., N:]) == 0  # padding columns get no gradient
        dbias = dbias[..., :N]
    assert dbias.shape == bshape

    b32 = bias.float()  # the bias values the kernels read, widened
    ro, rrm, rrz = T.forward(q, k, v, bias=b32, is_causal=causal, part_len=PART, micro=PART, dtype=dt)
    eo, em, ez = T.exact_forward(q, k, v, bias=b32, is_causal=causal, row_chunk=512)
    describe(f"  out {assert_parity(_np(got['out']), _np(eo), _np(ro), FWD_TOL[dt], 'out', dt)}")
    fin = np.isfinite(_np(em))
    assert np.abs(_np(rm.float().cpu())[fin] - _np(em)[fin]).max() <= 1e-3
    np.testing.assert_allclose(_np(rz.float().cpu()), _np(ez), rtol=3e-3)
    rg = T.backward(q, k, v, ro, do, rrm, rrz, bias=b32, is_causal=causal, dtype=dt, row_chunk=512)
    eg = T.exact_backward(q, k, v, do, bias=b32, is_causal=causal, row_chunk=512)
    for name, r, e in zip(("dq", "dk", "dv"), rg, eg):
        describe(f"  {name} {assert_parity(_np(got[name]), _np(e), _np(r), GRAD_TOL[dt], name, dt)}")
    # dbias: the reference's reduction of dS over the broadcast dims, from its own forward
    # (reference-rounded out and state) and from the exact one
    qf, kf, vf, dof = (x.float().numpy() for x in (q, k, v, do))
    bnp = b32.numpy()
    rdb = O.dbias(qf, kf, vf, _np(ro), dof, _np(rrm), _np(rrz), bias=bnp, is_causal=causal, mode="ref")
    edb = O.dbias(qf, kf, vf, _np(eo), dof, _np(em), _np(ez), bias=bnp, is_causal=causal)
    summed = (shape[0] * shape[1]) // int(np.prod(bshape[:-2]))
    # the gradient comes back in the bias's own dtype: one ulp of it is allowed on top
    describe(f"  dbias {assert_parity(_np(dbias), edb, rdb, GRAD_TOL[dt] * summed, 'dbias', bdt)}")
