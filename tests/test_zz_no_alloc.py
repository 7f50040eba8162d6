"""elsa_fwd_noalloc -- the forward whose Phase-1 summaries live in a device array built into the
library, for callers that cannot allocate -- against elsa_fwd with a caller-allocated workspace:
the same output and row state, bit for bit, on calls in a row, each smaller than the one before.
The first call's summaries (142 MB) exceed the 64 MiB array, so it runs in several q-chunks
over it; later calls find the array holding the previous call's contents."""
from __future__ import annotations

import ctypes
import math

import pytest
import torch

from elsa_amd import _lib
from elsa_amd.attention import _canonical_bias, _make_fwd_args, forward_plan
from tests.gpu_util import TORCH_DT, describe

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20

# (B, H, N, D), dtype, causal, bias, exact row maximum (else the relaxed row state), whether
# the summaries exceed the array (several q-chunks over it)
CALLS = [
    ((1, 8, 65536, 64), "fp16", False, False, True, True),
    ((1, 8, 65536, 64), "fp16", False, False, False, True),
    ((1, 8, 16384, 64), "fp16", False, False, True, False),
    ((2, 3, 1025, 64), "bf16", True, True, True, False),
]


def _forward(lib, q, k, v, bias, causal, noalloc, exact=True):
    b, h, n, d = q.shape
    out = torch.full_like(q, float("nan"))
    rm = torch.full((b * h, n), float("nan"), device=q.device)
    rz = torch.full_like(rm, float("nan"))
    meta = _canonical_bias(bias, batch=b, heads=h, seq_len=n, device=q.device)
    args = _make_fwd_args(q, k, v, out, rm, rz, meta, is_causal=causal, summary_dtype=q.dtype, partition_len=None,
                          q_chunk=None, scale=1.0 / math.sqrt(d), exact_row_max=exact)
    stream = _lib.stream_handle(q.device)
    if noalloc:
        _lib.check(lib.elsa_fwd_noalloc(ctypes.byref(args), stream), "elsa_fwd_noalloc")
    else:
        plan = _lib.FwdPlan()
        _lib.check(lib.elsa_fwd_plan_get(ctypes.byref(args), ctypes.byref(plan)), "elsa_fwd_plan_get")
        ws = torch.empty(int(plan.workspace_bytes), dtype=torch.uint8, device=q.device)
        args.workspace, args.workspace_bytes = ws.data_ptr(), int(plan.workspace_bytes)
        _lib.check(lib.elsa_fwd(ctypes.byref(args), stream), "elsa_fwd")
    torch.cuda.synchronize()
    return out, rm, rz


def test_noalloc_forward_is_elsa_fwd_bit_for_bit_on_calls_in_a_row():
    lib = _lib.load()
    for i, (shape, dt, causal, with_bias, exact, chunked) in enumerate(CALLS):
        b, h, n, d = shape
        describe(f"elsa_fwd_noalloc call {i}: {shape} {dt} causal={causal} bias={with_bias} exact_row_max={exact}")
        g = torch.Generator().manual_seed(700 + i)
        q, k, v = (torch.randn(shape, generator=g).to(TORCH_DT[dt]).cuda() for _ in range(3))
        bias = (torch.randn((h, n, n), generator=g) * 0.5).to(TORCH_DT[dt]).cuda() if with_bias else None
        need = forward_plan(q, bias=bias, is_causal=causal)["workspace_bytes"]
        assert (need > SCRATCH_BYTES) == chunked, need  # the 64K calls run in several q-chunks
        ref = _forward(lib, q, k, v, bias, causal, noalloc=False, exact=exact)
        got = _forward(lib, q, k, v, bias, causal, noalloc=True, exact=exact)
        for name, a, r in zip(("out", "row_m", "row_z"), got, ref):
            assert torch.equal(a, r), (i, name)
        assert not torch.isnan(got[0]).any()


def test_noalloc_forward_replays_under_graph_capture():
    """Captured into a HIP graph (after one eager call on the device, which resolves the array's
    address) and replayed on new inputs, with eager work in between: every replay gives
    elsa_fwd's bits.  The 64K call runs several q-chunks over the array inside the graph."""
    lib = _lib.load()
    shape = (1, 8, 65536, 64)
    b, h, n, d = shape
    describe(f"elsa_fwd_noalloc under graph capture {shape} fp16")
    q, k, v = (torch.randn(shape, device="cuda", dtype=torch.float16) for _ in range(3))
    out = torch.empty_like(q)
    rm = torch.empty((b * h, n), device="cuda")
    rz = torch.empty_like(rm)
    args = _make_fwd_args(q, k, v, out, rm, rz, _canonical_bias(None, batch=b, heads=h, seq_len=n, device=q.device),
                          is_causal=False, summary_dtype=q.dtype, partition_len=None, q_chunk=None,
                          scale=1.0 / math.sqrt(d))
    _lib.check(lib.elsa_fwd_noalloc(ctypes.byref(args), _lib.stream_handle(q.device)), "elsa_fwd_noalloc")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _lib.check(lib.elsa_fwd_noalloc(ctypes.byref(args), _lib.stream_handle(q.device)), "elsa_fwd_noalloc")
    gen = torch.Generator(device="cuda").manual_seed(9)
    for i in range(3):
        for t in (q, k, v):
            t.copy_(torch.randn(shape, device="cuda", dtype=torch.float16, generator=gen))
        graph.replay()
        torch.cuda.synchronize()
        ref = _forward(lib, q, k, v, None, False, noalloc=False)
        for name, a, r in zip(("out", "row_m", "row_z"), (out, rm, rz), ref):
            assert torch.equal(a, r), (i, name)
