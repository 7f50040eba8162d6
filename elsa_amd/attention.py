"""Public forward API: ``twopass_attention`` (mirrors reference attention.py:239-321).

Validation order, messages and defaults follow the reference so callers and tests
port unchanged.  Execution always goes to the HIP library (``libelsa_hip.so``):
Phase 1 writes one ``(m, z, s)`` summary per (row, K partition) to HBM, Phase 2
reads them back and merges them (up-sweep tree; causal rows consume the prefix at
their own partition).

Triton-only knobs (``block_m``, ``phase*_warps``, ``phase*_stages``) are validated
exactly like the reference and otherwise ignored: the HIP kernels pick their own
tile shapes for gfx950.  ``block_n`` is honoured as the K-partition width,
``q_chunk_size`` as the number of query rows per Phase1+Phase2 pass, and
``summary_dtype`` as the storage type of the ``s`` summaries.  ``input_precision``
is validated; fp32 inputs always use full-fp32 MFMA products (gfx950 has no
reduced-precision fp32 MFMA), which is at least as accurate as ``tf32x3``.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Literal, Optional

import torch
import torch.nn.functional as F

from . import _lib


@dataclass(frozen=True)
class _BiasMeta:
    tensor: Optional[torch.Tensor]
    stride_b: int
    stride_h: int
    stride_q: int
    stride_k: int
    has_bias: bool


def _next_power_of_2(x: int) -> int:
    return 1 << (int(x) - 1).bit_length()


def _validate_warps(name: str, value: int) -> int:
    """attention.py:113-117."""
    value = int(value)
    if value not in (1, 2, 4, 8):
        raise ValueError(f"{name} must be one of 1, 2, 4, or 8")
    return value


def _canonical_bias(
    bias: Optional[torch.Tensor],
    *,
    batch: int,
    heads: int,
    seq_len: int,
    device: torch.device,
) -> _BiasMeta:
    """Bias shapes [N,N], [1|H,N,N], [1|B,1|H,N,N] broadcast by zero strides (attention.py:120-159)."""
    if bias is None:
        return _BiasMeta(None, 0, 0, 0, 0, False)
    if bias.device != device:
        raise ValueError("bias must live on the same device as q/k/v")
    if bias.shape[-2:] != (seq_len, seq_len):
        raise ValueError(f"bias last dims must be {(seq_len, seq_len)}, got {tuple(bias.shape)}")
    if bias.dim() == 2:
        view = bias.contiguous().view(1, 1, seq_len, seq_len)
    elif bias.dim() == 3:
        if bias.shape[0] not in (1, heads):
            raise ValueError("3D bias must have shape [1,N,N] or [H,N,N]")
        view = bias.contiguous().view(1, bias.shape[0], seq_len, seq_len)
    elif bias.dim() == 4:
        if bias.shape[0] not in (1, batch) or bias.shape[1] not in (1, heads):
            raise ValueError("4D bias must broadcast as [B,H,N,N]")
        # the kernels take any strides: a 4D bias with dense keys and no broadcast (zero-stride)
        # dimension is used as it is, e.g. rows padded to a 16-byte multiple for vector loads
        dense_keys = bias.stride(-1) == 1
        no_broadcast = all(st > 0 or sz == 1 for st, sz in zip(bias.stride(), bias.shape))
        view = bias if dense_keys and no_broadcast else bias.contiguous()
    else:
        raise ValueError("bias must have shape [N,N], [H,N,N], or [B,H,N,N]")
    if view.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        view = view.float()
    stride_b = 0 if view.shape[0] == 1 else view.stride(0)
    stride_h = 0 if view.shape[1] == 1 else view.stride(1)
    return _BiasMeta(view, int(stride_b), int(stride_h), int(view.stride(2)), int(view.stride(3)), True)


def _user_tiles(
    *,
    dtype: torch.dtype,
    head_dim: int,
    block_m: Optional[int],
    block_n: Optional[int],
    q_chunk_size: Optional[int],
    phase1_warps: Optional[int],
    phase2_warps: Optional[int],
    phase1_stages: Optional[int],
    phase2_stages: Optional[int],
) -> tuple[Optional[int], Optional[int]]:
    """What the reference's routing (attention.py:162-236, :302) does to user-given knobs.

    Warps must be 1, 2, 4 or 8 and stages convert to int (the reference's validation);
    ``block_n`` and ``q_chunk_size`` are clamped to at least 16, and ``q_chunk_size`` is
    rounded down to a multiple of block_m (the reference's default: 32 rows for fp32 or head
    dims above 64, else 64), but not below it.  Returns (partition_len, q_chunk), None
    where the caller gave nothing: the HIP planner routes those itself.
    """
    _validate_warps("phase1_warps", 4 if phase1_warps is None else phase1_warps)
    _validate_warps("phase2_warps", 4 if phase2_warps is None else phase2_warps)
    for stages in (phase1_stages, phase2_stages):
        if stages is not None:
            int(stages)
    bm = max(16, int(block_m)) if block_m is not None else (32 if dtype == torch.float32 or head_dim > 64 else 64)
    bn = None if block_n is None else max(16, int(block_n))
    qc = None if q_chunk_size is None else max(bm, (max(16, int(q_chunk_size)) // bm) * bm)
    return bn, qc


def _check_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, who: str) -> None:
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must have shape [B,H,N,D]")
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k, v must have identical shapes")
    if q.device.type != "cuda":
        raise ValueError(f"{who} currently requires CUDA tensors")
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("supported dtypes are fp16, bf16, and fp32")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k, v must share one dtype")
    if k.device != q.device or v.device != q.device:
        raise ValueError("q, k, v must live on one device")


def _resolve_precision(input_precision: str, dtype: torch.dtype) -> str:
    if input_precision == "auto":
        input_precision = "tf32x3" if dtype == torch.float32 else "ieee"
    if input_precision not in ("ieee", "tf32", "tf32x3"):
        raise ValueError("input_precision must be 'auto', 'ieee', 'tf32', or 'tf32x3'")
    return input_precision


def _operand(x: torch.Tensor) -> torch.Tensor:
    """x itself when the kernels can read it in place (contiguous head dim of a multiple of
    8 elements, batch/head/row strides that are multiples of 8, 16-byte aligned base),
    else a dense, padded copy."""
    st = x.stride()
    if (x.shape[-1] % 8 == 0 and st[-1] == 1 and all(s % 8 == 0 and s >= 0 for s in st[:3])
            and st[2] >= x.shape[-1] and x.data_ptr() % 16 == 0):
        return x
    return _pad_head_dim(x.contiguous())


def _pad_head_dim(x: torch.Tensor) -> torch.Tensor:
    """Zero-pad the head dim to a multiple of 8 and make the base 16-byte aligned.

    The kernels move 16-byte chunks of rows; zero columns do not change q.k, and
    the padded output columns are dropped by the caller.
    """
    d = x.shape[-1]
    dp = (d + 7) // 8 * 8
    if dp != d:
        return F.pad(x, (0, dp - d))
    return x if x.data_ptr() % 16 == 0 else x.clone()


def _make_fwd_args(q_c, k_c, v_c, out, row_m, row_z, bias_meta: _BiasMeta, *, is_causal, summary_dtype,
                   partition_len, q_chunk, scale, exact_row_max=True) -> _lib.FwdArgs:
    batch, heads, seq_len, head_dim = map(int, q_c.shape)
    a = _lib.FwdArgs()
    a.q, a.k, a.v, a.out = q_c.data_ptr(), k_c.data_ptr(), v_c.data_ptr(), out.data_ptr()
    a.row_m = _lib.ptr(row_m)
    a.row_z = _lib.ptr(row_z)
    a.bias = _lib.bias_desc(bias_meta.tensor, (bias_meta.stride_b, bias_meta.stride_h, bias_meta.stride_q,
                                               bias_meta.stride_k))
    a.batch, a.heads, a.seq_len, a.head_dim = batch, heads, seq_len, head_dim
    a.dtype = _lib.dtype_code(q_c.dtype)
    a.summary_dtype = _lib.dtype_code(summary_dtype)
    a.is_causal = 1 if is_causal else 0
    a.partition_len = int(partition_len or 0)
    a.q_chunk = int(q_chunk or 0)
    a.scale = float(scale)
    a.q_layout, a.k_layout, a.v_layout = (_lib.layout_of(t) for t in (q_c, k_c, v_c))
    a.out_layout = _lib.layout_of(out)
    a.exact_row_max = 1 if exact_row_max else 0
    return a


def _elsa_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    bias: Optional[torch.Tensor],
    is_causal: bool,
    summary_dtype: torch.dtype,
    partition_len: Optional[int],
    q_chunk: Optional[int],
    want_state: bool,
    out_bnhd: bool = False,
    exact_row_max: bool = True,
):
    """Run Phase 1 + Phase 2 on the HIP library.  Returns (out, row_m, row_z, q_c, k_c, v_c).

    ``exact_row_max`` False lets row_m be the fold's lazy reference (at most 8 below the row
    maximum, row_z relative to it): the same log-sum-exp for the backward, and the fp16/bf16 d64
    fold skips most per-stage maxima.  A forward without state takes that path.

    q, k, v may be strided views (read in place when ``_operand`` allows); ``out_bnhd``
    allocates the output as [B, N, H, D] memory (returned as its [B, H, N, D] view), so
    that ``out.transpose(1, 2).reshape(B, N, H * D)`` costs no copy.
    """
    lib = _lib.load()
    batch, heads, seq_len, head_dim = map(int, q.shape)
    bias_meta = _canonical_bias(bias, batch=batch, heads=heads, seq_len=seq_len, device=q.device)
    scale = 1.0 / math.sqrt(head_dim)
    qp, kp, vp = _operand(q), _operand(k), _operand(v)
    q_c, k_c, v_c = qp, kp, vp
    dp = int(qp.shape[-1])
    if out_bnhd and dp == head_dim:
        out = torch.empty((batch, seq_len, heads, dp), dtype=q.dtype, device=q.device).permute(0, 2, 1, 3)
    else:
        out = torch.empty((batch, heads, seq_len, dp), dtype=q.dtype, device=q.device)
    row_m = torch.empty((batch * heads, seq_len), device=q.device, dtype=torch.float32) if want_state else None
    row_z = torch.empty_like(row_m) if want_state else None
    args = _make_fwd_args(qp, kp, vp, out, row_m, row_z, bias_meta, is_causal=is_causal,
                          summary_dtype=summary_dtype, partition_len=partition_len, q_chunk=q_chunk, scale=scale,
                          exact_row_max=exact_row_max and want_state)
    plan = _lib.FwdPlan()
    _lib.check(lib.elsa_fwd_plan_get(ctypes.byref(args), ctypes.byref(plan)), "elsa_fwd_plan_get")
    ws = torch.empty(int(plan.workspace_bytes), dtype=torch.uint8, device=q.device)
    args.workspace = ws.data_ptr()
    args.workspace_bytes = int(plan.workspace_bytes)
    with torch.cuda.device(q.device):
        _lib.check(lib.elsa_fwd(ctypes.byref(args), _lib.stream_handle(q.device)), "elsa_fwd")
    if dp != head_dim:
        out = out[..., :head_dim].contiguous()
        q_c, k_c, v_c = (t[..., :head_dim] for t in (qp, kp, vp))
    return out, row_m, row_z, q_c, k_c, v_c


def _resolve_forward_options(q, *, block_m, block_n, q_chunk_size, summary_dtype, phase1_warps, phase2_warps,
                             phase1_stages, phase2_stages, input_precision):
    """Shared validation of the forward kwargs; returns (partition_len, q_chunk, summary_dtype)."""
    _resolve_precision(input_precision, q.dtype)
    if summary_dtype is None:
        summary_dtype = torch.float32 if q.dtype == torch.float32 else q.dtype
    if summary_dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("summary_dtype must be fp16, bf16, or fp32")
    bn, qc = _user_tiles(dtype=q.dtype, head_dim=int(q.shape[3]), block_m=block_m, block_n=block_n,
                         q_chunk_size=q_chunk_size, phase1_warps=phase1_warps, phase2_warps=phase2_warps,
                         phase1_stages=phase1_stages, phase2_stages=phase2_stages)
    return bn, qc, summary_dtype


def twopass_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    bias: Optional[torch.Tensor] = None,
    is_causal: bool = False,
    block_m: Optional[int] = None,
    block_n: Optional[int] = None,
    q_chunk_size: Optional[int] = None,
    summary_dtype: Optional[torch.dtype] = None,
    phase1_warps: Optional[int] = None,
    phase2_warps: Optional[int] = None,
    phase1_stages: Optional[int] = None,
    phase2_stages: Optional[int] = None,
    input_precision: Literal["auto", "ieee", "tf32", "tf32x3"] = "auto",
    algorithm: Literal["auto", "paper_scan"] = "auto",
) -> torch.Tensor:
    """Strict two-pass ELSA attention (reference attention.py:239-321).

    Phase 1 writes one exact ``(m, z, s)`` summary per K partition; Phase 2 merges
    the partition summaries of every row and emits ``s / z``.  q, k and v may be strided
    views (e.g. slices of a fused qkv projection): they are read in place when their
    strides allow.
    """
    return _twopass_attention(q, k, v, bias=bias, is_causal=is_causal, block_m=block_m, block_n=block_n,
                              q_chunk_size=q_chunk_size, summary_dtype=summary_dtype, phase1_warps=phase1_warps,
                              phase2_warps=phase2_warps, phase1_stages=phase1_stages, phase2_stages=phase2_stages,
                              input_precision=input_precision, algorithm=algorithm, out_bnhd=False)


def _twopass_attention(q, k, v, *, bias, is_causal, block_m, block_n, q_chunk_size, summary_dtype, phase1_warps,
                       phase2_warps, phase1_stages, phase2_stages, input_precision, algorithm, out_bnhd):
    """twopass_attention; ``out_bnhd`` returns a [B,H,N,D] view of [B,N,H,D] memory (for
    callers that go on to ``transpose(1, 2).reshape(B, N, H*D)``, which is then free)."""
    _check_qkv(q, k, v, "twopass_attention")
    if algorithm not in ("auto", "paper_scan"):
        raise ValueError("only algorithm='paper_scan' is available in this strict release")
    batch, heads, seq_len, head_dim = map(int, q.shape)
    if seq_len <= 0:
        return torch.empty_like(q)
    if head_dim > 128:
        raise ValueError("head_dim > 128 is not supported by the current Triton kernels")
    part, qc, sdt = _resolve_forward_options(
        q, block_m=block_m, block_n=block_n, q_chunk_size=q_chunk_size, summary_dtype=summary_dtype,
        phase1_warps=phase1_warps, phase2_warps=phase2_warps, phase1_stages=phase1_stages,
        phase2_stages=phase2_stages, input_precision=input_precision,
    )
    if batch * heads == 0:
        return torch.empty_like(q)
    if all(_operand(t) is t for t in (q, k, v)):
        # operands the kernels read in place: the C++ twin of _elsa_forward (elsa_torch.cpp,
        # attention_forward) keeps the host side of the call out of Python; same launches and bits
        meta = _canonical_bias(bias, batch=batch, heads=heads, seq_len=seq_len, device=q.device)
        return _lib.torch_module().attention_forward(q, k, v, meta.tensor, bool(is_causal), _lib.dtype_code(sdt),
                                                     int(part or 0), int(qc or 0), bool(out_bnhd))
    out, *_ = _elsa_forward(q, k, v, bias=bias, is_causal=is_causal, summary_dtype=sdt, partition_len=part,
                            q_chunk=qc, want_state=False, out_bnhd=out_bnhd)
    return out


def forward_plan(q: torch.Tensor, *, bias=None, is_causal=False, block_n=None, q_chunk_size=None,
                 summary_dtype=None) -> dict:
    """The HIP planner's routing for a forward call (partitions, widths, workspace bytes)."""
    lib = _lib.load()
    batch, heads, seq_len, head_dim = map(int, q.shape)
    sdt = summary_dtype or (torch.float32 if q.dtype == torch.float32 else q.dtype)
    qp = _pad_head_dim(q[:, :, :1]) if head_dim % 8 else q
    a = _lib.FwdArgs()
    a.q = a.k = a.v = a.out = 1  # plan queries never dereference pointers
    a.batch, a.heads, a.seq_len, a.head_dim = batch, heads, seq_len, int(qp.shape[-1])
    a.dtype = _lib.dtype_code(q.dtype)
    a.summary_dtype = _lib.dtype_code(sdt)
    a.is_causal = int(bool(is_causal))
    a.partition_len = int(block_n or 0)
    a.q_chunk = int(q_chunk_size or 0)
    plan = _lib.FwdPlan()
    _lib.check(lib.elsa_fwd_plan_get(ctypes.byref(a), ctypes.byref(plan)), "elsa_fwd_plan_get")
    return {"partitions": plan.partitions, "partition_len": plan.partition_len, "q_chunk": plan.q_chunk,
            "block_m": plan.block_m, "key_tile": plan.key_tile, "workspace_bytes": int(plan.workspace_bytes)}


def two_pass_explicit(q, k, v, *, is_causal=False, block_n=None, summary_dtype=None):
    """Run Phase 1 and Phase 2 as two separate library calls and return the HBM summaries.

    Structural check of the two-pass property (the reference's scripts/verify_2pass.py):
    returns ``(out, row_m, row_z, m_buf, z_buf, s_buf, plan)`` where the three summary
    buffers are views of the workspace Phase 1 wrote and Phase 2 read.
    """
    lib = _lib.load()
    _check_qkv(q, k, v, "two_pass_explicit")
    batch, heads, seq_len, head_dim = map(int, q.shape)
    if head_dim % 8:
        raise ValueError("two_pass_explicit needs head_dim % 8 == 0")
    sdt = summary_dtype or (torch.float32 if q.dtype == torch.float32 else q.dtype)
    q_c, k_c, v_c = q.contiguous(), k.contiguous(), v.contiguous()
    out = torch.empty_like(q_c)
    bh = batch * heads
    row_m = torch.empty((bh, seq_len), device=q.device, dtype=torch.float32)
    row_z = torch.empty_like(row_m)
    args = _make_fwd_args(q_c, k_c, v_c, out, row_m, row_z, _BiasMeta(None, 0, 0, 0, 0, False),
                          is_causal=is_causal, summary_dtype=sdt, partition_len=block_n, q_chunk=None,
                          scale=1.0 / math.sqrt(head_dim))
    plan = _lib.FwdPlan()
    _lib.check(lib.elsa_fwd_plan_get(ctypes.byref(args), ctypes.byref(plan)), "elsa_fwd_plan_get")
    if plan.q_chunk != seq_len:
        raise ValueError("two_pass_explicit expects a single q-chunk")
    ws = torch.zeros(int(plan.workspace_bytes), dtype=torch.uint8, device=q.device)
    args.workspace = ws.data_ptr()
    args.workspace_bytes = int(plan.workspace_bytes)
    stream = _lib.stream_handle(q.device)
    with torch.cuda.device(q.device):
        _lib.check(lib.elsa_phase1(ctypes.byref(args), 0, seq_len, stream), "elsa_phase1")
        torch.cuda.synchronize(q.device)
        rows = plan.partitions * bh * seq_len
        al = lambda x: (x + 255) // 256 * 256  # noqa: E731
        m_buf = ws[: rows * 4].view(torch.float32).view(plan.partitions, bh, seq_len).clone()
        z_buf = ws[al(rows * 4): al(rows * 4) + rows * 4].view(torch.float32).view(plan.partitions, bh,
                                                                                   seq_len).clone()
        s_off = 2 * al(rows * 4)
        esz = torch.empty((), dtype=sdt).element_size()
        s_buf = ws[s_off: s_off + rows * head_dim * esz].view(sdt).view(plan.partitions, bh, seq_len,
                                                                         head_dim).clone()
        _lib.check(lib.elsa_phase2(ctypes.byref(args), 0, seq_len, stream), "elsa_phase2")
    plan_d = {"partitions": plan.partitions, "partition_len": plan.partition_len, "q_chunk": plan.q_chunk}
    return out, row_m, row_z, m_buf, z_buf, s_buf, plan_d
