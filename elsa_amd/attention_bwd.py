"""Training API: forward with row state, recompute backward, autograd and dbias.

Mirrors the reference's attention_bwd.py (``twopass_attention_with_state``
:77-185, ``twopass_attention_backward`` :661-839, ``_TwopassAttentionAutograd``
:842-905, ``_dense_bias_backward`` :908-1000, ``twopass_attention_train``
:1003-1030).  All device work goes to libelsa_hip.so: ``elsa_fwd`` (with row
state), ``elsa_row_stats`` when the caller has no state, ``elsa_bwd`` (D/LSE2
preprocess, dq kernel, dk/dv kernel) and ``elsa_dbias``.

Backward tile knobs (``block_m``, ``block_n``, ``num_warps``, ``num_stages``)
are validated like the reference and otherwise ignored.
"""
from __future__ import annotations

import ctypes
import math
from typing import Literal, Optional

import torch

from . import _lib
from .attention import (
    _canonical_bias,
    _check_qkv,
    _elsa_forward,
    _operand,
    _resolve_forward_options,
    _resolve_precision,
    _validate_warps,
)


def twopass_attention_with_state(
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
    return_contiguous_inputs: bool = False,
) -> tuple[torch.Tensor, ...]:
    """Training forward: ``(out, row_m, row_z[, q_c, k_c, v_c])`` with base-2 row state."""
    return _with_state(q, k, v, bias=bias, is_causal=is_causal, block_m=block_m, block_n=block_n,
                       q_chunk_size=q_chunk_size, summary_dtype=summary_dtype, phase1_warps=phase1_warps,
                       phase2_warps=phase2_warps, phase1_stages=phase1_stages, phase2_stages=phase2_stages,
                       input_precision=input_precision, algorithm=algorithm,
                       return_contiguous_inputs=return_contiguous_inputs, out_bnhd=False)


def _with_state(q, k, v, *, bias=None, is_causal=False, block_m=None, block_n=None, q_chunk_size=None,
                summary_dtype=None, phase1_warps=None, phase2_warps=None, phase1_stages=None, phase2_stages=None,
                input_precision="auto", algorithm="auto", return_contiguous_inputs=False, out_bnhd=False,
                exact_row_max=True):
    """twopass_attention_with_state; ``out_bnhd`` returns out as a [B,H,N,D] view of [B,N,H,D] memory.
    The training autograd functions pass ``exact_row_max=False``: their row state only feeds the
    backward, which reads row_m + log2(row_z)."""
    _check_qkv(q, k, v, "twopass_attention_with_state")
    batch, heads, seq_len, head_dim = map(int, q.shape)
    if seq_len > 0:
        part, qc, sdt = _state_options(q, block_m=block_m, block_n=block_n, q_chunk_size=q_chunk_size,
                                       summary_dtype=summary_dtype, phase1_warps=phase1_warps,
                                       phase2_warps=phase2_warps, phase1_stages=phase1_stages,
                                       phase2_stages=phase2_stages, input_precision=input_precision,
                                       algorithm=algorithm)
    else:
        empty_state = torch.empty((batch * heads, 0), device=q.device, dtype=torch.float32)
        out_empty = torch.empty_like(q)
        if return_contiguous_inputs:
            return out_empty, empty_state, empty_state, q.contiguous(), k.contiguous(), v.contiguous()
        return out_empty, empty_state, empty_state
    out, row_m, row_z, q_c, k_c, v_c = _elsa_forward(
        q, k, v, bias=bias, is_causal=is_causal, summary_dtype=sdt, partition_len=part, q_chunk=qc, want_state=True,
        out_bnhd=out_bnhd, exact_row_max=exact_row_max,
    )
    if return_contiguous_inputs:
        return out, row_m, row_z, q_c.contiguous(), k_c.contiguous(), v_c.contiguous()
    return out, row_m, row_z


def _state_options(q, *, block_m, block_n, q_chunk_size, summary_dtype, phase1_warps, phase2_warps, phase1_stages,
                   phase2_stages, input_precision, algorithm):
    """Validation and routing of twopass_attention_with_state (attention_bwd.py:77-185): returns
    (partition_len, q_chunk, summary_dtype)."""
    if int(q.shape[-1]) > 128:
        raise ValueError("head_dim > 128 is not supported by the current Triton kernels")
    if algorithm not in ("auto", "paper_scan"):
        raise ValueError("only algorithm='paper_scan' is available in this strict release")
    return _resolve_forward_options(
        q, block_m=block_m, block_n=block_n, q_chunk_size=q_chunk_size, summary_dtype=summary_dtype,
        phase1_warps=phase1_warps, phase2_warps=phase2_warps, phase1_stages=phase1_stages,
        phase2_stages=phase2_stages, input_precision=input_precision,
    )


def _bwd_args(q_c, k_c, v_c, out_c, do_c, row_m, row_z, dq, dk, dv, bias_meta, *, is_causal, scale):
    """elsa_bwd_args for [B,H,N,D] tensors, which may be strided views (their layouts are passed)."""
    batch, heads, seq_len, head_dim = map(int, q_c.shape)
    a = _lib.BwdArgs()
    a.q, a.k, a.v = q_c.data_ptr(), k_c.data_ptr(), v_c.data_ptr()
    a.out, a.dout = _lib.ptr(out_c), _lib.ptr(do_c)
    a.row_m, a.row_z = _lib.ptr(row_m), _lib.ptr(row_z)
    a.dq, a.dk, a.dv = _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv)
    a.q_layout, a.k_layout, a.v_layout = (_lib.layout_of(t) for t in (q_c, k_c, v_c))
    if out_c is not None:
        a.out_layout, a.dout_layout = _lib.layout_of(out_c), _lib.layout_of(do_c)
    if dq is not None:
        a.dq_layout, a.dk_layout, a.dv_layout = (_lib.layout_of(t) for t in (dq, dk, dv))
    a.bias = _lib.bias_desc(bias_meta.tensor, (bias_meta.stride_b, bias_meta.stride_h, bias_meta.stride_q,
                                               bias_meta.stride_k))
    a.batch, a.heads, a.seq_len, a.head_dim = batch, heads, seq_len, head_dim
    a.dtype = _lib.dtype_code(q_c.dtype)
    a.is_causal = 1 if is_causal else 0
    a.scale = float(scale)
    return a


def _attach_workspace(lib, args, device):
    nbytes = int(lib.elsa_bwd_workspace_bytes(ctypes.byref(args)))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    args.workspace = ws.data_ptr()
    args.workspace_bytes = nbytes
    return ws


def _row_stats(q_c, k_c, bias_meta, *, is_causal, scale):
    lib = _lib.load()
    bh, n = q_c.shape[0] * q_c.shape[1], q_c.shape[2]
    row_m = torch.empty((bh, n), dtype=torch.float32, device=q_c.device)
    row_z = torch.empty_like(row_m)
    args = _bwd_args(q_c, k_c, k_c, None, None, None, None, None, None, None, bias_meta, is_causal=is_causal,
                     scale=scale)
    with torch.cuda.device(q_c.device):
        _lib.check(lib.elsa_row_stats(ctypes.byref(args), row_m.data_ptr(), row_z.data_ptr(),
                                      _lib.stream_handle(q_c.device)), "elsa_row_stats")
    return row_m, row_z


def twopass_attention_backward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    out: torch.Tensor,
    grad_out: torch.Tensor,
    *,
    bias: Optional[torch.Tensor] = None,
    is_causal: bool = False,
    block_m: Optional[int] = None,
    block_n: Optional[int] = None,
    num_warps: Optional[int] = None,
    num_stages: Optional[int] = None,
    input_precision: Literal["auto", "ieee", "tf32", "tf32x3"] = "auto",
    row_m: Optional[torch.Tensor] = None,
    row_z: Optional[torch.Tensor] = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Recompute backward: ``(dq, dk, dv)`` (reference attention_bwd.py:661-839). No dbias."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must have shape [B,H,N,D]")
    if q.shape != k.shape or q.shape != v.shape or q.shape != out.shape or q.shape != grad_out.shape:
        raise ValueError("q, k, v, out, and grad_out must have identical shapes")
    if q.device.type != "cuda":
        raise ValueError("twopass_attention_backward currently requires CUDA tensors")
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("supported dtypes are fp16, bf16, and fp32")
    batch, heads, seq_len, head_dim = map(int, q.shape)
    if head_dim > 128:
        raise ValueError("head_dim > 128 is not supported by the current Triton kernels")
    if seq_len <= 0:
        return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    _resolve_precision(input_precision, q.dtype)
    if block_m is not None:
        max(16, int(block_m))
    if block_n is not None:
        max(16, int(block_n))
    if num_warps is not None:
        _validate_warps("num_warps", num_warps)
    for t in (k, v, out, grad_out):
        if t.dtype != q.dtype:
            raise ValueError("q, k, v, out, and grad_out must share one dtype")
    bh = batch * heads
    bias_meta = _canonical_bias(bias, batch=batch, heads=heads, seq_len=seq_len, device=q.device)
    if row_m is not None and row_z is not None:
        if row_m.shape != (bh, seq_len) or row_z.shape != (bh, seq_len):
            raise ValueError("row_m and row_z must have shape [B*H,N]")
        row_m = row_m.contiguous().float()
        row_z = row_z.contiguous().float()
    return _backward(q, k, v, out, grad_out, bias_meta, is_causal=is_causal, row_m=row_m, row_z=row_z)


def _backward(q, k, v, out, grad_out, bias_meta, *, is_causal, row_m, row_z, grads=None, dbias_out=None):
    """dq, dk, dv on the HIP library.  Operands are read in place when their layout allows
    (``_operand``); ``grads`` optionally names [B,H,N,D] (possibly strided) tensors to write
    dq, dk, dv into, such as views of one fused qkv gradient.  With ``dbias_out`` (fp32
    [bias_batch, bias_heads, N, N]) the same call also writes the bias gradient
    (``elsa_bwd_dbias``: dS from the dk/dv kernel, summed over the broadcast dims)."""
    head_dim = int(q.shape[-1])
    scale = 1.0 / math.sqrt(head_dim)
    lib = _lib.load()
    q_c, k_c, v_c, out_c, do_c = (_operand(t) for t in (q, k, v, out, grad_out))
    if row_m is None or row_z is None:
        row_m, row_z = _row_stats(q_c, k_c, bias_meta, is_causal=is_causal, scale=scale)
    padded = q_c.shape[-1] != head_dim
    if grads is None or padded:
        dq, dk, dv = (torch.empty(t.shape, dtype=t.dtype, device=t.device) for t in (q_c, k_c, v_c))
    else:
        dq, dk, dv = grads
    args = _bwd_args(q_c, k_c, v_c, out_c, do_c, row_m, row_z, dq, dk, dv, bias_meta, is_causal=is_causal,
                     scale=scale)
    if dbias_out is None:
        ws = _attach_workspace(lib, args, q.device)
        with torch.cuda.device(q.device):
            _lib.check(lib.elsa_bwd(ctypes.byref(args), _lib.stream_handle(q.device)), "elsa_bwd")
    else:
        bias_b, bias_h = int(dbias_out.shape[0]), int(dbias_out.shape[1])
        nbytes = int(lib.elsa_bwd_dbias_workspace_bytes(ctypes.byref(args), bias_b, bias_h))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
        args.workspace, args.workspace_bytes = ws.data_ptr(), nbytes
        with torch.cuda.device(q.device):
            _lib.check(lib.elsa_bwd_dbias(ctypes.byref(args), dbias_out.data_ptr(), bias_b, bias_h,
                                          _lib.stream_handle(q.device)), "elsa_bwd_dbias")
    del ws
    if padded:
        dq, dk, dv = (t[..., :head_dim] for t in (dq, dk, dv))
        if grads is not None:
            for dst, src in zip(grads, (dq, dk, dv)):
                dst.copy_(src)
            return grads
        dq, dk, dv = (t.contiguous() for t in (dq, dk, dv))
    return dq, dk, dv


def _dense_bias_backward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    out: torch.Tensor,
    grad_out: torch.Tensor,
    *,
    bias: torch.Tensor,
    is_causal: bool,
    row_m: Optional[torch.Tensor] = None,
    row_z: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """dbias summed over the bias's broadcast dims (reference attention_bwd.py:908-1000).

    One HIP kernel covers every bias rank ([N,N], [1|H,N,N], [1|B,1|H,N,N]): it
    accumulates ``p*(dp - D)`` over the broadcast (b, h) pairs of each output tile
    without materialising the [B,H,N,N] score tensor, so the reference's 64M-element
    dense fallback limit does not apply.
    """
    batch, heads, seq_len, head_dim = map(int, q.shape)
    lib = _lib.load()
    meta = _canonical_bias(bias, batch=batch, heads=heads, seq_len=seq_len, device=q.device)
    bias_b = 1 if meta.stride_b == 0 else batch
    bias_h = 1 if meta.stride_h == 0 else heads
    scale = 1.0 / math.sqrt(head_dim)
    q_c, k_c, v_c, out_c, do_c = (_operand(t) for t in (q, k, v, out, grad_out))
    if row_m is None or row_z is None:
        row_m, row_z = _row_stats(q_c, k_c, meta, is_causal=is_causal, scale=scale)
    dbias = torch.empty((bias_b, bias_h, seq_len, seq_len), dtype=torch.float32, device=q.device)
    args = _bwd_args(q_c, k_c, v_c, out_c, do_c, row_m.contiguous(), row_z.contiguous(), None, None, None, meta,
                     is_causal=is_causal, scale=scale)
    nbytes = int(lib.elsa_dbias_workspace_bytes(ctypes.byref(args), bias_b, bias_h))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    args.workspace, args.workspace_bytes = ws.data_ptr(), nbytes
    with torch.cuda.device(q.device):
        _lib.check(lib.elsa_dbias(ctypes.byref(args), dbias.data_ptr(), bias_b, bias_h,
                                  _lib.stream_handle(q.device)), "elsa_dbias")
    del ws
    return dbias.reshape(bias.shape).to(dtype=bias.dtype)


class _TwopassAttentionAutograd(torch.autograd.Function):
    """Forward with row state, recompute backward (reference attention_bwd.py:842-905).

    The reference saves contiguous copies of q, k, v; here the inputs are saved as given
    and the backward kernels read them in place whenever their layout allows."""

    @staticmethod
    def forward(ctx, q, k, v, bias, is_causal, fwd_kwargs, bwd_kwargs, out_bnhd=False):
        out, row_m, row_z = _with_state(q, k, v, bias=bias, is_causal=is_causal, out_bnhd=out_bnhd,
                                        exact_row_max=False, **fwd_kwargs)
        _save(ctx, (q, k, v), out, bias, row_m, row_z, is_causal, bwd_kwargs)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        q, k, v, out, bias, row_m, row_z = _saved(ctx)
        if ctx.bias_requires_grad:  # dq, dk, dv and dbias in one call
            meta, d32 = _dbias_target(q, bias)
            dq, dk, dv = _backward(q, k, v, out, grad_out, meta, is_causal=ctx.is_causal, row_m=row_m, row_z=row_z,
                                   dbias_out=d32)
            return dq, dk, dv, d32.reshape(bias.shape).to(bias.dtype), None, None, None, None
        dq, dk, dv = twopass_attention_backward(
            q, k, v, out, grad_out, bias=bias, is_causal=ctx.is_causal, row_m=row_m, row_z=row_z, **ctx.bwd_kwargs
        )
        return dq, dk, dv, None, None, None, None, None


class _TwopassQkvAutograd(torch.autograd.Function):
    """The same on a fused [B, N, 3, H, D] qkv projection (the timm drop-ins' layout).

    q, k, v are read as strided views of it, out is written as [B, N, H, D] memory, and
    the backward writes dq, dk, dv straight into one [B, N, 3, H, D] gradient, so neither
    pass makes a transposing copy."""

    @staticmethod
    def forward(ctx, qkv, bias, is_causal, fwd_kwargs, bwd_kwargs):
        q, k, v = qkv.permute(2, 0, 3, 1, 4).unbind(0)
        out, row_m, row_z = _with_state(q, k, v, bias=bias, is_causal=is_causal, out_bnhd=True, exact_row_max=False,
                                        **fwd_kwargs)
        _save(ctx, (qkv,), out, bias, row_m, row_z, is_causal, bwd_kwargs)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        qkv, out, bias, row_m, row_z = _saved(ctx)
        q, k, v = qkv.permute(2, 0, 3, 1, 4).unbind(0)
        batch, heads, seq_len, _ = map(int, q.shape)
        dqkv = torch.empty_like(qkv, memory_format=torch.contiguous_format)
        grads = dqkv.permute(2, 0, 3, 1, 4).unbind(0)
        if ctx.bias_requires_grad:  # dq, dk, dv and dbias in one call
            meta, d32 = _dbias_target(q, bias)
            _backward(q, k, v, out, grad_out, meta, is_causal=ctx.is_causal, row_m=row_m, row_z=row_z, grads=grads,
                      dbias_out=d32)
            return dqkv, d32.reshape(bias.shape).to(bias.dtype), None, None, None
        meta = _canonical_bias(bias, batch=batch, heads=heads, seq_len=seq_len, device=q.device)
        _backward(q, k, v, out, grad_out, meta, is_causal=ctx.is_causal, row_m=row_m, row_z=row_z, grads=grads)
        return dqkv, None, None, None, None


def _save(ctx, inputs, out, bias, row_m, row_z, is_causal, bwd_kwargs):
    ctx.has_bias = bias is not None
    saved_bias = bias if bias is not None else torch.empty(0, device=out.device)
    ctx.save_for_backward(*inputs, out, saved_bias, row_m, row_z)
    ctx.bias_requires_grad = bool(bias is not None and bias.requires_grad)
    ctx.is_causal = bool(is_causal)
    ctx.bwd_kwargs = dict(bwd_kwargs)


def _saved(ctx):
    *inputs, out, saved_bias, row_m, row_z = ctx.saved_tensors
    return (*inputs, out, saved_bias if ctx.has_bias else None, row_m, row_z)


def _dbias_target(q, bias):
    """The bias's canonical view and an fp32 gradient of its [1|B, 1|H, N, N] shape."""
    batch, heads, seq_len, _ = map(int, q.shape)
    meta = _canonical_bias(bias, batch=batch, heads=heads, seq_len=seq_len, device=q.device)
    bias_b = 1 if meta.stride_b == 0 else batch
    bias_h = 1 if meta.stride_h == 0 else heads
    return meta, torch.empty((bias_b, bias_h, seq_len, seq_len), dtype=torch.float32, device=q.device)


def _split_train_kwargs(bwd_block_m, bwd_block_n, bwd_num_warps, bwd_num_stages, bwd_input_precision, fwd_kwargs):
    if bwd_input_precision == "auto":
        fwd_input_precision = fwd_kwargs.get("input_precision")
        if fwd_input_precision in ("ieee", "tf32", "tf32x3"):
            bwd_input_precision = fwd_input_precision
    bwd_kwargs = {
        "block_m": bwd_block_m,
        "block_n": bwd_block_n,
        "num_warps": bwd_num_warps,
        "num_stages": bwd_num_stages,
        "input_precision": bwd_input_precision,
    }
    return {key: value for key, value in bwd_kwargs.items() if value is not None}


def qkv_attention_train(qkv: torch.Tensor, *, bias: Optional[torch.Tensor] = None, is_causal: bool = False,
                        bwd_block_m: Optional[int] = None, bwd_block_n: Optional[int] = None,
                        bwd_num_warps: Optional[int] = None, bwd_num_stages: Optional[int] = None,
                        bwd_input_precision: Literal["auto", "ieee", "tf32", "tf32x3"] = "auto",
                        **fwd_kwargs) -> torch.Tensor:
    """``twopass_attention_train`` on q, k, v = ``qkv[:, :, 0..2]`` of a [B, N, 3, H, D] tensor.

    Returns the [B, H, N, D] output as a view of [B, N, H, D] memory; the gradient of qkv
    comes back in qkv's own layout.  Same numerics as ``twopass_attention_train``."""
    if qkv.dim() != 5 or qkv.shape[2] != 3:
        raise ValueError("qkv must have shape [B,N,3,H,D]")
    bwd_kwargs = _split_train_kwargs(bwd_block_m, bwd_block_n, bwd_num_warps, bwd_num_stages, bwd_input_precision,
                                     fwd_kwargs)
    q, k, v = qkv.permute(2, 0, 3, 1, 4).unbind(0)
    _check_qkv(q, k, v, "qkv_attention_train")
    _check_bwd_kwargs(bwd_kwargs, qkv.dtype)
    batch, heads, seq_len, head_dim = map(int, q.shape)
    if seq_len > 0 and head_dim % 8 == 0 and qkv.is_contiguous() and qkv.data_ptr() % 16 == 0:
        # the whole call in C++ (elsa_torch.cpp): no Python between the launches of either pass
        part, qc, sdt = _state_options(q, **_fwd_options(fwd_kwargs, "qkv_attention_train"))
        meta = _canonical_bias(bias, batch=batch, heads=heads, seq_len=seq_len, device=q.device)
        return _lib.torch_module().qkv_attention_train(qkv, meta.tensor, bool(is_causal), _lib.dtype_code(sdt),
                                                       int(part or 0), int(qc or 0))
    return _TwopassQkvAutograd.apply(qkv, bias, is_causal, dict(fwd_kwargs), bwd_kwargs)


def _check_bwd_kwargs(bwd_kwargs, dtype):
    """The validation twopass_attention_backward applies to its tile knobs (attention_bwd.py:698-716)."""
    _resolve_precision(bwd_kwargs.get("input_precision", "auto"), dtype)
    for key in ("block_m", "block_n"):
        if bwd_kwargs.get(key) is not None:
            max(16, int(bwd_kwargs[key]))
    if bwd_kwargs.get("num_warps") is not None:
        _validate_warps("num_warps", bwd_kwargs["num_warps"])
    if bwd_kwargs.get("num_stages") is not None:
        max(1, int(bwd_kwargs["num_stages"]))


def _train_bnhd(q, k, v, *, bias=None, is_causal=False, bwd_block_m=None, bwd_block_n=None, bwd_num_warps=None,
                bwd_num_stages=None, bwd_input_precision="auto", **fwd_kwargs):
    """twopass_attention_train with out returned as a [B,H,N,D] view of [B,N,H,D] memory."""
    bwd_kwargs = _split_train_kwargs(bwd_block_m, bwd_block_n, bwd_num_warps, bwd_num_stages, bwd_input_precision,
                                     fwd_kwargs)
    return _train(q, k, v, bias, is_causal, dict(fwd_kwargs), bwd_kwargs, True)


_FWD_OPTION_DEFAULTS = dict(block_m=None, block_n=None, q_chunk_size=None, summary_dtype=None, phase1_warps=None,
                            phase2_warps=None, phase1_stages=None, phase2_stages=None, input_precision="auto",
                            algorithm="auto")


def _fwd_options(fwd_kwargs, who):
    unknown = set(fwd_kwargs) - set(_FWD_OPTION_DEFAULTS)
    if unknown:
        raise TypeError(f"{who}() got unexpected keyword arguments {sorted(unknown)}")
    opts = dict(_FWD_OPTION_DEFAULTS)
    opts.update(fwd_kwargs)
    return opts


def _train(q, k, v, bias, is_causal, fwd_kwargs, bwd_kwargs, out_bnhd):
    """Autograd forward + recompute backward.  Inputs the kernels read in place take the C++
    autograd function (elsa_torch.cpp); the rest (head dims that need a padded copy, empty
    sequences) the Python one."""
    _check_qkv(q, k, v, "twopass_attention_with_state")
    batch, heads, seq_len, _ = map(int, q.shape)
    if seq_len > 0 and all(_operand(t) is t for t in (q, k, v)):
        part, qc, sdt = _state_options(q, **_fwd_options(fwd_kwargs, "twopass_attention_train"))
        _check_bwd_kwargs(bwd_kwargs, q.dtype)
        meta = _canonical_bias(bias, batch=batch, heads=heads, seq_len=seq_len, device=q.device)
        return _lib.torch_module().attention_train(q, k, v, meta.tensor, bool(is_causal), _lib.dtype_code(sdt),
                                                   int(part or 0), int(qc or 0), bool(out_bnhd))
    return _TwopassAttentionAutograd.apply(q, k, v, bias, is_causal, dict(fwd_kwargs), bwd_kwargs, out_bnhd)


def twopass_attention_train(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    bias: Optional[torch.Tensor] = None,
    is_causal: bool = False,
    bwd_block_m: Optional[int] = None,
    bwd_block_n: Optional[int] = None,
    bwd_num_warps: Optional[int] = None,
    bwd_num_stages: Optional[int] = None,
    bwd_input_precision: Literal["auto", "ieee", "tf32", "tf32x3"] = "auto",
    **fwd_kwargs,
) -> torch.Tensor:
    """Autograd wrapper: two-pass forward with state plus recompute backward (attention_bwd.py:1003-1030)."""
    bwd_kwargs = _split_train_kwargs(bwd_block_m, bwd_block_n, bwd_num_warps, bwd_num_stages, bwd_input_precision,
                                     fwd_kwargs)
    return _train(q, k, v, bias, is_causal, dict(fwd_kwargs), bwd_kwargs, False)
