"""Pure-PyTorch (CPU) restatement of ELSA's two-pass monoid scan, forward and backward.

TEST INFRASTRUCTURE AND THE TIMED CPU BASELINE ONLY.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import
this module: as the checker of the HIP path at large shapes, and as the "pure-PyTorch
restatement of the reference's monoid scan" that the CPU baseline times.  The product
(``elsa_amd``) never imports it.

It is the same algorithm, with the same rounding points, as ``oracle/elsa_oracle.py``
(the numpy restatement, whose docstring lists the reference lines each step follows),
written with torch CPU operations so that the large configurations -- N up to 65536,
the B8 H3 ViT lengths -- finish in seconds: BLAS and element-wise kernels run on every
host thread, and query rows are processed in chunks so memory stays bounded.

* ``forward``: Phase 1 per K partition (the running ``(m, z, s)`` fold over micro-tiles,
  attention_parallel_scan.py:227-295 / :298-372, generic attention.py:22-106), the
  partition summaries rounded to ``summary_dtype`` (:476-478), Phase 2 as the Blelloch
  up-sweep (:67-120) or the flat per-row merge (paper_scan_d64_kernel.cu:39-95), then
  ``out = s/z`` with the ``z > 0`` guard and the base-2 row state (:375-415).
* ``backward``: D and LSE2 (attention_bwd.py:188-224), p recomputed from the saved
  state, ``ds`` and ``p`` cast to the input dtype before the dQ/dK and dV products
  (:404, :512, :514).
* ``exact_*``: float64 closed forms (softmax attention and its gradients), chunked.

Pins (``tests/test_oracle.py``): ``forward``/``backward`` against ``elsa_oracle`` in
both modes on causal, biased, ragged and multi-partition cases, and the ``exact_*``
functions against ``elsa_oracle.exact_*`` (themselves checked against finite
differences and math SDPA).
"""
from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np
import torch

LOG2E = 1.4426950408889634
NEG_INF = float("-inf")


def _t(x, dt=torch.float32) -> torch.Tensor:
    if isinstance(x, torch.Tensor):
        return x.detach().to("cpu", dt)
    return torch.from_numpy(np.ascontiguousarray(np.asarray(x, dtype=np.float64))).to(dt)


def round_to(x: torch.Tensor, dtype: str) -> torch.Tensor:
    """Round float32 values to ``dtype`` (nearest-even) and return float32."""
    if dtype == "fp16":
        return x.to(torch.float16).to(torch.float32)
    if dtype == "bf16":
        return x.to(torch.bfloat16).to(torch.float32)
    return x


def _canonical_bias(bias, b: int, h: int, n: int, dt) -> Optional[torch.Tensor]:
    """[N,N], [1|H,N,N] or [1|B,1|H,N,N] broadcast to a [B*H, N, N] view (attention.py:120-159)."""
    if bias is None:
        return None
    t = _t(bias, dt)
    if t.dim() == 2:
        t = t.view(1, 1, n, n)
    elif t.dim() == 3:
        t = t.view(1, t.shape[0], n, n)
    return t.expand(b, h, n, n).reshape(b * h, n, n)


# --------------------------------------------------------------------------- monoid
def merge(a, b):
    """(m, z, s) merge (attention_parallel_scan.py:55-60): alpha/beta are 0 for an empty side."""
    m_a, z_a, s_a = a
    m_b, z_b, s_b = b
    m = torch.maximum(m_a, m_b)
    safe = torch.where(m > NEG_INF, m, torch.zeros_like(m))
    alpha = torch.where(z_a > 0, torch.exp2(m_a - safe), torch.zeros_like(m))
    beta = torch.where(z_b > 0, torch.exp2(m_b - safe), torch.zeros_like(m))
    z = z_a * alpha + z_b * beta
    s = s_a * alpha[..., None] + s_b * beta[..., None]
    m = torch.where(z > 0, m, torch.full_like(m, NEG_INF))
    return m, z, s


def merge_tree(parts):
    """Blelloch up-sweep, identity on the right past the end (attention_parallel_scan.py:67-120)."""
    level = list(parts)
    while len(level) > 1:
        nxt = []
        for j in range(0, len(level), 2):
            if j + 1 < len(level):
                nxt.append(merge(level[j], level[j + 1]))
            else:
                m, z, s = level[j]
                nxt.append(merge(level[j], (torch.full_like(m, NEG_INF), torch.zeros_like(z), torch.zeros_like(s))))
        level = nxt
    return level[0]


def merge_flat(parts):
    """Flat per-row merge of the d64 fast path (paper_scan_d64_kernel.cu:39-95)."""
    ms = torch.stack([p[0] for p in parts])
    zs = torch.stack([p[1] for p in parts])
    ss = torch.stack([p[2] for p in parts])
    big = ms.max(0).values
    safe = torch.where(big > NEG_INF, big, torch.zeros_like(big))
    w = torch.where(zs > 0, torch.exp2(ms - safe[None]), torch.zeros_like(zs))
    z = (zs * w).sum(0)
    s = (ss * w[..., None]).sum(0)
    return torch.where(z > 0, big, torch.full_like(big, NEG_INF)), z, s


# --------------------------------------------------------------------------- Phase 1
def _fold_partition(qs, q_raw, k, v, bias, rows, k_begin, k_end, n, *, causal, generic, p_round, micro, scale, wd):
    """Running (m, z, s) over the micro-tiles of keys [k_begin, k_end) for query rows ``rows``.

    Fast path (attention_parallel_scan.py:256-259, :332): ``scores = q_s @ k^T`` with q
    prescaled by log2(e)/sqrt(d); generic (attention.py:72, :77-90): ``(q @ k^T) * scale``,
    ``+ bias``, ``* log2(e)``.  Masked keys score -inf; ``p = exp2(s - local_m)`` with the
    fully-masked guard (:281); p rounded to fp16 before ``p @ v`` on fp16 inputs (:283).
    Micro-tiles with no valid key for any of these rows are the identity and skipped.
    """
    bh, r, d = q_raw.shape
    m_run = torch.full((bh, r), NEG_INF, dtype=wd)
    z_run = torch.zeros((bh, r), dtype=wd)
    s_run = torch.zeros((bh, r, d), dtype=wd)
    row_max = int(rows.max()) if r else -1
    for t0 in range(k_begin, k_end, micro):
        if causal and t0 > row_max:
            break
        t1 = min(t0 + micro, k_end)
        kt = k[:, t0:t1]
        if generic:
            sc = torch.matmul(q_raw, kt.transpose(1, 2)) * torch.tensor(scale, dtype=wd)
            if bias is not None:
                sc = sc + bias[:, rows][:, :, t0:t1]
            sc = sc * torch.tensor(LOG2E, dtype=wd)
        else:
            sc = torch.matmul(qs, kt.transpose(1, 2))
        kid = torch.arange(t0, t1)
        valid = (kid[None, :] < n) & (rows[:, None] < n)
        if causal:
            valid = valid & (rows[:, None] >= kid[None, :])
        sc = torch.where(valid[None], sc, torch.full_like(sc, NEG_INF))
        local_m = sc.max(-1).values
        finite = local_m > NEG_INF
        safe_m = torch.where(finite, local_m, torch.zeros_like(local_m))
        p = torch.where(valid[None] & finite[..., None], torch.exp2(sc - safe_m[..., None]), torch.zeros_like(sc))
        local_z = p.sum(-1)
        pv = round_to(p, "fp16") if p_round else p
        local_s = torch.matmul(pv, v[:, t0:t1])
        m_new = torch.maximum(m_run, local_m)
        safe_new = torch.where(m_new > NEG_INF, m_new, torch.zeros_like(m_new))
        alpha = torch.where(z_run > 0, torch.exp2(m_run - safe_new), torch.zeros_like(m_run))
        beta = torch.where(finite, torch.exp2(local_m - safe_new), torch.zeros_like(m_run))
        z_run = z_run * alpha + local_z * beta
        s_run = s_run * alpha[..., None] + local_s * beta[..., None]
        m_run = torch.where(z_run > 0, m_new, torch.full_like(m_new, NEG_INF))
    return m_run, z_run, s_run


def forward(q, k, v, *, bias=None, is_causal: bool = False, part_len: Optional[int] = None, micro: int = 64,
            dtype: str, mode: str = "ref", merge_kind: str = "tree", summary_dtype: Optional[str] = None,
            rows: Optional[Sequence[int]] = None, row_chunk: int = 4096):
    """Two-pass forward for query rows ``rows`` (default all).

    ``q, k, v``: [B, H, N, D] (numpy or torch; values representable in ``dtype``).
    Returns torch float tensors ``out [B, H, R, D]`` (rounded to ``dtype`` in ``ref``
    mode), ``row_m, row_z [B*H, R]`` (base-2 state, -inf / 0 for empty rows).
    """
    wd = torch.float64 if mode == "fp64" else torch.float32
    summary_dtype = summary_dtype or dtype
    b, h, n, d = q.shape
    bh = b * h
    qf = _t(q, wd).reshape(bh, n, d)
    kf = _t(k, wd).reshape(bh, n, d)
    vf = _t(v, wd).reshape(bh, n, d)
    bb = _canonical_bias(bias, b, h, n, wd)
    rows_t = torch.arange(n) if rows is None else torch.as_tensor(np.asarray(rows), dtype=torch.int64)
    generic = not (bb is None and not is_causal and d == 64 and dtype in ("fp16", "fp32")
                   and summary_dtype == dtype and (part_len is None or part_len % 64 == 0))
    if mode == "fp64":
        generic = True
    scale = 1.0 / math.sqrt(d)
    # p rounded to fp16 for p @ v only without SUMMARY_DOT_FP32 (fp16 inputs, 16-bit summaries:
    # attention_parallel_scan.py:701, :902; attention.py:96-99)
    p_round = mode != "fp64" and dtype == "fp16" and summary_dtype != "fp32"
    part_len = part_len or n
    outs, ms, zs = [], [], []
    for r0 in range(0, len(rows_t), row_chunk):
        rr = rows_t[r0:r0 + row_chunk]
        q_raw = qf[:, rr]
        qs = None
        if not generic:
            qs = q_raw * torch.tensor(scale * LOG2E, dtype=torch.float32)
            if dtype == "fp16":
                qs = round_to(qs, "fp16")
        parts = []
        for k0 in range(0, n, part_len):
            m, z, s = _fold_partition(qs, q_raw, kf, vf, bb, rr, k0, min(n, k0 + part_len), n, causal=is_causal,
                                      generic=generic, p_round=p_round, micro=micro, scale=scale, wd=wd)
            if mode != "fp64":
                s = round_to(s, summary_dtype)
            parts.append((m, z, s))
        if merge_kind == "tree":
            m, z, s = merge_tree(parts)
        elif merge_kind == "flat":
            m, z, s = merge_flat(parts)
        else:
            raise ValueError(merge_kind)
        out = torch.where(z[..., None] > 0, s / torch.where(z > 0, z, torch.ones_like(z))[..., None],
                          torch.zeros_like(s))
        if mode != "fp64":
            out = round_to(out, dtype)
        outs.append(out)
        ms.append(torch.where(z > 0, m, torch.full_like(m, NEG_INF)))
        zs.append(z)
    out = torch.cat(outs, 1).reshape(b, h, len(rows_t), d)
    return out, torch.cat(ms, 1), torch.cat(zs, 1)


# --------------------------------------------------------------------------- backward
def backward(q, k, v, out, dout, row_m, row_z, *, bias=None, is_causal: bool = False, dtype: str,
             mode: str = "ref", rows: Optional[Sequence[int]] = None, row_chunk: int = 1024, need_kv: bool = True):
    """Recompute backward (attention_bwd.py:309-527).

    ``out``, ``dout``, ``row_m``, ``row_z`` cover all N rows ([B,H,N,D] / [B*H, N]).
    ``p = exp2(s*log2e - LSE2)`` with ``LSE2 = m + log2(max(z, 1e-30))``, ``dp = dO V^T``,
    ``ds = p (dp - D)`` cast to the input dtype (:404, :514), ``dv += cast(p)^T dO``
    (:512), ``dq = scale ds K``, ``dk = scale ds^T Q``.  With ``rows`` only those query
    rows are processed: dq is theirs, dk/dv are their contributions.  Returns torch
    tensors dq [B,H,R,D], dk, dv [B,H,N,D] (dk/dv None when ``need_kv`` is False).
    """
    wd = torch.float64 if mode == "fp64" else torch.float32
    rnd = (lambda x: x) if mode == "fp64" else (lambda x: round_to(x, dtype))
    b, h, n, d = q.shape
    bh = b * h
    scale = 1.0 / math.sqrt(d)
    qf = _t(q, wd).reshape(bh, n, d)
    kf = _t(k, wd).reshape(bh, n, d)
    vf = _t(v, wd).reshape(bh, n, d)
    of = _t(out, torch.float64).reshape(bh, n, d)
    dof64 = _t(dout, torch.float64).reshape(bh, n, d)
    dof = dof64.to(wd)
    # D = rowsum(O * dO) and LSE2 (attention_bwd.py:188-224), formed in float64, used in wd
    dd = (of * dof64).sum(-1).to(wd)
    rm = _t(row_m, torch.float64).reshape(bh, n)
    rz = _t(row_z, torch.float64).reshape(bh, n)
    lse = (rm + torch.log2(torch.clamp(rz, min=1e-30))).to(wd)
    bb = _canonical_bias(bias, b, h, n, wd)
    rows_t = torch.arange(n) if rows is None else torch.as_tensor(np.asarray(rows), dtype=torch.int64)
    c_sl = torch.tensor(scale * LOG2E, dtype=wd)
    dq_parts = []
    dk = torch.zeros((bh, n, d), dtype=wd) if need_kv else None
    dv = torch.zeros((bh, n, d), dtype=wd) if need_kv else None
    kid = torch.arange(n)
    for r0 in range(0, len(rows_t), row_chunk):
        rr = rows_t[r0:r0 + row_chunk]
        sc = torch.matmul(qf[:, rr], kf.transpose(1, 2))
        if bb is not None:
            sc = (sc * torch.tensor(scale, dtype=wd) + bb[:, rr]) * torch.tensor(LOG2E, dtype=wd)
        else:
            sc = sc * c_sl
        p = torch.exp2(sc - lse[:, rr][..., None])
        if is_causal:
            p = torch.where((rr[:, None] >= kid[None, :])[None], p, torch.zeros_like(p))
        dp = torch.matmul(dof[:, rr], vf.transpose(1, 2))
        ds = rnd(p * (dp - dd[:, rr][..., None]))
        dq_parts.append(torch.matmul(ds, kf) * torch.tensor(scale, dtype=wd))
        if need_kv:
            dv += torch.matmul(rnd(p).transpose(1, 2), dof[:, rr])
            dk += torch.matmul(ds.transpose(1, 2), qf[:, rr])
    dq = torch.cat(dq_parts, 1).reshape(b, h, len(rows_t), d)
    if need_kv:
        dk = (dk * torch.tensor(scale, dtype=wd)).reshape(b, h, n, d)
        dv = dv.reshape(b, h, n, d)
    return dq, dk, dv


def backward_key_columns(q, k, v, out, dout, row_m, row_z, keys, *, bias=None, is_causal: bool = False,
                         dtype: str, mode: str = "ref", row_chunk: int = 2048):
    """dk, dv of the key columns ``keys`` only, with the same per-element arithmetic as
    ``backward`` (every query row contributes): ``[B, H, len(keys), D]`` torch tensors."""
    wd = torch.float64 if mode == "fp64" else torch.float32
    rnd = (lambda x: x) if mode == "fp64" else (lambda x: round_to(x, dtype))
    b, h, n, d = q.shape
    bh = b * h
    scale = 1.0 / math.sqrt(d)
    qf, kf, vf = (_t(x, wd).reshape(bh, n, d) for x in (q, k, v))
    dof64 = _t(dout, torch.float64).reshape(bh, n, d)
    dof = dof64.to(wd)
    dd = (_t(out, torch.float64).reshape(bh, n, d) * dof64).sum(-1).to(wd)
    rm = _t(row_m, torch.float64).reshape(bh, n)
    rz = _t(row_z, torch.float64).reshape(bh, n)
    lse = (rm + torch.log2(torch.clamp(rz, min=1e-30))).to(wd)
    bb = _canonical_bias(bias, b, h, n, wd)
    keys_t = torch.as_tensor(np.asarray(keys), dtype=torch.int64)
    kj, vj = kf[:, keys_t], vf[:, keys_t]
    dk = torch.zeros((bh, len(keys_t), d), dtype=wd)
    dv = torch.zeros((bh, len(keys_t), d), dtype=wd)
    for r0 in range(0, n, row_chunk):
        rr = torch.arange(r0, min(n, r0 + row_chunk))
        sc = torch.matmul(qf[:, rr], kj.transpose(1, 2))
        if bb is not None:
            sc = (sc * torch.tensor(scale, dtype=wd) + bb[:, rr][:, :, keys_t]) * torch.tensor(LOG2E, dtype=wd)
        else:
            sc = sc * torch.tensor(scale * LOG2E, dtype=wd)
        p = torch.exp2(sc - lse[:, rr][..., None])
        if is_causal:
            p = torch.where((rr[:, None] >= keys_t[None, :])[None], p, torch.zeros_like(p))
        dp = torch.matmul(dof[:, rr], vj.transpose(1, 2))
        ds = rnd(p * (dp - dd[:, rr][..., None]))
        dv += torch.matmul(rnd(p).transpose(1, 2), dof[:, rr])
        dk += torch.matmul(ds.transpose(1, 2), qf[:, rr])
    return (dk * torch.tensor(scale, dtype=wd)).reshape(b, h, -1, d), dv.reshape(b, h, -1, d)


# --------------------------------------------------------------------------- closed forms (float64)
def _exact_scores(qr, kf, rr, n, scale, bb, causal):
    sc = torch.matmul(qr, kf.transpose(1, 2)) * scale
    if bb is not None:
        sc = sc + bb[:, rr]
    if causal:
        sc = torch.where((rr[:, None] >= torch.arange(n)[None, :])[None], sc, torch.full_like(sc, NEG_INF))
    return sc


def exact_forward(q, k, v, *, bias=None, is_causal: bool = False, rows=None, row_chunk: int = 1024):
    """``softmax(q k^T / sqrt(d) + bias, causal) v`` in float64 for rows ``rows``, plus the
    base-2 row state.  Returns out [B,H,R,D], row_m, row_z [B*H, R] (torch float64)."""
    b, h, n, d = q.shape
    bh = b * h
    qf, kf, vf = (_t(x, torch.float64).reshape(bh, n, d) for x in (q, k, v))
    bb = _canonical_bias(bias, b, h, n, torch.float64)
    rows_t = torch.arange(n) if rows is None else torch.as_tensor(np.asarray(rows), dtype=torch.int64)
    scale = 1.0 / math.sqrt(d)
    outs, ms, zs = [], [], []
    for r0 in range(0, len(rows_t), row_chunk):
        rr = rows_t[r0:r0 + row_chunk]
        sc = _exact_scores(qf[:, rr], kf, rr, n, scale, bb, is_causal)
        mx = sc.max(-1, keepdim=True).values
        has = torch.isfinite(mx)
        e = torch.where(has, torch.exp(sc - torch.where(has, mx, torch.zeros_like(mx))), torch.zeros_like(sc))
        den = e.sum(-1, keepdim=True)
        pr = torch.where(den > 0, e / torch.where(den > 0, den, torch.ones_like(den)), torch.zeros_like(e))
        outs.append(torch.matmul(pr, vf))
        zs.append(den[..., 0])
        ms.append(torch.where(den[..., 0] > 0, mx[..., 0] * LOG2E, torch.full_like(den[..., 0], NEG_INF)))
    return torch.cat(outs, 1).reshape(b, h, len(rows_t), d), torch.cat(ms, 1), torch.cat(zs, 1)


def exact_backward(q, k, v, dout, *, bias=None, is_causal: bool = False, rows=None, keys=None,
                   row_chunk: int = 1024):
    """Closed-form gradients in float64: dq for the query rows ``rows`` (default all) and
    dk, dv for the keys ``keys`` (default all; every query row contributes to them).
    ``dS = P (dP - D)`` with ``D_i = sum_j P_ij dP_ij = dO_i . O_i``, ``dq = dS K / sqrt(d)``,
    ``dk = dS^T Q / sqrt(d)``, ``dv = P^T dO``; dP is formed only for the requested rows and
    key columns.  Returns torch float64 (dq [B,H,R,D], dk, dv [B,H,K,D])."""
    b, h, n, d = q.shape
    bh = b * h
    qf, kf, vf, dof = (_t(x, torch.float64).reshape(bh, n, d) for x in (q, k, v, dout))
    bb = _canonical_bias(bias, b, h, n, torch.float64)
    scale = 1.0 / math.sqrt(d)
    want_rows = torch.arange(n) if rows is None else torch.as_tensor(np.asarray(rows), dtype=torch.int64)
    keys_t = torch.arange(n) if keys is None else torch.as_tensor(np.asarray(keys), dtype=torch.int64)
    row_pos = torch.full((n,), -1, dtype=torch.int64)
    row_pos[want_rows] = torch.arange(len(want_rows))
    dq = torch.zeros((bh, len(want_rows), d), dtype=torch.float64)
    dk = torch.zeros((bh, len(keys_t), d), dtype=torch.float64)
    dv = torch.zeros((bh, len(keys_t), d), dtype=torch.float64)
    vk = vf[:, keys_t]
    # without key columns only the requested rows need scoring
    row_list = want_rows if len(keys_t) == 0 else torch.arange(n)
    for r0 in range(0, len(row_list), row_chunk):
        rr = row_list[r0:r0 + row_chunk]
        sc = _exact_scores(qf[:, rr], kf, rr, n, scale, bb, is_causal)
        mx = sc.max(-1, keepdim=True).values
        e = torch.exp(sc - mx)
        pr = e / e.sum(-1, keepdim=True)
        dd = (dof[:, rr] * torch.matmul(pr, vf)).sum(-1, keepdim=True)
        sel = row_pos[rr] >= 0
        if bool(sel.any()):
            ps = pr[:, sel]
            ds = ps * (torch.matmul(dof[:, rr][:, sel], vf.transpose(1, 2)) - dd[:, sel])
            dq[:, row_pos[rr][sel]] = torch.matmul(ds, kf) * scale
        if len(keys_t) == 0:
            continue
        pk = pr[:, :, keys_t]
        dsk = pk * (torch.matmul(dof[:, rr], vk.transpose(1, 2)) - dd)
        dk += torch.matmul(dsk.transpose(1, 2), qf[:, rr]) * scale
        dv += torch.matmul(pk.transpose(1, 2), dof[:, rr])
    return (dq.reshape(b, h, len(want_rows), d), dk.reshape(b, h, len(keys_t), d),
            dv.reshape(b, h, len(keys_t), d))
