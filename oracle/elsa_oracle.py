"""CPU restatement of ELSA two-pass monoid-scan attention.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or as the timed CPU baseline). The product path (``elsa_amd``) never
imports it and fails loudly when its HIP library is missing.

What this restates (paths relative to the reference's
``src/elsa_twopass_clean/``):

* ``phase1_partition``: the per-K-partition ``(m, z, s)`` fold over 64-key
  micro-tiles, ``attention_parallel_scan.py:227-295`` (fp16, tiled) and
  ``:298-372`` (fp32, tiled); the non-tiled single-tile form
  ``:123-224`` is the same fold with one micro-tile.  The generic kernel
  ``attention.py:22-106`` (bias, causal, identity guard ``row_has``) is the
  ``generic=True`` branch.
* ``merge``: the monoid operator, ``attention_parallel_scan.py:55-60`` and
  ``:111-116``; identity ``(-inf, 0, 0)``.
* ``merge_tree``: Blelloch up-sweep with identity padding,
  ``attention_parallel_scan.py:67-120`` driven at ``:911-935``.
* ``merge_flat``: the d64 fast-path Phase 2, ``paper_scan_d64_kernel.cu:39-95``.
* ``scan_hillis_steele``: inclusive prefix scan, ``attention_parallel_scan.py:13-64``
  driven at ``:710-733``.
* ``finalize``: ``out = s/z`` with the ``z>0`` guard and row state,
  ``attention_parallel_scan.py:375-415`` / ``paper_scan_d64_kernel.cu:72-95``.
* ``backward``: ``attention_bwd.py:188-224`` (D, LSE2), ``:309-412`` (dq) and
  ``:415-527`` (dk/dv), including the casts at ``:404``, ``:512``, ``:514``.
* ``row_stats``: ``attention_bwd.py:227-306``.
* ``dbias``: ``attention_bwd.py:529-624`` and ``:973-1000`` (``mode="ref"``: the
  kernel's float32 arithmetic with its tf32x3 dots on fp32 inputs; default float64).
* ``matmul_tf32x3``: Triton's ``tl.dot(input_precision="tf32x3")`` (third-party, Triton
  unpinned by the reference's pyproject.toml:10-13; the 3xTF32 split: big*small + small*big +
  big*big of TF32 heads and tails, round-to-nearest-away TF32 conversion).
* ``reference_routing``: the reference's partition and micro-tile widths per call
  (``attention.py:175-226``, ``attention_bwd.py:130-158``,
  ``attention_parallel_scan.py:467-468``).

Rounding modes (``mode``):

* ``"fp64"``: every step in float64, no intermediate rounding.  This is the
  monoid algorithm itself, checked against ``exact_forward``/``exact_backward``.
* ``"ref"``: the reference's rounding points for the input dtype: fp16 inputs
  pre-scale ``q`` by ``log2(e)/sqrt(d)`` and round it to fp16 on the d64 fast
  path (``attention_parallel_scan.py:256-259``), round ``p`` to fp16 before
  ``p @ v`` (``:283``) and store ``s`` summaries in fp16 (``:478``); bf16 inputs
  go through the generic kernel (fp32 ``p @ v``, bf16 summaries); fp32 inputs
  stay in fp32 throughout.

Parity pins: the fp64 mode against the independent closed forms below and against
PyTorch's math SDPA with autograd in float64 (``tests/test_oracle.py``,
``tests/test_golden.py``); the ``ref`` mode from above, within the error magnitudes the
reference publishes (README.md:31, 78-79), and from below, by an independent hand fold
whose fp16 roundings of q, p, s and the output the oracle must reproduce, where deleting
any one of them fails (``tests/test_oracle_rounding.py``); monoid identity,
associativity, partition-count and merge-order invariance; finite differences of the
closed-form forward for the backward; the float32 dbias against the float64 one; the
routing table against the reference's values; and the committed fixtures under
``tests/golden/``.  ``oracle/torch_scan.py`` restates the same algorithm with torch CPU
operations for large shapes and is pinned against this module
(``tests/test_oracle_torch.py``).  No part of this module is "parity unpinned".
"""
from __future__ import annotations

import math
from typing import Optional

import numpy as np

LOG2E = 1.4426950408889634
NEG_INF = -np.inf


# --------------------------------------------------------------------------
# dtype emulation helpers
# --------------------------------------------------------------------------
def round_fp16(x: np.ndarray) -> np.ndarray:
    """Round to IEEE binary16 (nearest-even) and return float32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (nearest-even on the bit pattern), return float32."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    bits = a.view(np.uint32).astype(np.uint64)
    nan = np.isnan(a)
    lsb = (bits >> 16) & 1
    bits = (bits + 0x7FFF + lsb) & 0xFFFF0000
    out = bits.astype(np.uint32).view(np.float32)
    out = np.where(nan, np.float32(np.nan), out)
    return out.astype(np.float32)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "fp16":
        return round_fp16(x)
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "fp32":
        return np.asarray(x, dtype=np.float32)
    if dtype == "fp64":
        return np.asarray(x, dtype=np.float64)
    raise ValueError(dtype)


def _work_dtype(mode: str):
    return np.float64 if mode == "fp64" else np.float32


def _exp2(x):
    with np.errstate(invalid="ignore", over="ignore"):
        return np.exp2(x)


# --------------------------------------------------------------------------
# the monoid
# --------------------------------------------------------------------------
def identity(shape_rows: tuple, d: int, dt=np.float64):
    """Identity summary (-inf, 0, 0) (attention.py:91-100)."""
    m = np.full(shape_rows, NEG_INF, dtype=dt)
    z = np.zeros(shape_rows, dtype=dt)
    s = np.zeros(tuple(shape_rows) + (d,), dtype=dt)
    return m, z, s


def merge(a, b):
    """Monoid merge of two (m, z, s) summaries.

    attention_parallel_scan.py:55-60 / :111-116::

        m = max(m_a, m_b); alpha = z_a>0 ? exp2(m_a-m) : 0; beta = z_b>0 ? exp2(m_b-m) : 0
        z = z_a*alpha + z_b*beta; s = s_a*alpha + s_b*beta; m = z>0 ? m : -inf
    """
    m_a, z_a, s_a = a
    m_b, z_b, s_b = b
    m = np.maximum(m_a, m_b)
    with np.errstate(invalid="ignore"):
        alpha = np.where(z_a > 0, _exp2(m_a - m), 0.0).astype(m.dtype)
        beta = np.where(z_b > 0, _exp2(m_b - m), 0.0).astype(m.dtype)
    z = z_a * alpha + z_b * beta
    s = s_a * alpha[..., None] + s_b * beta[..., None]
    m = np.where(z > 0, m, NEG_INF).astype(m.dtype)
    return m, z, s


def merge_tree(parts):
    """Blelloch up-sweep over a list of summaries (attention_parallel_scan.py:67-120, :911-935).

    Level by level, ``out[j] = merge(in[2j], in[2j+1])`` with the identity standing
    in for a missing right operand (:102-109).
    """
    level = list(parts)
    while len(level) > 1:
        nxt = []
        for j in range(0, len(level), 2):
            if j + 1 < len(level):
                nxt.append(merge(level[j], level[j + 1]))
            else:
                m, z, s = level[j]
                nxt.append(merge(level[j], identity(m.shape, s.shape[-1], m.dtype)))
        level = nxt
    return level[0]


def merge_flat(parts):
    """Flat per-row merge of the d64 fast path (paper_scan_d64_kernel.cu:39-95).

    Max over partitions, weights ``w = z>0 ? exp2(m - M) : 0``, ``Z = sum z*w``,
    ``S = sum s*w``, ``M = -inf`` when ``Z == 0``.
    """
    ms = np.stack([p[0] for p in parts])
    zs = np.stack([p[1] for p in parts])
    ss = np.stack([p[2] for p in parts])
    big_m = ms.max(axis=0)
    with np.errstate(invalid="ignore"):
        w = np.where(zs > 0, _exp2(ms - big_m[None]), 0.0).astype(ms.dtype)
    big_z = (zs * w).sum(axis=0)
    big_s = (ss * w[..., None]).sum(axis=0)
    big_m = np.where(big_z > 0, big_m, NEG_INF).astype(ms.dtype)
    return big_m, big_z, big_s


def scan_hillis_steele(parts):
    """Inclusive Hillis-Steele prefix scan (attention_parallel_scan.py:13-64, :710-733).

    Step ``s``: ``out[j] = merge(in[j-s], in[j])`` for ``j >= s`` else ``in[j]``.
    Returns the list of all inclusive prefixes.
    """
    cur = list(parts)
    step = 1
    while step < len(cur):
        cur = [merge(cur[j - step], cur[j]) if j >= step else cur[j] for j in range(len(cur))]
        step *= 2
    return cur


def finalize(summary):
    """``out = z>0 ? s/z : 0`` plus row state (attention_parallel_scan.py:375-415)."""
    m, z, s = summary
    with np.errstate(invalid="ignore", divide="ignore"):
        out = np.where(z[..., None] > 0, s / np.where(z > 0, z, 1.0)[..., None], 0.0)
    row_m = np.where(z > 0, m, NEG_INF)
    return out, row_m, z


# --------------------------------------------------------------------------
# bias canonicalisation (attention.py:120-159)
# --------------------------------------------------------------------------
def canonical_bias(bias: Optional[np.ndarray], batch: int, heads: int, n: int) -> Optional[np.ndarray]:
    """Broadcast a bias of shape [N,N], [1|H,N,N] or [1|B,1|H,N,N] to [B,H,N,N]."""
    if bias is None:
        return None
    b = np.asarray(bias)
    if b.shape[-2:] != (n, n):
        raise ValueError(f"bias last dims must be {(n, n)}, got {tuple(b.shape)}")
    if b.ndim == 2:
        b = b.reshape(1, 1, n, n)
    elif b.ndim == 3:
        if b.shape[0] not in (1, heads):
            raise ValueError("3D bias must have shape [1,N,N] or [H,N,N]")
        b = b.reshape(1, b.shape[0], n, n)
    elif b.ndim == 4:
        if b.shape[0] not in (1, batch) or b.shape[1] not in (1, heads):
            raise ValueError("4D bias must broadcast as [B,H,N,N]")
    else:
        raise ValueError("bias must have shape [N,N], [H,N,N], or [B,H,N,N]")
    return np.broadcast_to(b, (batch, heads, n, n))


# --------------------------------------------------------------------------
# the reference's Phase-1 layout
# --------------------------------------------------------------------------
def reference_routing(n: int, d: int, dtype: str, *, training: bool = False, is_causal: bool = False,
                      has_bias: bool = False) -> tuple:
    """(part_len, micro): keys per K partition and per fold micro-tile in the reference.

    Partition width ``block_n``: inference ``_paper_scan_defaults`` (attention.py:175-226),
    training ``twopass_attention_with_state`` (attention_bwd.py:130-158).  The d64 fast
    path (``_can_use_d64_parallel_final``, attention_parallel_scan.py:418-440, never causal,
    :983-1018) folds 64-key micro-tiles when ``block_n > 512`` (:467-468) and one
    ``block_n`` tile otherwise (K3/K4, :123-224); the generic kernel (attention.py:22-106:
    bias, causal, bf16, D != 64) folds one ``block_n`` tile per program.
    """
    if dtype == "fp32":
        if d <= 64:
            bn = 256 if n <= 512 else (((n + 63) // 64) * 64 if n < 2048 else 2048)
        else:
            bn = 64
    elif not training and dtype == "fp16" and d == 64 and n >= 8192:
        bn = 2048
    else:
        bn = 256 if d <= 64 else 64
    fast = not has_bias and not is_causal and d == 64 and dtype in ("fp16", "fp32") and bn % 64 == 0
    micro = 64 if (fast and bn > 512) else bn
    return bn, micro


# --------------------------------------------------------------------------
# Phase 1
# --------------------------------------------------------------------------
def _scores(q_rows, k_tile, *, dtype: str, mode: str, generic: bool, scale: float, bias_tile, wd):
    """Scores in the base-2 domain for one micro-tile, following the reference path.

    fast path (attention_parallel_scan.py:256-259, :332): q pre-scaled by log2e/sqrt(d)
    (rounded to fp16 for fp16 inputs) and ``scores = q_s @ k^T``;
    generic path (attention.py:72, :77-90): ``(q @ k^T) * scale (+bias)`` then ``*log2e``.
    """
    if mode == "fp64" or generic:
        t = np.matmul(q_rows.astype(wd), np.swapaxes(k_tile.astype(wd), -1, -2)) * wd(scale)
        if bias_tile is not None:
            t = t + bias_tile.astype(wd)
        return t * wd(LOG2E)
    return np.matmul(q_rows, np.swapaxes(k_tile.astype(wd), -1, -2))


def _prescaled_q(q_rows, *, dtype: str, mode: str, generic: bool, scale: float, wd):
    if mode == "fp64" or generic:
        return q_rows.astype(wd)
    qs = q_rows.astype(np.float32) * np.float32(scale * LOG2E)
    return round_fp16(qs) if dtype == "fp16" else qs


def phase1_partition(
    q_rows: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    *,
    row_idx: np.ndarray,
    k_begin: int,
    k_end: int,
    n_ctx: int,
    is_causal: bool,
    bias: Optional[np.ndarray],
    dtype: str,
    mode: str,
    micro: int = 64,
    generic: Optional[bool] = None,
    summary_dtype: Optional[str] = None,
):
    """Fold one K partition ``[k_begin, k_end)`` into a running (m, z, s) summary.

    ``q_rows`` is [BH, R, D] (already restricted to the rows of interest), ``k``/``v``
    are [BH, N, D], ``bias`` (if given) is [BH, N, N].  The fold runs over micro-tiles
    of ``micro`` keys exactly like attention_parallel_scan.py:261-291: per tile
    ``local_m = max``, ``p = exp2(s - local_m)`` with the fully-masked guard (:281),
    ``local_z = sum p``, ``local_s = p @ v`` and the running merge with
    ``alpha = z_run>0 ? exp2(m_run - m_new) : 0`` (:285-290).  Masked keys (``>= n_ctx``
    or ``> row`` when causal) score ``-inf`` (:268-275; attention.py:73-75, :90).
    """
    wd = _work_dtype(mode)
    if generic is None:
        generic = bias is not None or is_causal or q_rows.shape[-1] != 64 or dtype == "bf16"
    d = q_rows.shape[-1]
    scale = 1.0 / math.sqrt(d)
    bh, r, _ = q_rows.shape
    qs = _prescaled_q(q_rows, dtype=dtype, mode=mode, generic=generic, scale=scale, wd=wd)
    m_run = np.full((bh, r), NEG_INF, dtype=wd)
    z_run = np.zeros((bh, r), dtype=wd)
    s_run = np.zeros((bh, r, d), dtype=wd)
    # p @ v takes p rounded to fp16 only for fp16 inputs with 16-bit summaries: the reference
    # launches its summary kernel with SUMMARY_DOT_FP32 = q.dtype != fp16 or summary_dtype ==
    # fp32 (attention_parallel_scan.py:701, :902) and then forms p @ v from the fp32 p
    # (attention.py:96-99); its fp16 d64 folds cast p to fp16 (attention_parallel_scan.py:167, :283)
    p_round = mode != "fp64" and dtype == "fp16" and (summary_dtype or dtype) != "fp32"
    for t0 in range(k_begin, k_end, micro):
        t1 = min(t0 + micro, k_end)
        kt = k[:, t0:t1]
        vt = v[:, t0:t1]
        bt = None if bias is None else bias[:, row_idx][:, :, t0:t1]
        sc = _scores(qs, kt, dtype=dtype, mode=mode, generic=generic, scale=scale, bias_tile=bt, wd=wd)
        kid = np.arange(t0, t1)
        valid = (kid[None, :] < n_ctx) & (row_idx[:, None] < n_ctx)
        if is_causal:
            valid = valid & (row_idx[:, None] >= kid[None, :])
        sc = np.where(valid[None], sc, NEG_INF).astype(wd)
        local_m = sc.max(axis=-1)
        finite = local_m > NEG_INF
        safe_m = np.where(finite, local_m, 0.0).astype(wd)
        p = np.where(valid[None] & finite[..., None], _exp2(sc - safe_m[..., None]), 0.0).astype(wd)
        local_z = p.sum(axis=-1)
        pv = round_fp16(p) if p_round else p
        local_s = np.matmul(pv, vt.astype(wd))
        m_new = np.maximum(m_run, local_m)
        safe_new = np.where(m_new > NEG_INF, m_new, 0.0).astype(wd)
        alpha = np.where(z_run > 0, _exp2(m_run - safe_new), 0.0).astype(wd)
        beta = np.where(finite, _exp2(local_m - safe_new), 0.0).astype(wd)
        z_run = z_run * alpha + local_z * beta
        s_run = s_run * alpha[..., None] + local_s * beta[..., None]
        m_run = np.where(z_run > 0, m_new, NEG_INF).astype(wd)
    return m_run, z_run, s_run


def _summary_round(s: np.ndarray, summary_dtype: str, mode: str) -> np.ndarray:
    if mode == "fp64":
        return s
    return round_to(s, summary_dtype).astype(np.float32)


def forward(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    *,
    bias: Optional[np.ndarray] = None,
    is_causal: bool = False,
    part_len: Optional[int] = None,
    micro: int = 64,
    dtype: Optional[str] = None,
    mode: str = "ref",
    merge_kind: str = "tree",
    summary_dtype: Optional[str] = None,
    rows: Optional[np.ndarray] = None,
):
    """Two-pass ELSA forward: Phase 1 per-partition summaries, Phase 2 merge.

    ``q, k, v``: [B, H, N, D] arrays (values already representable in ``dtype``).
    ``merge_kind``: ``"tree"`` (Blelloch up-sweep), ``"flat"`` (d64 fast path) or
    ``"scan"`` (Hillis-Steele inclusive scan, last prefix consumed, as the causal path
    does at attention_parallel_scan.py:745).  Returns ``out [B,H,R,D]`` and
    ``row_m, row_z [B*H, R]`` (base-2 state).  ``rows`` restricts the query rows.
    """
    if dtype is None:
        dtype = {np.dtype(np.float16): "fp16", np.dtype(np.float32): "fp32",
                 np.dtype(np.float64): "fp64"}[np.asarray(q).dtype]
    if summary_dtype is None:
        summary_dtype = dtype
    wd = _work_dtype(mode)
    b, h, n, d = q.shape
    bh = b * h
    qf = np.asarray(q, dtype=np.float32).reshape(bh, n, d)
    kf = np.asarray(k, dtype=np.float32).reshape(bh, n, d)
    vf = np.asarray(v, dtype=np.float32).reshape(bh, n, d)
    if mode == "fp64":
        qf, kf, vf = qf.astype(np.float64), kf.astype(np.float64), vf.astype(np.float64)
    bb = canonical_bias(bias, b, h, n)
    bb = None if bb is None else np.asarray(bb, dtype=wd).reshape(bh, n, n)
    if rows is None:
        rows = np.arange(n)
    rows = np.asarray(rows)
    # the d64 fast path (pre-scaled q) only under _can_use_d64_parallel_final's conditions
    # (attention_parallel_scan.py:418-440) and without a causal mask (:983-1018)
    generic = not (bb is None and not is_causal and d == 64 and dtype in ("fp16", "fp32")
                   and summary_dtype == dtype and (part_len is None or part_len % 64 == 0))
    if part_len is None:
        part_len = n
    parts = []
    for k0 in range(0, n, part_len):
        m, z, s = phase1_partition(
            qf[:, rows], kf, vf, row_idx=rows, k_begin=k0, k_end=min(n, k0 + part_len), n_ctx=n,
            is_causal=is_causal, bias=bb, dtype=dtype, mode=mode, micro=micro, generic=generic,
            summary_dtype=summary_dtype,
        )
        parts.append((m, z, _summary_round(s, summary_dtype, mode)))
    if merge_kind == "tree":
        total = merge_tree(parts)
    elif merge_kind == "flat":
        total = merge_flat(parts)
    elif merge_kind == "scan":
        total = scan_hillis_steele(parts)[-1]
    else:
        raise ValueError(merge_kind)
    out, row_m, row_z = finalize(total)
    out = out.reshape(b, h, len(rows), d)
    if mode != "fp64":
        out = round_to(out, dtype)
    return out, row_m.reshape(bh, len(rows)), row_z.reshape(bh, len(rows))


# --------------------------------------------------------------------------
# backward (attention_bwd.py)
# --------------------------------------------------------------------------
def preprocess(out: np.ndarray, dout: np.ndarray, row_m: np.ndarray, row_z: np.ndarray):
    """``D = rowsum(O*dO)`` (fp32) and ``LSE2 = m + log2(max(z,1e-30))`` (attention_bwd.py:188-224)."""
    b, h, n, d = out.shape
    o = np.asarray(out, dtype=np.float64).reshape(b * h, n, d)
    do = np.asarray(dout, dtype=np.float64).reshape(b * h, n, d)
    dd = (o * do).sum(-1)
    with np.errstate(divide="ignore"):
        lse = np.asarray(row_m, np.float64) + np.log2(np.maximum(np.asarray(row_z, np.float64), 1e-30))
    return dd, lse


def row_stats(q, k, *, bias=None, is_causal=False):
    """Online (m, z) recompute when no state is saved (attention_bwd.py:227-306), in fp64."""
    b, h, n, d = q.shape
    qf = np.asarray(q, np.float64).reshape(b * h, n, d)
    kf = np.asarray(k, np.float64).reshape(b * h, n, d)
    sc = np.matmul(qf, np.swapaxes(kf, -1, -2)) / math.sqrt(d)
    bb = canonical_bias(bias, b, h, n)
    if bb is not None:
        sc = sc + np.asarray(bb, np.float64).reshape(b * h, n, n)
    sc = sc * LOG2E
    if is_causal:
        sc = np.where(np.tril(np.ones((n, n), bool))[None], sc, NEG_INF)
    m = sc.max(-1)
    safe = np.where(m > NEG_INF, m, 0.0)
    z = _exp2(sc - safe[..., None]).sum(-1)
    return np.where(z > 0, m, NEG_INF), z


def backward(q, k, v, out, dout, row_m, row_z, *, bias=None, is_causal=False, dtype=None, mode="ref", rows=None):
    """Recompute backward (attention_bwd.py:309-527).

    ``p = exp2(s*log2e - LSE2)`` recomputed exactly from the saved state (:402, :511),
    ``dp = dO @ V^T``, ``ds = p*(dp - D)`` cast to the input dtype (:404, :514),
    ``dv = p(cast)^T @ dO`` (:512), ``dq = scale * ds @ K`` (:405-407),
    ``dk = scale * ds^T @ Q`` (:515-517).  Computed densely per head; the reference's
    tiling only reorders fp32 accumulation.  With ``rows`` (indices into N), ``q``,
    ``out``, ``dout``, ``row_m``, ``row_z`` hold only those query rows: dq is returned
    for them and dk/dv are the contributions of those rows.
    """
    if dtype is None:
        dtype = {np.dtype(np.float16): "fp16", np.dtype(np.float32): "fp32",
                 np.dtype(np.float64): "fp64"}[np.asarray(q).dtype]
    wd = _work_dtype(mode)
    rnd = (lambda x: x) if mode == "fp64" else (lambda x: round_to(x, dtype).astype(np.float32))
    b, h, r, d = q.shape
    n = k.shape[2]
    rows = np.arange(n) if rows is None else np.asarray(rows)
    bh = b * h
    scale = 1.0 / math.sqrt(d)
    qf = np.asarray(q, wd).reshape(bh, r, d)
    kf = np.asarray(k, wd).reshape(bh, n, d)
    vf = np.asarray(v, wd).reshape(bh, n, d)
    dof = np.asarray(dout, wd).reshape(bh, r, d)
    dd, lse = preprocess(out, dout, row_m, row_z)
    dd = dd.astype(wd)
    lse = lse.astype(wd)
    sc = np.matmul(qf, np.swapaxes(kf, -1, -2))
    bb = canonical_bias(bias, b, h, n)
    if bb is not None:
        sc = (sc * wd(scale) + np.asarray(bb, wd)[:, :, rows].reshape(bh, r, n)) * wd(LOG2E)
    else:
        sc = sc * wd(scale * LOG2E)
    valid = np.ones((r, n), bool)
    if is_causal:
        valid = rows[:, None] >= np.arange(n)[None, :]
    sc = np.where(valid[None], sc, NEG_INF)
    p = np.where(valid[None], _exp2(sc - lse[..., None]), 0.0).astype(wd)
    dp = np.matmul(dof, np.swapaxes(vf, -1, -2))
    ds = rnd(p * (dp - dd[..., None])).astype(wd)
    dv = np.matmul(np.swapaxes(rnd(p).astype(wd), -1, -2), dof)
    dq = np.matmul(ds, kf) * wd(scale)
    dk = np.matmul(np.swapaxes(ds, -1, -2), qf) * wd(scale)
    return dq.reshape(b, h, r, d), dk.reshape(b, h, n, d), dv.reshape(b, h, n, d)


def dbias(q, k, v, out, dout, row_m, row_z, *, bias, is_causal=False, mode="fp64"):
    """dbias = sum over broadcast dims of ``p*(dp - D)``.

    Follows the reference's dense-bias kernel (attention_bwd.py:529-624):
    ``p = exp2((q.k * scale + bias) * log2e - m) * (1 / max(z, 1e-30))``,
    ``dp = dO . v``, ``D = rowsum(out * dO)``, and the broadcast reduction of the dense
    fallback (:987-999).  ``mode="fp64"`` evaluates it in float64; ``mode="ref"`` in float32
    as the kernel does (fp32 dots, fp32 accumulation over the broadcast pairs).
    """
    b, h, n, d = q.shape
    bh = b * h
    if mode == "ref":
        return _dbias_ref32(q, k, v, out, dout, row_m, row_z, bias, is_causal)
    scale = 1.0 / math.sqrt(d)
    qf = np.asarray(q, np.float64).reshape(bh, n, d)
    kf = np.asarray(k, np.float64).reshape(bh, n, d)
    vf = np.asarray(v, np.float64).reshape(bh, n, d)
    dof = np.asarray(dout, np.float64).reshape(bh, n, d)
    dd, _ = preprocess(out, dout, row_m, row_z)
    bb = np.asarray(canonical_bias(bias, b, h, n), np.float64).reshape(bh, n, n)
    sc = np.matmul(qf, np.swapaxes(kf, -1, -2)) * scale + bb
    return _dbias_from_scores(sc, qf, kf, vf, dof, dd, row_m, row_z, b, h, n, np.shape(bias), is_causal, bb)


def round_tf32(x: np.ndarray) -> np.ndarray:
    """float32 -> TF32 (10-bit mantissa), round to nearest with ties away from zero, as float32."""
    a = np.ascontiguousarray(np.asarray(x, np.float32))
    bits = a.view(np.uint32).astype(np.uint64)
    bits = ((bits + 0x1000) & 0xFFFFE000).astype(np.uint32)
    return np.where(np.isfinite(a), bits.view(np.float32), a)


def matmul_tf32x3(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """``a @ b`` the way a Triton ``tl.dot(..., input_precision="tf32x3")`` forms it on fp32
    operands (the reference's fp32 default, attention.py:281-282): each operand split into a TF32
    head and a TF32 tail, and big*small + small*big + big*big summed -- the small*small term is
    dropped.  The three products are exact here (float64) and summed before one rounding to
    float32, so this carries the split's error but not the tensor cores' accumulation order."""
    a32 = np.asarray(a, np.float32)
    b32 = np.asarray(b, np.float32)
    ah = round_tf32(a32)
    bh = round_tf32(b32)
    al = round_tf32(a32 - ah)
    bl = round_tf32(b32 - bh)
    f64 = np.float64
    acc = np.matmul(ah.astype(f64), bl.astype(f64)) + np.matmul(al.astype(f64), bh.astype(f64))
    return (acc + np.matmul(ah.astype(f64), bh.astype(f64))).astype(np.float32)


def _dbias_ref32(q, k, v, out, dout, row_m, row_z, bias, is_causal):
    """The dense-bias kernel's float32 arithmetic (attention_bwd.py:596-614), per (b, h), then
    the broadcast dims summed in float32 in increasing (b, h) order.  fp32 inputs take the
    kernel's tf32x3 dots; 16-bit inputs exact products (``ieee``)."""
    b, h, n, d = q.shape
    f32 = np.float32
    dot = matmul_tf32x3 if np.asarray(q).dtype == np.float32 else (lambda x, y: np.matmul(x, y))
    qf, kf, vf, dof, of = (np.asarray(x, f32).reshape(b * h, n, d) for x in (q, k, v, dout, out))
    bb = np.asarray(canonical_bias(bias, b, h, n), f32).reshape(b * h, n, n)
    rm = np.asarray(row_m, f32).reshape(b * h, n)
    inv_z = f32(1.0) / np.maximum(np.asarray(row_z, f32).reshape(b * h, n), f32(1e-30))
    valid = np.tril(np.ones((n, n), bool)) if is_causal else np.ones((n, n), bool)
    sc = (dot(qf, np.swapaxes(kf, -1, -2)) * f32(1.0 / math.sqrt(d)) + bb) * f32(LOG2E)
    sc = np.where(valid[None], sc, f32(-np.inf))
    with np.errstate(invalid="ignore"):
        p = np.where(valid[None], _exp2(sc - rm[..., None]) * inv_z[..., None], f32(0)).astype(f32)
    dp = dot(dof, np.swapaxes(vf, -1, -2))
    dd = (of * dof).sum(-1, dtype=f32)
    ds = (p * (dp - dd[..., None])).astype(f32).reshape(b, h, n, n)
    shape = tuple(np.shape(bias))
    keep_b = len(shape) == 4 and shape[0] != 1
    keep_h = (len(shape) == 4 and shape[1] != 1) or (len(shape) == 3 and shape[0] != 1)
    acc = np.zeros((b if keep_b else 1, h if keep_h else 1, n, n), f32)
    for bi in range(b):
        for hi in range(h):
            acc[bi if keep_b else 0, hi if keep_h else 0] += ds[bi, hi]
    if len(shape) == 2:
        return acc[0, 0]
    if len(shape) == 3:
        return acc[0]
    return acc


def _dbias_from_scores(sc, qf, kf, vf, dof, dd, row_m, row_z, b, h, n, bias_shape, is_causal, bb):
    sc = sc * LOG2E
    valid = np.ones((n, n), bool)
    if is_causal:
        valid = np.tril(valid)
    rm = np.asarray(row_m, np.float64).reshape(b * h, n)
    rz = np.asarray(row_z, np.float64).reshape(b * h, n)
    inv_z = 1.0 / np.maximum(rz, 1e-30)
    p = np.where(valid[None], _exp2(np.where(valid[None], sc, NEG_INF) - rm[..., None]) * inv_z[..., None], 0.0)
    dp = np.matmul(dof, np.swapaxes(vf, -1, -2))
    ds = (p * (dp - dd[..., None])).reshape(b, h, n, n)
    shape = tuple(bias_shape)
    if len(shape) == 2:
        return ds.sum(axis=(0, 1))
    if len(shape) == 3:
        if shape[0] == 1:
            return ds.sum(axis=(0, 1))[None]
        return ds.sum(axis=0)
    grad = ds
    if shape[0] == 1:
        grad = grad.sum(axis=0, keepdims=True)
    if shape[1] == 1:
        grad = grad.sum(axis=1, keepdims=True)
    return grad


# --------------------------------------------------------------------------
# independent closed forms (fp64) -- not monoid code
# --------------------------------------------------------------------------
def exact_forward(q, k, v, *, bias=None, is_causal=False):
    """``softmax(q k^T/sqrt(d) + bias, causal) v`` in float64, plus base-2 row state."""
    b, h, n, d = q.shape
    qf = np.asarray(q, np.float64)
    kf = np.asarray(k, np.float64)
    vf = np.asarray(v, np.float64)
    sc = np.matmul(qf, np.swapaxes(kf, -1, -2)) / math.sqrt(d)
    bb = canonical_bias(bias, b, h, n)
    if bb is not None:
        sc = sc + np.asarray(bb, np.float64)
    if is_causal:
        sc = np.where(np.tril(np.ones((n, n), bool)), sc, NEG_INF)
    mx = sc.max(-1, keepdims=True)
    has = np.isfinite(mx)
    e = np.where(has, np.exp(sc - np.where(has, mx, 0.0)), 0.0)
    den = e.sum(-1, keepdims=True)
    pr = np.where(den > 0, e / np.where(den > 0, den, 1.0), 0.0)
    out = np.matmul(pr, vf)
    row_m = (mx[..., 0] * LOG2E).reshape(b * h, n)
    row_z = den[..., 0].reshape(b * h, n)
    row_m = np.where(row_z > 0, row_m, NEG_INF)
    return out, row_m, row_z


def exact_backward(q, k, v, dout, *, bias=None, is_causal=False):
    """Closed-form softmax-attention gradients in float64 (dq, dk, dv, dscores)."""
    b, h, n, d = q.shape
    qf = np.asarray(q, np.float64)
    kf = np.asarray(k, np.float64)
    vf = np.asarray(v, np.float64)
    do = np.asarray(dout, np.float64)
    scale = 1.0 / math.sqrt(d)
    sc = np.matmul(qf, np.swapaxes(kf, -1, -2)) * scale
    bb = canonical_bias(bias, b, h, n)
    if bb is not None:
        sc = sc + np.asarray(bb, np.float64)
    if is_causal:
        sc = np.where(np.tril(np.ones((n, n), bool)), sc, NEG_INF)
    mx = sc.max(-1, keepdims=True)
    e = np.exp(sc - mx)
    pr = e / e.sum(-1, keepdims=True)
    dv = np.matmul(np.swapaxes(pr, -1, -2), do)
    dp = np.matmul(do, np.swapaxes(vf, -1, -2))
    ds = pr * (dp - (dp * pr).sum(-1, keepdims=True))
    dq = np.matmul(ds, kf) * scale
    dk = np.matmul(np.swapaxes(ds, -1, -2), qf) * scale
    return dq, dk, dv, ds


def make_inputs(shape, seed: int, *, dtype: str = "fp32", with_dout: bool = False, q_scale=1.0, k_scale=1.0,
                dout_scale=1.0):
    """Seeded N(0,1) inputs drawn in the order q, k, v[, dO] with numpy's PCG64.

    Values are rounded to ``dtype`` and returned as float16 (fp16) or float32 arrays.
    """
    rng = np.random.default_rng(seed)
    arrs = [rng.standard_normal(shape).astype(np.float32) for _ in range(4 if with_dout else 3)]
    scales = [q_scale, k_scale, 1.0, dout_scale][: len(arrs)]
    arrs = [a * np.float32(s) for a, s in zip(arrs, scales)]
    if dtype == "fp16":
        arrs = [a.astype(np.float16) for a in arrs]
    elif dtype == "bf16":
        arrs = [round_bf16(a) for a in arrs]
    return arrs
