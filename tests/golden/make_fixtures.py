"""Write the golden vectors of the two-pass attention path (``tests/golden/*.npz``).

Run from the repository root: ``python tests/golden/make_fixtures.py``.

The reference ships no golden vectors (its tests compare against SDPA at run time,
``tests/test_attention.py:16-25``) and cannot run in this image, so these files hold
the CPU oracle's outputs at the reference's rounding points (``mode="ref"``) next to
the fp64 closed form, on small seeded inputs drawn on the CPU.  The shapes are the
ones the reference's tests and benchmarks exercise, shrunk so that each file stays
small: a 64-token fp32 call, the NEEDS_MASK lengths 197 and 257
(``attention_parallel_scan.py:472``) on the fp16 d64 fast path with several
partitions and on the causal path, a bf16 call through the generic kernel, and a
Swin window with relative-position bias and the shifted-window mask
(``timm_dropin.py:85-90``), whose dbias the reference reduces at
``attention_bwd.py:908-1000``.

Each ``.npz`` holds:

* inputs ``q, k, v, dout`` (float16 for fp16, float32 otherwise; bf16 values are
  float32 arrays rounded to bf16) and ``bias`` when the case has one;
* ``meta``: a JSON string (dtype, causal flag, partition width, seed);
* the reference restatement: ``out`` (rounded to the input dtype), ``row_m``, ``row_z``
  (base-2 state), ``dq, dk, dv`` (fp32 accumulators; the reference stores them in the
  input dtype), ``dbias`` (fp64 reduction);
* the closed form: ``out_exact, row_m_exact, row_z_exact, dq_exact, dk_exact,
  dv_exact, dbias_exact`` (float64 for fp32 cases, float32 otherwise).

``tests/test_golden.py`` checks these files against the closed form and the oracle on
the CPU, and the HIP path against them on the GPU.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import elsa_oracle as O  # noqa: E402

# name: (B, H, N, D), dtype, causal, part_len, bias kind, seed
CASES = {
    "fp32_b1h2n64d32_full": ((1, 2, 64, 32), "fp32", False, None, None, 1234),
    "fp16_b1h1n197d64_full_p64": ((1, 1, 197, 64), "fp16", False, 64, None, 2026),
    "fp16_b1h1n257d32_causal": ((1, 1, 257, 32), "fp16", True, None, None, 2027),
    "fp32_b1h1n97d32_causal": ((1, 1, 97, 32), "fp32", True, None, None, 2028),
    "bf16_b1h1n100d32_full": ((1, 1, 100, 32), "bf16", False, None, None, 2029),
    "fp16_swin_b2h2n49d32_bias": ((2, 2, 49, 32), "fp16", False, None, "swin", 7),
}


def swin_bias(b: int, h: int, n: int, seed: int) -> np.ndarray:
    """A [B, H, 49, 49] window bias: a relative-position-style N(0, 0.5^2) table and, on
    the odd windows, the shifted-window mask's -100 on keys from 30 on."""
    rng = np.random.default_rng(seed)
    bias = (rng.standard_normal((b, h, n, n)) * 0.5).astype(np.float32)
    bias[1::2, :, :, 30:] -= 100.0
    return bias


def compute(case):
    shape, dt, causal, part_len, bias_kind, seed = case
    q, k, v, do = O.make_inputs(shape, seed=seed, dtype=dt, with_dout=True, dout_scale=1.0)
    bias = swin_bias(shape[0], shape[1], shape[2], seed) if bias_kind == "swin" else None
    out, rm, rz = O.forward(q, k, v, bias=bias, is_causal=causal, part_len=part_len, dtype=dt, mode="ref")
    dq, dk, dv = O.backward(q, k, v, out, do, rm, rz, bias=bias, is_causal=causal, dtype=dt, mode="ref")
    qf, kf, vf, dof = (np.asarray(x, np.float32) for x in (q, k, v, do))
    eo, em, ez = O.exact_forward(qf, kf, vf, bias=bias, is_causal=causal)
    eq, ek, ev, _ = O.exact_backward(qf, kf, vf, dof, bias=bias, is_causal=causal)
    ex = np.float64 if dt == "fp32" else np.float32
    rec = {
        "q": q, "k": k, "v": v, "dout": do,
        "out": np.asarray(out, np.float32), "row_m": np.asarray(rm, np.float32),
        "row_z": np.asarray(rz, np.float32),
        "dq": np.asarray(dq, np.float32), "dk": np.asarray(dk, np.float32), "dv": np.asarray(dv, np.float32),
        "out_exact": eo.astype(ex), "row_m_exact": np.asarray(em, np.float64),
        "row_z_exact": np.asarray(ez, np.float64),
        "dq_exact": eq.astype(ex), "dk_exact": ek.astype(ex), "dv_exact": ev.astype(ex),
    }
    if bias is not None:
        rec["bias"] = bias
        rec["dbias"] = O.dbias(qf, kf, vf, out, dof, rm, rz, bias=bias, is_causal=causal).astype(np.float32)
        rec["dbias_exact"] = O.dbias(qf, kf, vf, eo, dof, em, ez, bias=bias, is_causal=causal).astype(ex)
    meta = {"shape": list(shape), "dtype": dt, "causal": causal, "part_len": part_len,
            "bias": bias_kind, "seed": seed, "dout_scale": 1.0}
    rec["meta"] = np.array(json.dumps(meta, sort_keys=True))
    return rec


def main() -> None:
    for name, case in CASES.items():
        rec = compute(case)
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **rec)
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
