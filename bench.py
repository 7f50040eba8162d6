"""Benchmark of the ELSA two-pass attention hot path on one MI355X.

One step = the training-path attention of BASELINE config 2 at the north-star shape, through
twopass_attention_train as the reference's benchmarks/bench_bwd.py times it: two-pass forward
keeping the row state the backward reads (Phase 1 fold on MFMA -> HBM summaries -> Phase 2
merge) plus the exact-recompute backward (preprocess, dq, dk/dv), B=1 H=8 N=16384 d=64 fp16,
non-causal, synthetic N(0,1) q/k/v/dO (seed 2026) resident in HBM.

Prints ONE JSON line.  ``value`` is the algorithmic fwd+bwd throughput
(3.5 * 4*B*H*N^2*d flop per step, recompute not counted).  ``kernels`` holds each
kernel's HIP-event average on the launch stream; ``roofline`` is computed for the
kernel with the largest share of the step.  ``baseline_configs`` times the other shapes of
BASELINE configs 2 and 3 (B1 H8 d64: fp16 and fp32 at 1K-64K, causal fp16 at 197-32K) the same
way, each with its training-step wall clock and a sampled fp64 check.  ``cpu_baseline`` times BASELINE config 1
(B1 H8 N1024 d64 fp32 forward) through the pure-PyTorch restatement of the reference's
monoid scan (oracle/torch_scan.py) on the host cores, with a row sample of this step's
own work beside it.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "ELSA attn fwd/bwd TFLOP/s + %MFMA peak (B1 H8 d64 16K fp16); ViT-T img/s"
PEAK_TFLOPS = {"fp16": 2516.6, "bf16": 2516.6, "fp32": 157.3}
HBM_GBPS = 8000.0


def _args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=25)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--heads", type=int, default=8)
    ap.add_argument("--seq", type=int, default=16384)
    ap.add_argument("--dim", type=int, default=64)
    ap.add_argument("--dtype", choices=["fp16", "bf16", "fp32"], default="fp16")
    ap.add_argument("--causal", action="store_true")
    ap.add_argument("--block-n", type=int, default=None, help="K-partition width (default: planner)")
    ap.add_argument("--fill", choices=["randn", "sign", "zeros", "const"], default="randn",
                    help="input values: N(0,1) (the benchmark), their signs, zeros or 0.5 everywhere; the "
                         "kernels run the same instructions for all four, which isolates the data-dependent clock")
    ap.add_argument("--cpu-baseline", dest="cpu_baseline", action="store_true", default=True)
    ap.add_argument("--no-cpu-baseline", dest="cpu_baseline", action="store_false")
    ap.add_argument("--cpu-rows", type=int, default=2048, help="query rows of the north-star CPU sample")
    ap.add_argument("--traffic-file", default=os.path.join(ROOT, "profiles", "traffic_north_star.json"))
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="after timing, run one copy kernel over this many MiB (HBM-counter calibration)")
    # BASELINE configs 4 and 5: ViT-T at 224/512/1024/2048 px and Swin-T at 224/384/512 px, batch 8
    ap.add_argument("--vit-img", type=int, nargs="*", default=[224, 512, 1024, 2048],
                    help="ViT-Tiny image sizes for the img/s fields in --dtype (empty: skip)")
    ap.add_argument("--swin-img", type=int, nargs="*", default=[224, 384, 512],
                    help="Swin-Tiny image sizes for the img/s fields in --dtype (empty: skip)")
    # the same models in fp32 as second fields (BASELINE config 4's four ViT sizes in fp32 too)
    ap.add_argument("--vit-img-fp32", type=int, nargs="*", default=[224, 512, 1024, 2048],
                    help="ViT-Tiny image sizes of the fp32 fields (empty: skip)")
    ap.add_argument("--swin-img-fp32", type=int, nargs="*", default=[224, 384, 512],
                    help="Swin-Tiny image sizes of the fp32 fields (empty: skip)")
    # BASELINE configs 2 and 3 beside the main line: B1 H8 d64 fp16/fp32 1K-64K, causal fp16 197-32K
    ap.add_argument("--configs", dest="configs", action="store_true", default=True)
    ap.add_argument("--no-configs", dest="configs", action="store_false")
    ap.add_argument("--config-steps", type=int, default=10, help="timed iterations per baseline_configs case")
    ap.add_argument("--vit-batch", type=int, default=8, help="image batch of the ViT-T / Swin-T fields")
    ap.add_argument("--vit-steps", type=int, default=10, help="timed iterations of the ViT-T / Swin-T fields")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="no GPU work: turn two rocprofv3 --pmc counter_collection.csv files (FETCH_SIZE, "
                         "WRITE_SIZE) of a --copy-mib run into per-launch HBM bytes, written to --traffic-file")
    return ap.parse_args()


# rocprofv3 kernel-name fragment -> bench kernel name
_KERNEL_KEYS = (("phase1_half_kernel", "phase1_fold"), ("phase1_pp_kernel", "phase1_fold"), ("phase1_kernel", "phase1_fold"),
                ("phase2_kernel", "phase2_merge"), ("phase2_np_kernel", "phase2_merge"),
                ("bwd_pre_kernel", "bwd_preprocess"),
                ("bwd_dq_half_kernel", "bwd_dq"), ("bwd_dq_kernel", "bwd_dq"),
                ("bwd_dkdv_half_kernel", "bwd_dkdv"), ("bwd_dkdv_kernel", "bwd_dkdv"))


def _read_pmc(path, counter):
    import csv

    rows = []
    with open(path, newline="") as fh:
        for r in csv.DictReader(fh):
            if r["Counter_Name"] == counter:
                rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
    rows.sort()
    return rows


def summarize_pmc(fetch_csv, write_csv, copy_mib, out_path):
    """Per-launch HBM bytes of each ELSA kernel from FETCH_SIZE / WRITE_SIZE (KiB per dispatch).

    Each counter is scaled by what it reads for the calibration kernel of the same run
    (``torch.add`` over ``copy_mib`` MiB of fp32: copy_mib MiB read and copy_mib MiB written,
    the last elementwise add dispatch), so the figures are bytes, whatever fraction of the
    memory channels the counter samples.
    """
    out = {"copy_calibration_mib": copy_mib}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        rows = _read_pmc(path, counter)
        cal = [v for _, name, v in rows if "add" in name.lower() and "elementwise" in name.lower()]
        if not cal or cal[-1] <= 0:
            raise SystemExit(f"{path}: no calibration add kernel with a positive {counter}")
        factor = copy_mib * 1024.0 / cal[-1]
        out[f"{counter.lower()}_factor"] = round(factor, 4)
        per = {}
        for _, name, v in rows:
            key = next((b for frag, b in _KERNEL_KEYS if frag in name), None)
            if key is not None:
                per.setdefault(key, []).append(v * factor * 1024.0)
        for key, vals in per.items():
            ent = out.setdefault(key, {})
            ent[counter.lower() + "_bytes"] = sum(vals) / len(vals)
            ent["dispatches"] = len(vals)
    for key, ent in out.items():
        if isinstance(ent, dict) and "fetch_size_bytes" in ent and "write_size_bytes" in ent:
            ent["hbm_bytes_per_launch"] = round(ent["fetch_size_bytes"] + ent["write_size_bytes"])
    with open(out_path, "w") as fh:
        json.dump(out, fh, indent=1, sort_keys=True)
        fh.write("\n")
    return out


def _flops_fwd(b, h, n, d, causal):
    return 4.0 * b * h * d * (n * (n + 1) / 2 if causal else n * n)


def _mfma_ceiling(args, lib, dev, stream) -> float:
    """TFLOP/s of elsa_debug_mfma_rate on operands drawn as the inputs are (``--fill``)."""
    import torch

    from elsa_amd import _lib

    variant, kp, flop, iters = {"fp16": (0, 8, 32768, 20000), "bf16": (1, 8, 32768, 20000),
                                "fp32": (2, 1, 4096, 2000)}[args.dtype]
    dt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[args.dtype]
    x = torch.randn(16 * 256 * kp, generator=torch.Generator().manual_seed(7))
    if args.fill == "sign":
        x = x.sign()
    elif args.fill != "randn":
        x = torch.full_like(x, 0.0 if args.fill == "zeros" else 0.5)
    src = x.to(dt).to(dev)
    wgs = 2048
    out = torch.empty(wgs * 256, dtype=torch.float32, device=dev)
    sh = stream.cuda_stream

    def launch():
        _lib.check(lib.elsa_debug_mfma_rate(variant, src.data_ptr(), out.data_ptr(), iters, wgs, sh),
                   "elsa_debug_mfma_rate")

    launch()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(3):
        launch()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / 3
    tflops = wgs * 4 * iters * 8 * flop / (ms * 1e-3) / 1e12
    print(f"bench: MFMA ceiling ({args.fill} operands) {tflops:.1f} TFLOP/s", file=sys.stderr, flush=True)
    return tflops



def _kernel_ms(lib, stream, q, k, v, do, causal, block_n, steps):
    """HIP-event average of each hot-path launch set on ``stream``, through the C ABI.

    Phase 1 + Phase 2 run the training forward (the relaxed row state the backward reads); the
    three backward stages run on that forward's output and row state.  A plan of one partition
    is timed as ``elsa_fwd`` runs it, one Phase-1 launch with the finalize fused into its epilogue
    (phase2_merge is then 0: no launch); where the dq kernel runs the preprocess (fp16/bf16 at
    d = 64) bwd_preprocess is 0 the same way.  Returns (ms by kernel, the forward plan, the
    forward output)."""
    import torch

    from elsa_amd import _lib
    from elsa_amd.attention import _BiasMeta, _make_fwd_args, forward_plan
    from elsa_amd.attention_bwd import _attach_workspace, _bwd_args

    B, H, N, D = q.shape
    dev = q.device
    sh = stream.cuda_stream
    plan = forward_plan(q, is_causal=causal, block_n=block_n)
    out = torch.empty_like(q)
    rm = torch.empty((B * H, N), device=dev, dtype=torch.float32)
    rz = torch.empty_like(rm)
    fa = _make_fwd_args(q, k, v, out, rm, rz, _BiasMeta(None, 0, 0, 0, 0, False), is_causal=causal,
                        summary_dtype=q.dtype, partition_len=block_n, q_chunk=None, scale=1.0 / math.sqrt(D),
                        exact_row_max=False)
    ws_f = torch.empty(plan["workspace_bytes"], dtype=torch.uint8, device=dev)
    fa.workspace, fa.workspace_bytes = ws_f.data_ptr(), plan["workspace_bytes"]
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ba = _bwd_args(q, k, v, out, do, rm, rz, dq, dk, dv, _BiasMeta(None, 0, 0, 0, 0, False), is_causal=causal,
                   scale=1.0 / math.sqrt(D))
    ws_b = _attach_workspace(lib, ba, dev)
    qc = plan["q_chunk"]
    chunks = [(s_, min(qc, N - s_)) for s_ in range(0, N, qc)]

    fused = plan["partitions"] == 1
    # fp16/bf16 at d = 64 (dense operands, N rows under 2 GiB) and fp32 at d <= 64: the dq kernels run
    # the preprocess of their rows, and a whole backward (elsa_bwd) launches no preprocess kernel
    pre_fused = ((q.dtype in (torch.float16, torch.bfloat16) and D == 64 and N * D * q.element_size() < 2**31)
                 or (q.dtype == torch.float32 and D <= 64))
    # each launch set takes the stream handle it launches on
    launches = {
        "phase1_fold": ((lambda h: [lib.elsa_fwd(ctypes.byref(fa), h)]) if fused else
                        (lambda h: [lib.elsa_phase1(ctypes.byref(fa), s_, n_, h) for s_, n_ in chunks])),
        "phase2_merge": None if fused else (lambda h: [lib.elsa_phase2(ctypes.byref(fa), s_, n_, h)
                                                       for s_, n_ in chunks]),
        "bwd_preprocess": None if pre_fused else (lambda h: [lib.elsa_bwd_stage(ctypes.byref(ba), 0, h)]),
        "bwd_dq": lambda h: [lib.elsa_bwd_stage(ctypes.byref(ba), 1, h)],
        "bwd_dkdv": lambda h: [lib.elsa_bwd_stage(ctypes.byref(ba), 2, h)],
    }
    kern_ms = {}
    for name, fn in launches.items():
        if fn is None:
            kern_ms[name] = 0.0
            continue
        for rc in fn(sh):
            _lib.check(rc, name)
        torch.cuda.synchronize()
        # warm-up of about 25 ms of GPU work: after a host-side phase (drawing the next case's inputs)
        # the GPU clock ramps up over several ms, and a single 1 ms launch set would be timed at the
        # idle clock (causal 32K Phase 1 measured 1.31 ms after an idle gap, 1.13 ms when warm)
        t0 = time.perf_counter()
        fn(sh)
        torch.cuda.synchronize()
        one = max(time.perf_counter() - t0, 1e-6)
        for _ in range(min(200, int(0.025 / one))):
            fn(sh)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        if one < 2e-4:
            # a launch set shorter than about 0.2 ms: an eager loop of ctypes launches would time the
            # host's launch rate, so REPS of them are captured in a graph and its replays are timed
            reps = 20
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                hc = torch.cuda.current_stream().cuda_stream
                for _ in range(reps):
                    for rc in fn(hc):
                        _lib.check(rc, name)
            graph.replay()
            torch.cuda.synchronize()
            e0.record(stream)
            for _ in range(steps):
                graph.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            kern_ms[name] = e0.elapsed_time(e1) / (steps * reps)
            del graph
            continue
        e0.record(stream)
        for _ in range(steps):
            fn(sh)
        e1.record(stream)
        torch.cuda.synchronize()
        kern_ms[name] = e0.elapsed_time(e1) / steps
    del ws_f, ws_b, dq, dk, dv
    return kern_ms, plan, out


def _sampled_max_abs(q, k, v, out, causal, nrows=16, seed=0):
    """max |out - softmax(q k^T / sqrt(d)) v| over ``nrows`` sampled query rows, fp64 on the CPU."""
    import numpy as np

    N, D = q.shape[2], q.shape[3]
    rows = np.random.default_rng(seed).choice(N, min(nrows, N), replace=False)
    qs = q[:, :, rows].float().cpu().double().numpy()
    kk = k.float().cpu().double().numpy()
    vv = v.float().cpu().double().numpy()
    sc = np.einsum("bhid,bhjd->bhij", qs, kk) / math.sqrt(D)
    if causal:
        sc = np.where(np.arange(N)[None, None, None, :] <= rows[None, None, :, None], sc, -np.inf)
    sc -= sc.max(-1, keepdims=True)
    p = np.exp(sc)
    p /= p.sum(-1, keepdims=True)
    ref_o = np.einsum("bhij,bhjd->bhid", p, vv)
    return float(np.abs(out[:, :, rows].float().cpu().double().numpy() - ref_o).max())


# BASELINE config 2 (non-causal fp16 / fp32) and config 3 (causal fp16, with the non-divisible
# lengths) at B1 H8 d64: (dtype, causal, seq_len)
_CONFIG_CASES = ([("fp16", False, n) for n in (1024, 4096, 16384, 65536)]
                 + [("fp32", False, n) for n in (1024, 4096, 16384, 65536)]
                 + [("fp16", True, n) for n in (2048, 8192, 32768, 197, 1025, 4097)])


def _baseline_configs(args, lib, dev, stream):
    """The other shapes of BASELINE configs 2 and 3, each timed as the main line is.

    Per case: the kernels' HIP-event averages (forward = Phase 1 + Phase 2, backward = the three
    backward stages), the algorithmic TFLOP/s and fraction of the dtype's dense MFMA peak, the
    wall-clock of the public training step (twopass_attention_train + autograd.grad, host work
    included) and a sampled fp64 check of the forward.  Inputs q, k, v, dO ~ N(0,1), seed 1234."""
    import torch

    import elsa_amd

    res = {}
    for dts, causal, n in _CONFIG_CASES:
        if (dts, causal, n) == (args.dtype, bool(args.causal), args.seq) and (args.batch, args.heads, args.dim) == (1, 8, 64):
            continue  # the main line
        dt = {"fp16": torch.float16, "fp32": torch.float32}[dts]
        gen = torch.Generator().manual_seed(1234)
        q, k, v, do = (torch.randn((1, 8, n, 64), generator=gen).to(dt).to(dev) for _ in range(4))
        f_fwd = _flops_fwd(1, 8, n, 64, causal)
        steps = max(2, min(args.config_steps, int(2e13 / f_fwd) if dts == "fp32" else args.config_steps))
        kern_ms, plan, out = _kernel_ms(lib, stream, q, k, v, do, causal, None, steps)
        qg, kg, vg = (t.detach().requires_grad_() for t in (q, k, v))

        def step():
            o = elsa_amd.twopass_attention_train(qg, kg, vg, is_causal=causal)
            return torch.autograd.grad(o, (qg, kg, vg), do)

        step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        step_ms = e0.elapsed_time(e1) / steps
        fwd_ms = kern_ms["phase1_fold"] + kern_ms["phase2_merge"]
        bwd_ms = kern_ms["bwd_preprocess"] + kern_ms["bwd_dq"] + kern_ms["bwd_dkdv"]
        peak = PEAK_TFLOPS[dts]
        key = f"{dts}_{'causal_' if causal else ''}n{n}"
        res[key] = {
            "seq_len": n, "dtype": dts, "causal": causal, "partitions": plan["partitions"],
            "partition_len": plan["partition_len"], "steps": steps,
            "fwd_ms": round(fwd_ms, 4), "bwd_ms": round(bwd_ms, 4),
            "fwd_tflops": round(f_fwd / (fwd_ms * 1e-3) / 1e12, 1),
            "bwd_tflops": round(2.5 * f_fwd / (bwd_ms * 1e-3) / 1e12, 1),
            "fwd_frac_peak": round(f_fwd / (fwd_ms * 1e-3) / 1e12 / peak, 4),
            "bwd_frac_peak": round(2.5 * f_fwd / (bwd_ms * 1e-3) / 1e12 / peak, 4),
            "train_step_ms": round(step_ms, 4),
            "max_abs_sampled_fwd": _sampled_max_abs(q, k, v, out, causal, nrows=8),
        }
        print(f"bench: config {key}: fwd {fwd_ms:.4f} ms, bwd {bwd_ms:.4f} ms, step {step_ms:.4f} ms",
              file=sys.stderr, flush=True)
        del q, k, v, do, qg, kg, vg, out
        torch.cuda.empty_cache()
    return res


def main() -> int:
    args = _args()
    if args.summarize_pmc:
        res = summarize_pmc(*args.summarize_pmc, args.copy_mib or 1024, args.traffic_file)
        print(json.dumps(res))
        return 0
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures a single GPU: this build has no multi-GPU path (the attention would shard "
              "by batch x heads with no communication). Run with --gpus 1.", file=sys.stderr, flush=True)
        return 2

    import torch

    import elsa_amd
    from elsa_amd import _lib

    dt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[args.dtype]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, H, N, D = args.batch, args.heads, args.seq, args.dim
    shape = (B, H, N, D)
    g = torch.Generator().manual_seed(2026)
    def _input():
        x = torch.randn(shape, generator=g)
        if args.fill == "sign":
            x = x.sign()
        elif args.fill != "randn":
            x = torch.full(shape, 0.0 if args.fill == "zeros" else 0.5)
        return x.to(dt).to(dev)

    q, k, v, do = (_input() for _ in range(4))
    causal = bool(args.causal)
    print(f"bench: {shape} {args.dtype} causal={causal} steps={args.steps} warmup={args.warmup}", file=sys.stderr,
          flush=True)

    # ---- per-kernel HIP-event timing through the C ABI, on the stream the kernels run on (first, so
    # that the GPU clock has left its idle state before the warm-up and timed steps below)
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev)
    kern_ms, plan, out = _kernel_ms(lib, stream, q, k, v, do, causal, args.block_n, args.steps)
    print("bench: kernels " + ", ".join(f"{k_}={v_:.3f}ms" for k_, v_ in kern_ms.items()), file=sys.stderr,
          flush=True)

    # one training step through the reference's training entry point (its benchmarks/bench_bwd.py
    # times twopass_attention_train(...).backward(dout)): forward with the row state the backward
    # reads, then the recompute backward; torch.autograd.grad returns the gradients without
    # accumulating them into .grad
    qg, kg, vg = (t.detach().requires_grad_() for t in (q, k, v))

    def step():
        out = elsa_amd.twopass_attention_train(qg, kg, vg, is_causal=causal, block_n=args.block_n)
        return torch.autograd.grad(out, (qg, kg, vg), do)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = ev0.elapsed_time(ev1) / args.steps
    print(f"bench: step {ms_step:.3f} ms (wall {wall * 1e3 / args.steps:.3f} ms)", file=sys.stderr, flush=True)

    # ---- the matrix cores' sustained rate on operands with this run's value statistics
    ceiling = _mfma_ceiling(args, lib, dev, stream)

    # ---- latency ratio against PyTorch's SDPA on the same inputs, the reference's headline
    # comparison (README.md:55-58: ELSA / FlashAttention on A100), for fp16 only
    vs_sdpa = _vs_sdpa(args, q, k, v, do, causal) if args.dtype == "fp16" else None

    # ---- sampled parity check of this very run (closed form, fp64 on CPU)
    max_abs = _sampled_max_abs(q, k, v, out, causal)

    # ---- derived numbers
    f_fwd = _flops_fwd(B, H, N, D, causal)
    f_bwd = 2.5 * f_fwd
    peak = PEAK_TFLOPS[args.dtype]
    ssz = torch.empty((), dtype=dt).element_size()
    p2_bytes = plan["partitions"] * B * H * N * (8 + D * ssz) + B * H * N * D * ssz + 8 * B * H * N
    fwd_ms = kern_ms["phase1_fold"] + kern_ms["phase2_merge"]
    bwd_ms = kern_ms["bwd_preprocess"] + kern_ms["bwd_dq"] + kern_ms["bwd_dkdv"]
    algo = {  # algorithmic work per launch set (flop, or bytes for the HBM-bound kernels)
        "phase1_fold": ("mfma", f_fwd),
        "phase2_merge": ("hbm", p2_bytes),
        "bwd_preprocess": ("hbm", 2 * B * H * N * D * ssz + 16 * B * H * N),
        "bwd_dq": ("mfma", 0.5 * f_fwd),
        "bwd_dkdv": ("mfma", 2.0 * f_fwd),
    }
    kernels = {}
    for name, ms in kern_ms.items():
        bound, work = algo[name]
        if ms == 0.0:  # Phase 2 fused into the Phase-1 launch (one partition), the preprocess into dq
            kernels[name] = {"ms": 0.0, "fused_into": "bwd_dq" if name == "bwd_preprocess" else "phase1_fold"}
        elif bound == "mfma":
            ach = work / (ms * 1e-3) / 1e12
            kernels[name] = {"ms": round(ms, 4), "tflops": round(ach, 1), "frac_peak": round(ach / peak, 4)}
        else:
            ach = work / (ms * 1e-3) / 1e9
            kernels[name] = {"ms": round(ms, 4), "gbps": round(ach, 1), "frac_peak": round(ach / HBM_GBPS, 4)}
    dom = max(kern_ms, key=kern_ms.get)
    bound, work = algo[dom]
    # HBM bytes per launch come from rocprofv3 counters, which this run does not collect: the
    # figure of the committed profile (FETCH_SIZE + WRITE_SIZE of this kernel, calibrated), valid
    # while the kernels are the ones profiled there
    traffic = None
    traffic_source = None
    if os.path.exists(args.traffic_file):
        try:
            with open(args.traffic_file) as fh:
                traffic = json.load(fh).get(dom, {}).get("hbm_bytes_per_launch")
            traffic_source = os.path.relpath(args.traffic_file, ROOT) + " (committed rocprofv3 --pmc profile)"
        except (OSError, ValueError):
            traffic = None
    if bound == "mfma":
        achieved = work / (kern_ms[dom] * 1e-3) / 1e12
        roofline = {"bound": "mfma", "achieved": round(achieved, 1), "peak": peak, "unit": "TFLOP/s",
                    "frac": round(achieved / peak, 4), "traffic": traffic, "traffic_source": traffic_source,
                    "kernel": dom, "work_per_launch": work}
    else:
        achieved = work / (kern_ms[dom] * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_GBPS, "unit": "GB/s",
                    "frac": round(achieved / HBM_GBPS, 4), "traffic": traffic, "traffic_source": traffic_source,
                    "kernel": dom, "work_per_launch": work}

    value = (f_fwd + f_bwd) / (ms_step * 1e-3) / 1e12
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": ("synthetic: q,k,v,dO ~ N(0,1), torch.Generator seed 2026, resident in HBM" if args.fill == "randn"
                 else f"synthetic, diagnostic fill '{args.fill}' (not the benchmark input)"),
        "config": {"workload": "ELSA two-pass attention training step (twopass_attention_train fwd + bwd), "
                               + ("causal" if causal else "non-causal"),
                   "batch": B, "heads": H, "seq_len": N, "head_dim": D,
                   "partitions": plan["partitions"], "partition_len": plan["partition_len"],
                   "q_chunk": plan["q_chunk"]},
        "fwd_ms": round(fwd_ms, 4),
        "bwd_ms": round(bwd_ms, 4),
        "fwd_tflops": round(f_fwd / (fwd_ms * 1e-3) / 1e12, 1),
        "bwd_tflops": round(f_bwd / (bwd_ms * 1e-3) / 1e12, 1),
        "fwd_frac_peak": round(f_fwd / (fwd_ms * 1e-3) / 1e12 / peak, 4),
        "bwd_frac_peak": round(f_bwd / (bwd_ms * 1e-3) / 1e12 / peak, 4),
        "phase2_gbps": kernels["phase2_merge"].get("gbps"),  # None when fused into Phase 1
        "max_abs_sampled_fwd": max_abs,
        "kernels": kernels,
        "roofline": roofline,
    }
    # executed MFMA work per launch (the dq kernel recomputes S and dP: 3 GEMMs of N^2 d)
    executed = {"phase1_fold": f_fwd, "bwd_dq": 1.5 * f_fwd, "bwd_dkdv": 2.0 * f_fwd}
    result["mfma_ceiling"] = {
        "fill": args.fill, "tflops": round(ceiling, 1), "frac_peak": round(ceiling / peak, 4),
        "what": "sustained v_mfma_f32_32x32x* rate of 8 independent chains per wave on operands drawn like the "
                "inputs (elsa_debug_mfma_rate); the power limit sets it below the nominal peak",
        "executed_frac_of_ceiling": {n: round(w / (kern_ms[n] * 1e-3) / 1e12 / ceiling, 4)
                                     for n, w in executed.items()},
    }
    if vs_sdpa is not None:
        result["vs_sdpa"] = vs_sdpa
    from elsa_amd.vision_models import swin_tiny_patch4_window7, vit_tiny_patch16

    vit = ("vit_tiny_patch16 (embed 192, depth 12, heads 3, d 64), random init", lambda img: (img // 16) ** 2 + 1)
    swin = ("swin_tiny_patch4_window7 (embed 96, depths 2-2-6-2, heads 3-6-12-24, d 32, window 7; feature maps "
            "padded to whole windows), random init", lambda img: 49)
    model_runs = [("vit_tiny", dt, vit_tiny_patch16, args.vit_img, vit),
                  ("swin_tiny", dt, swin_tiny_patch4_window7, args.swin_img, swin)]
    if dt != torch.float32:
        model_runs += [("vit_tiny_fp32", torch.float32, vit_tiny_patch16, args.vit_img_fp32, vit),
                       ("swin_tiny_fp32", torch.float32, swin_tiny_patch4_window7, args.swin_img_fp32, swin)]
    for key, mdt, builder, imgs, (label, tokens) in model_runs:
        if imgs:
            result[key] = _vision_bench(args, mdt, builder, imgs, label, tokens)
    if args.copy_mib > 0:
        # one elementwise kernel that reads and writes copy_mib MiB each: the FETCH_SIZE / WRITE_SIZE
        # calibration for the HBM-traffic figures
        src = torch.ones(args.copy_mib << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.add(src, 1.0, out=dst)
        torch.cuda.synchronize()
        result["copy_calibration_mib"] = args.copy_mib
    if args.configs:
        result["baseline_configs"] = _baseline_configs(args, lib, dev, stream)
    if args.cpu_baseline:
        result["cpu_baseline"] = _cpu_baseline(args, B, H, N, D, causal)
    print(json.dumps(result), flush=True)
    return 0


def _vs_sdpa(args, q, k, v, do, causal):
    """Mean latency of the public API calls against torch.nn.functional.scaled_dot_product_attention
    (PyTorch picks its fused kernel on ROCm), forward and forward+backward, timed the same way;
    backward = (forward+backward) - forward.  lat_ratio = ELSA / SDPA, as the reference reports."""
    import torch
    import torch.nn.functional as F

    import elsa_amd

    iters = max(5, min(args.steps, 20))

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters

    qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (q, k, v))

    def sdpa_fb():
        F.scaled_dot_product_attention(qg, kg, vg, is_causal=causal).backward(do)

    def elsa_fb():
        elsa_amd.twopass_attention_train(qg, kg, vg, is_causal=causal).backward(do)

    with torch.no_grad():
        s_f = timed(lambda: F.scaled_dot_product_attention(q, k, v, is_causal=causal))
        e_f = timed(lambda: elsa_amd.twopass_attention(q, k, v, is_causal=causal))
    s_fb, e_fb = timed(sdpa_fb), timed(elsa_fb)
    out = {"sdpa_fwd_ms": round(s_f, 4), "sdpa_bwd_ms": round(s_fb - s_f, 4),
           "elsa_fwd_ms": round(e_f, 4), "elsa_bwd_ms": round(e_fb - e_f, 4),
           "fwd_lat_ratio": round(e_f / s_f, 3), "bwd_lat_ratio": round((e_fb - e_f) / (s_fb - s_f), 3)}
    print(f"bench: vs SDPA {out}", file=sys.stderr, flush=True)
    return out


def _vision_bench(args, dt, builder, imgs, label, tokens):
    """img/s of a vision model with the ELSA drop-in against the same model on PyTorch SDPA.

    Follows the reference's model benchmarks (benchmarks/full_model_graph.py,
    benchmarks/full_model_bwd_min.py): random-init weights cast to the compute dtype, a
    synthetic N(0,1) image batch, forward timed as hipGraph replays, and a training step
    of forward, cross-entropy on synthetic labels over 1000 classes, backward and an SGD
    update.  Times are means over the timed iterations.
    """
    import copy

    import torch

    import elsa_amd

    out = {"model": label, "batch": args.vit_batch, "dtype": str(dt).replace("torch.", "")}
    for img in imgs:
        torch.manual_seed(2468 + img)
        base = builder(img)
        elsa_fwd = copy.deepcopy(base)
        elsa_amd.patch_timm_attention(elsa_fwd)
        elsa_train = copy.deepcopy(base)
        elsa_amd.patch_timm_attention_train(elsa_train)
        models = {"sdpa": base.to("cuda", dt), "elsa": elsa_fwd.to("cuda", dt)}
        x = torch.randn(args.vit_batch, 3, img, img, device="cuda", dtype=dt)
        labels = torch.randint(0, 1000, (args.vit_batch,), device="cuda")
        row = {"tokens": tokens(img)}
        # fp32 beyond 4K tokens: fewer timed iterations (a ViT-T fp32 training step at 16385 tokens
        # takes most of a second)
        steps = args.vit_steps
        if dt == torch.float32 and tokens(img) > 4097:
            steps = max(2, args.vit_steps * 4097 // tokens(img))
        row["steps"] = steps
        for name, m in models.items():
            m.eval()
            row[f"{name}_fwd_ms"] = _unless_oom(lambda: _graph_fwd_ms(m, x, steps))
        for name, m in (("sdpa", models["sdpa"]), ("elsa", elsa_train.to("cuda", dt))):
            row[f"{name}_train_ms"] = _unless_oom(lambda: _train_ms(m, x, labels, steps))
        for kind in ("fwd", "train"):
            e, b = row[f"elsa_{kind}_ms"], row[f"sdpa_{kind}_ms"]
            row[f"elsa_{kind}_img_s"] = round(args.vit_batch / (e * 1e-3), 1) if e else None
            row[f"{kind}_lat_ratio_vs_sdpa"] = round(e / b, 3) if e and b else None
        print(f"bench: {builder.__name__} {img}px {row}", file=sys.stderr, flush=True)
        out[str(img)] = row
        del models, elsa_train
        torch.cuda.empty_cache()
    return out


def _unless_oom(fn):
    """fn() in ms, or None where it ran out of device memory (PyTorch's SDPA math path keeps
    every layer's [B, H, N, N] attention matrix for the backward)."""
    import torch

    try:
        return fn()
    except torch.cuda.OutOfMemoryError:
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        return None


def _graph_fwd_ms(model, x, steps):
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s), torch.no_grad():
        for _ in range(3):
            model(x)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.graph(graph):
        model(x)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    del graph
    return round(ms, 4)


def _train_ms(model, x, labels, steps):
    import torch

    model.train()
    opt = torch.optim.SGD(model.parameters(), lr=1e-4, momentum=0.9)

    def one():
        opt.zero_grad(set_to_none=True)
        loss = torch.nn.functional.cross_entropy(model(x).float(), labels)
        loss.backward()
        opt.step()

    for _ in range(3):
        one()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        one()
    e1.record()
    torch.cuda.synchronize()
    return round(e0.elapsed_time(e1) / steps, 4)


def _cpu_model() -> str:
    cpu = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return cpu


def _median_s(fn, warmup=3, iters=10):
    import statistics

    for _ in range(warmup):
        fn()
    times = []
    for _ in range(iters):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def _cpu_baseline(args, B, H, N, D, causal):
    """The reference algorithm on the host cores, a reported baseline.

    The reference has no CPU path (every entry point rejects non-CUDA tensors,
    attention.py:268-269), so this times oracle/torch_scan.py, the build's pure-PyTorch
    restatement of the reference's monoid scan (Phase-1 fold per K partition at the
    reference's partition and micro-tile widths, the merge, out = s/z), on every thread
    torch is given (OMP_NUM_THREADS on the GPU box):

    * ``value``: BASELINE config 1 -- non-causal B1 H8 N1024 d64 fp32 forward, q, k, v
      ~ N(0,1) from torch.Generator seed 1234 in that order, scale 1/8 -- median of 10
      after 3 warm-ups, checked against math SDPA in float64, with CPU math SDPA timed
      beside it;
    * ``north_star_sample``: the benchmarked step's own work (fwd + bwd at the reference's
      rounding points) for the first query rows of this run's shape.
    """
    import numpy as np
    import torch
    import torch.nn.functional as F

    from oracle import elsa_oracle as O
    from oracle import torch_scan as T

    threads = torch.get_num_threads()
    cpu = _cpu_model()
    print(f"bench: cpu baseline (BASELINE config 1) on {threads} threads of {cpu}", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(1234)
    shape1 = (1, 8, 1024, 64)
    q1, k1, v1 = (torch.randn(shape1, generator=g) for _ in range(3))
    part1, micro1 = O.reference_routing(1024, 64, "fp32")
    res = {}

    def scan():
        res["out"] = T.forward(q1, k1, v1, part_len=part1, micro=micro1, dtype="fp32")[0]

    secs = _median_s(scan)
    sdpa_secs = _median_s(lambda: F.scaled_dot_product_attention(q1, k1, v1, scale=0.125))
    exact = F.scaled_dot_product_attention(q1.double(), k1.double(), v1.double(), scale=0.125)
    err = float((res["out"].double() - exact).abs().max())
    f1 = _flops_fwd(*shape1, False)
    out = {"value": round(f1 / secs / 1e12, 5), "unit": "TFLOP/s", "cores": int(threads), "kind": "port",
           "sample": f"BASELINE config 1: non-causal B1 H8 N1024 d64 fp32 forward (seed 1234, scale 1/8) through "
                     f"oracle/torch_scan.py, the pure-PyTorch restatement of the reference's monoid scan "
                     f"({part1}-key partition, {micro1}-key micro-tiles); median of 10 after 3 warm-ups: "
                     f"{secs * 1e3:.2f} ms on {threads} threads of {cpu} (os.cpu_count()={os.cpu_count()})",
           "ms": round(secs * 1e3, 3), "gflops": round(f1 / secs / 1e9, 2),
           "max_abs_vs_math_sdpa_fp64": err,
           "cpu_math_sdpa": {"ms": round(sdpa_secs * 1e3, 3), "gflops": round(f1 / sdpa_secs / 1e9, 2),
                             "what": "torch.nn.functional.scaled_dot_product_attention on the same fp32 inputs "
                                     "(CPU math path), for context"},
           "cpu_model": cpu}

    # the north-star step's own work on a row sample
    rows = np.arange(min(args.cpu_rows, N))
    g = torch.Generator().manual_seed(2026)
    tdt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[args.dtype]
    q, k, v, do = (torch.randn((B, H, N, D), generator=g).to(tdt) for _ in range(4))
    part, micro = O.reference_routing(N, D, args.dtype, training=True, is_causal=causal)
    t0 = time.perf_counter()
    ro, rm, rz = T.forward(q, k, v, is_causal=causal, part_len=part, micro=micro, dtype=args.dtype, rows=rows)
    full_o = torch.zeros((B, H, N, D))
    full_o[:, :, rows] = ro
    full_m = torch.full((B * H, N), float("-inf"))
    full_z = torch.zeros((B * H, N))
    full_m[:, rows] = rm
    full_z[:, rows] = rz
    T.backward(q, k, v, full_o, do, full_m, full_z, is_causal=causal, dtype=args.dtype, rows=rows)
    ns_secs = time.perf_counter() - t0
    frac = len(rows) / N if not causal else float((rows + 1).sum()) / (N * (N + 1) / 2)
    ns_flops = 3.5 * _flops_fwd(B, H, N, D, causal) * frac
    out["north_star_sample"] = {
        "value": round(ns_flops / ns_secs / 1e12, 5), "unit": "TFLOP/s", "seconds": round(ns_secs, 3),
        "sample": f"fwd + bwd at the reference's rounding points (oracle/torch_scan.py, {part}-key partitions) for "
                  f"query rows 0..{len(rows) - 1} of B{B} H{H} N{N} d{D} {args.dtype} against all keys, one run"}
    return out


if __name__ == "__main__":
    sys.exit(main())
