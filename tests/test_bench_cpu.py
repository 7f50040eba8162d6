"""CPU tests of bench.py's host logic: the single-GPU contract and the HBM-traffic
calibration that turns FETCH_SIZE / WRITE_SIZE counters into bytes per launch."""
from __future__ import annotations

import csv
import json
import math
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused_with_a_message():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                          timeout=300, cwd=ROOT)
    assert proc.returncode == 2
    assert "single GPU" in proc.stderr and proc.stdout == ""


def _write_counters(path: Path, counter: str, rows):
    with open(path, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for i, (name, value) in enumerate(rows):
            w.writerow({"Dispatch_Id": i, "Kernel_Name": name, "Counter_Name": counter, "Counter_Value": value})


def test_traffic_calibration_scales_each_counter_by_the_copy_kernel(tmp_path):
    """A counter that sees half of the memory channels reads half of a 1 GiB copy; every kernel's
    figure is scaled by the same factor, and kernels are averaged over their dispatches."""
    copy = "void at::native::vectorized_elementwise_kernel<4, at::native::CUDAFunctor_add<float>>"
    fetch_rows = [("_ZN4elsa18phase1_half_kernelIDF16_Li64ELi2ELi4ELb0EEEvNS_12Phase1ParamsE", 1000.0),
                  ("_ZN4elsa18phase1_half_kernelIDF16_Li64ELi2ELi4ELb0EEEvNS_12Phase1ParamsE", 1200.0),
                  ("_ZN4elsa13phase2_kernelIDF16_DF16_EEvNS_12Phase2ParamsE", 300.0),
                  ("some_other_kernel", 5.0),
                  (copy, 1024 * 1024 / 2)]            # sees half of the 1 GiB read
    write_rows = [("_ZN4elsa18phase1_half_kernelIDF16_Li64ELi2ELi4ELb0EEEvNS_12Phase1ParamsE", 700.0),
                  ("_ZN4elsa18phase1_half_kernelIDF16_Li64ELi2ELi4ELb0EEEvNS_12Phase1ParamsE", 700.0),
                  ("_ZN4elsa13phase2_kernelIDF16_DF16_EEvNS_12Phase2ParamsE", 100.0),
                  (copy, 1024 * 1024)]                # sees all of the 1 GiB write
    _write_counters(tmp_path / "f.csv", "FETCH_SIZE", fetch_rows)
    _write_counters(tmp_path / "w.csv", "WRITE_SIZE", write_rows)
    out = bench.summarize_pmc(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"), 1024, str(tmp_path / "t.json"))
    assert out["fetch_size_factor"] == 2.0 and out["write_size_factor"] == 1.0
    p1 = out["phase1_fold"]
    assert p1["dispatches"] == 2
    assert math.isclose(p1["fetch_size_bytes"], 1100.0 * 2 * 1024)
    assert math.isclose(p1["write_size_bytes"], 700.0 * 1024)
    assert p1["hbm_bytes_per_launch"] == round(1100.0 * 2 * 1024 + 700.0 * 1024)
    assert math.isclose(out["phase2_merge"]["fetch_size_bytes"], 300.0 * 2 * 1024)
    assert "some_other_kernel" not in json.dumps(out)
    assert json.loads((tmp_path / "t.json").read_text()) == json.loads(json.dumps(out))


def test_traffic_calibration_needs_the_copy_kernel(tmp_path):
    _write_counters(tmp_path / "f.csv", "FETCH_SIZE", [("_ZN4elsa13phase2_kernelIDF16_DF16_EE", 1.0)])
    _write_counters(tmp_path / "w.csv", "WRITE_SIZE", [("_ZN4elsa13phase2_kernelIDF16_DF16_EE", 1.0)])
    with pytest.raises(SystemExit, match="calibration"):
        bench.summarize_pmc(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"), 1024, str(tmp_path / "t.json"))


def test_every_elsa_kernel_name_maps_to_its_bench_kernel():
    """The counter summary recognises each launched kernel by a fragment of its mangled name."""
    names = {
        "_ZN4elsa18phase1_half_kernelIDF16_Li64ELi2ELi4ELb0ELb1EEEvNS_12Phase1ParamsE": "phase1_fold",
        "_ZN4elsa13phase1_kernelIfLi64ELi4ELb0EEEvNS_12Phase1ParamsE": "phase1_fold",
        "_ZN4elsa16phase2_np_kernelIDF16_DF16_Li2ELb1EEEvNS_12Phase2ParamsE": "phase2_merge",
        "_ZN4elsa13phase2_kernelIDF16_DF16_EEvNS_12Phase2ParamsE": "phase2_merge",
        "_ZN4elsa14bwd_pre_kernelIDF16_EEvNS_9BwdParamsE": "bwd_preprocess",
        "_ZN4elsa18bwd_dq_half_kernelIDF16_Li64ELi1ELi4ELb0EEEvNS_9BwdParamsE": "bwd_dq",
        "_ZN4elsa13bwd_dq_kernelIfLi64ELi4ELb0EEEvNS_9BwdParamsE": "bwd_dq",
        "_ZN4elsa20bwd_dkdv_half_kernelIDF16_Li64ELi1ELi4ELb0EEEvNS_9BwdParamsE": "bwd_dkdv",
        "_ZN4elsa15bwd_dkdv_kernelIfLi64ELi4ELb0EEEvNS_9BwdParamsE": "bwd_dkdv",
    }
    for name, key in names.items():
        assert next(b for frag, b in bench._KERNEL_KEYS if frag in name) == key, name


def test_algorithmic_flops():
    assert bench._flops_fwd(1, 8, 16384, 64, False) == 4.0 * 8 * 16384 ** 2 * 64
    assert bench._flops_fwd(1, 1, 4, 2, True) == 4.0 * 2 * (4 * 5 / 2)


def test_cpu_baseline_times_baseline_config_1():
    """cpu_baseline is BASELINE config 1 (B1 H8 N1024 d64 fp32 forward, seed 1234) through the
    pure-PyTorch restatement, checked against math SDPA, with CPU SDPA and a row sample of the
    benchmarked step beside it."""
    import types

    args = types.SimpleNamespace(cpu_rows=64, dtype="fp16")
    res = bench._cpu_baseline(args, 1, 2, 512, 64, False)
    assert res["kind"] == "port" and res["unit"] == "TFLOP/s" and res["value"] > 0 and res["cores"] >= 1
    assert "BASELINE config 1" in res["sample"] and "1234" in res["sample"]
    assert res["max_abs_vs_math_sdpa_fp64"] < 2e-6  # fp32 restatement against the fp64 closed form
    assert res["cpu_math_sdpa"]["ms"] > 0
    assert math.isclose(res["gflops"], 4 * 8 * 1024 ** 2 * 64 / (res["ms"] * 1e-3) / 1e9, rel_tol=1e-3)
    ns = res["north_star_sample"]
    assert ns["value"] > 0 and "rows 0..63" in ns["sample"]


def test_baseline_config_cases_cover_configs_2_and_3():
    """baseline_configs covers BASELINE config 2 (non-causal fp16 and fp32 at 1K, 4K, 16K, 64K) and
    config 3 (causal fp16 at 2K, 8K, 32K and the non-divisible 197, 1025, 4097)."""
    cases = set(bench._CONFIG_CASES)
    for dt in ("fp16", "fp32"):
        for n in (1024, 4096, 16384, 65536):
            assert (dt, False, n) in cases
    for n in (2048, 8192, 32768, 197, 1025, 4097):
        assert ("fp16", True, n) in cases
    assert len(cases) == len(bench._CONFIG_CASES) == 14


@pytest.mark.parametrize("causal", [False, True])
def test_sampled_max_abs_sees_one_wrong_row(causal):
    """The sampled forward check of every bench line: zero on the exact output, and a change to one
    sampled row shows up at its size."""
    import torch

    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn((1, 2, 40, 8), generator=g, dtype=torch.float64) for _ in range(3))
    mask = torch.ones(40, 40, dtype=torch.bool).tril() if causal else None
    out = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask)
    # the check reads the tensors through fp32, as it reads the kernels' fp16 / fp32 outputs
    assert bench._sampled_max_abs(q, k, v, out, causal, nrows=40) < 1e-6
    bad = out.clone()
    bad[0, 1, 17, 3] += 0.25
    assert abs(bench._sampled_max_abs(q, k, v, bad, causal, nrows=40) - 0.25) < 1e-6
