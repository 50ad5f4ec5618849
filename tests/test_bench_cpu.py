"""bench.py's host-side pieces that need no GPU: kernel-name shortening, the join of a
rocprofv3 trace with its counter passes (on synthetic CSVs of the same columns), the
one-GPU refusal, and the CPU baseline on a tiny workload."""
import csv
import importlib.util
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.mark.parametrize("name, short", [
    ("void (anonymous namespace)::gemm_kernel<H16F, 256, 256, 64, 4, 2, false, false, 1, 0>(GemmArgs)",
     "gemm_kernel<H16F, 256, 256, 64, 4, 2, false, false, 1, 0>"),
    ("void (anonymous namespace)::adam_kernel<H16F, true>(AdamArgs)", "adam_kernel<H16F, true>"),
    ("__amd_rocclr_copyBuffer", "__amd_rocclr_copyBuffer"),
    ("void at::native::(anonymous namespace)::fill<float>(float*, long)", "at::native::fill<float>"),
    ("sumsq2_kernel(float const*, long, float const*, long, double*, int)", "sumsq2_kernel"),
])
def test_short_kernel_names(bench, name, short):
    assert bench._short(name) == short


def _write(path, header, rows):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.writer(f, quoting=csv.QUOTE_ALL)
        w.writerow(header)
        w.writerows(rows)


def test_counters_collect_joins_passes(bench, tmp_path):
    adam = "void (anonymous namespace)::adam_kernel<H16F, true>(AdamArgs)"
    gemm = "void (anonymous namespace)::gemm_kernel<H16F, 64, 64, 128, 2, 2, true, true, 0, 0>(GemmArgs)"
    copy = "__amd_rocclr_copyBuffer"
    d = str(tmp_path)
    _write(os.path.join(d, "trace", "run_kernel_stats.csv"),
           ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs", "StdDev"],
           [[adam, 29, 29 * 100000, 100000, 60.0, 1, 1, 0], [gemm, 10, 10 * 20000, 20000, 40.0, 1, 1, 0]])
    cols = ["Kernel_Name", "Counter_Name", "Counter_Value"]
    # copies: three 1 GiB copies read 524288 KiB units each (2048 bytes per unit), one small one
    fetch = [[copy, "FETCH_SIZE", 524288.0]] * 3 + [[copy, "FETCH_SIZE", 10.0]] + \
            [[adam, "FETCH_SIZE", 1000.0], [adam, "FETCH_SIZE", 3000.0], [gemm, "FETCH_SIZE", 50.0]]
    write = [[copy, "WRITE_SIZE", 1048576.0]] * 3 + [[adam, "WRITE_SIZE", 500.0], [gemm, "WRITE_SIZE", 8.0]]
    mfma = [[gemm, "MfmaUtil", 5.0], [gemm, "SQ_INSTS_VALU_MFMA_MOPS_F16", 1000.0], [adam, "MfmaUtil", 0.0]]
    # dispatch order: two steps, each from one embedding lookup to the next (copies and the
    # MFMA-ceiling probe are not counted)
    emb = "void (anonymous namespace)::embed_fwd_kernel(float const*, int const*, float*, int, int)"
    probe = "void (anonymous namespace)::mfma_ceiling_kernel<H16F, true>(float*, int)"
    seq = [emb, gemm, copy, gemm, adam, emb, gemm, probe, gemm, adam, emb]
    _write(os.path.join(d, "trace", "run_kernel_trace.csv"), ["Kernel_Name", "Start_Timestamp"],
           [[n, 100 * (i + 1)] for i, n in reversed(list(enumerate(seq)))])
    _write(os.path.join(d, "fetch", "run_counter_collection.csv"), cols, fetch)
    _write(os.path.join(d, "write", "run_counter_collection.csv"), cols, write)
    _write(os.path.join(d, "mfma", "run_counter_collection.csv"), cols, mfma)
    result = {"roofline": {"kernel": "adam_kernel (AdamW)", "launches_per_pass": 29.0, "traffic": None,
                           "traffic_source": "x", "achieved": 1.0, "peak": 8000.0, "frac": 0.1,
                           "bytes_per_pass": 1e9},
              "config": {"workload": "w"}, "ms_per_step": 1.0}
    res = bench.counters_collect(d, result, {"trace": "cmd"})
    rows = {r["kernel"]: r for r in res["counters"]["kernels"]}
    a = rows["adam_kernel<H16F, true>"]
    assert a["calls"] == 29 and a["avg_us"] == pytest.approx(100.0)
    assert a["read_MB_per_launch"] == pytest.approx(2000.0 * 2048 / 1e6)   # mean of the two dispatches
    assert a["write_MB_per_launch"] == pytest.approx(500.0 * 1024 / 1e6)
    g = rows["gemm_kernel<H16F, 64, 64, 128, 2, 2, true, true, 0, 0>"]
    assert g["mfma_util_pct"] == pytest.approx(5.0)
    assert g["mfma_tflops"] == pytest.approx(1000.0 * 512 / 20e-6 / 1e12)
    cal = res["counters"]["calibration"]
    assert cal["fetch_bytes_per_unit"] == pytest.approx(2048.0) and cal["write_bytes_per_unit"] == pytest.approx(1024.0)
    assert res["roofline"]["traffic"] == pytest.approx((2000.0 * 2048 + 500.0 * 1024) * 29)
    assert "FETCH_SIZE" in res["roofline"]["traffic_source"]
    assert res["counters"]["launches_per_step"] == 4 and res["counters"]["steps_traced"] == 2
    md = bench.counters_markdown(res, "python3 bench.py --counters d")
    assert "`adam_kernel<H16F, true>`" in md and "python3 bench.py --counters d" in md
    assert "4 kernel launches per step" in md


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_cpu_baseline_tiny_workload(bench):
    w = dict(dim=64, hidden=128, n_heads=2, kv_heads=1, head_dim=32, n_layers=1, vocab=256, seq=16, batch=2,
             qk_norm=True, rope_theta=1e6)
    out = bench.cpu_baseline("tiny", w, n_runs=2, legs=False)
    assert out["kind"] == "port" and out["unit"] == "tokens/s" and out["value"] > 0
    assert out["cores"] >= 1 and "median of 2" in out["sample"]
    json.dumps(out)
