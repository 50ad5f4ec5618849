"""Benchmark of the training step (fwd + bwd + AdamW) on one MI355X through the C-ABI.

Default workload: Qwen3-0.6B shape (dim 1024, 28 layers, GQA 16/8, head_dim 128, QK-norm,
RoPE theta 1e6, SwiGLU 3072, vocab 151936, tied LM head), batch 1 x seq 256, fp32 master
weights + fp16 activations, N(0, 0.02) weights from seed 0, fresh uniform token batches per
step.  One step = ne_train_step + ne_optimizer_step (accumulation 1).

Prints ONE JSON line.  `value` is training tokens/s; `roofline` is for AdamW, the longest
single kernel of the step, timed with HIP events on the library's stream during the timed
steps; `cpu_baseline` is the numpy oracle on this host (a bounded sample: the median of 5
full steps of the same workload after one warm-up).  Extra keys: per-family kernel times,
MFMA utilisation of the GEMM and attention kernels (against the datasheet peak and the
measured MFMA issue ceiling of ne_k_mfma_ceiling), the same step at batch 8 x seq 2048
(`at_scale`), decode tokens/s at batch 1 and 32.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu] [--no-decode]
                  [--no-scale] [--no-graphs] [--no-overlap] [--calib-copy]
"""
import argparse
import json
import math
import os
import platform
import sys
import time

# The CPU baseline's BLAS threads, fixed before numpy loads: OMP_NUM_THREADS where the
# environment sets it (a GPU box's harness fixes a process's CPU share that way), else every
# core of the host; OpenBLAS follows it.
os.environ.setdefault("OMP_NUM_THREADS", str(os.cpu_count() or 1))
os.environ.setdefault("OPENBLAS_NUM_THREADS", os.environ["OMP_NUM_THREADS"])

import numpy as np  # noqa: E402

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "neural-engine_amd"))

import ne  # noqa: E402

PEAK_HBM = 8.0e12          # MI355X HBM3E, bytes/s
PEAK_MFMA_16 = 2.5e15      # MI355X dense fp16/bf16 MFMA, flop/s
# AdamW HBM bytes per parameter: rocprofv3 FETCH_SIZE / WRITE_SIZE (copy-calibrated) on Qwen3-0.6B
# measured its algorithmic 30 B/param (profiles/train_step_qwen3-0.6b_s256_b1_counters.md)
ADAM_TRAFFIC_B_PER_PARAM = 30.0
ADAM_TRAFFIC_SOURCE = ("algorithmic (30 B/param), not measured in this run; the committed counter report "
                       "profiles/train_step_qwen3-0.6b_s256_b1_counters.md (rocprofv3 FETCH_SIZE + WRITE_SIZE, "
                       "copy-calibrated) measured the same 17.88 GB per pass; `bench.py --counters DIR` "
                       "measures it in the same invocation")

WORKLOADS = {
    "qwen3-0.6b-s256-b1": dict(dim=1024, hidden=3072, n_heads=16, kv_heads=8, head_dim=128, n_layers=28,
                               vocab=151936, seq=256, batch=1, qk_norm=True, rope_theta=1e6),
    "qwen3-0.6b-s2048-b8": dict(dim=1024, hidden=3072, n_heads=16, kv_heads=8, head_dim=128, n_layers=28,
                                vocab=151936, seq=2048, batch=8, qk_norm=True, rope_theta=1e6),
    "stories110m-s256-b1": dict(dim=768, hidden=2048, n_heads=12, kv_heads=12, head_dim=64, n_layers=12,
                                vocab=32000, seq=256, batch=1, qk_norm=False, rope_theta=1e4),
}


def layer_params(w):
    D, H, Q, KV = w["dim"], w["hidden"], w["n_heads"] * w["head_dim"], w["kv_heads"] * w["head_dim"]
    return Q * D + 2 * KV * D + D * Q + 3 * H * D + 2 * D + (2 * w["head_dim"] if w["qk_norm"] else 0)


def n_params(w):
    return w["n_layers"] * layer_params(w) + w["dim"] + w["vocab"] * w["dim"]


def flops(w):
    """Algorithmic training FLOPs per step: 3 x forward, causal attention counted once."""
    B, S, L = w["batch"], w["seq"], w["n_layers"]
    T = B * S
    D, H, Q, KV = w["dim"], w["hidden"], w["n_heads"] * w["head_dim"], w["kv_heads"] * w["head_dim"]
    mat = Q * D + 2 * KV * D + D * Q + 3 * H * D
    lin = 2 * T * (L * mat + w["vocab"] * D)
    attn = 2 * L * B * w["n_heads"] * w["head_dim"] * S * S
    return {"linear_fwd": lin, "attn_fwd": attn, "total": 3 * (lin + attn)}


def init_weights(m, w, seed=0, std=0.02):
    rng = np.random.default_rng(seed)
    for name in m.names:
        n = m.numel(name)
        if name.endswith(("rms_att", "rms_ffn", "rms_final", "q_norm", "k_norm")):
            m.set(name, np.ones(n, np.float32))
        else:
            m.set(name, rng.standard_normal(n, dtype=np.float32) * np.float32(std))


def batches(w, n, seed0=1000):
    return [np.random.default_rng(seed0 + i).integers(0, w["vocab"], (w["batch"], w["seq"] + 1)).astype(np.int32)
            for i in range(n)]


def run_train(w, steps, warmup, graphs=True, overlap=True):
    alpha = 1.0 / math.sqrt(2.0 * w["n_layers"])
    m = ne.Model(**w, res_alpha=alpha, dtype=ne.NE_FP16)
    m.use_graphs(graphs)
    m.overlap_weight_grads(overlap)
    init_weights(m, w)
    toks = batches(w, steps + warmup)
    lr = 3e-4

    def step(t):
        m.train_step(t, 256.0, want_loss=False)
        m.optimizer_step(lr, 0.9, 0.95, 1e-8, 0.1, grad_scale=1.0 / 256, clip=1.0, want_norm=False)

    for i in range(warmup):
        step(toks[i])
    m.sync()
    # timed region: only the dominant family (AdamW) carries an event pair
    m.prof_reset()
    m.prof_enable(("adam",))
    t0 = time.perf_counter()
    for i in range(steps):
        step(toks[warmup + i])
    m.sync()
    t1 = time.perf_counter()
    adam_ms, adam_n = m.prof()["adam"]
    m.prof_enable(())
    ms = (t1 - t0) * 1e3 / steps
    # per-family breakdown over two more steps with every family timed
    m.prof_reset()
    m.prof_enable()
    for i in range(2):
        step(toks[i % len(toks)])
    fam = {k: v for k, v in m.prof().items() if v[1]}
    m.prof_enable(())
    scale, skipped, sites = m.grad_scale_info()
    loss = m.train_step(toks[0], 256.0)
    upd_launches = m.update_launches()
    m.close()
    return dict(ms=ms, adam=(adam_ms, adam_n), fam=fam, skipped=skipped, scale=scale, loss=loss, sites=sites,
                upd_launches=upd_launches)


def run_decode(w, B, n_new=200, prompt_len=32, graphs=True):
    m = ne.Model(**{**w, "batch": 1, "seq": 64}, res_alpha=1.0, decode_batch=B, decode_ctx=prompt_len + n_new,
                 dtype=ne.NE_BF16)
    m.use_graphs(graphs)
    init_weights(m, w)
    prompt = np.random.default_rng(2).integers(0, w["vocab"], (B, prompt_len)).astype(np.int32)
    m.decode(prompt[:, :4], 4)                       # warm-up
    t0 = time.perf_counter()
    m.decode(prompt, n_new)
    dt = time.perf_counter() - t0
    m.close()
    return B * n_new / dt, dt


def calib_copy(nbytes=1 << 30):
    """Three device-to-device copies of nbytes (reads nbytes, writes nbytes each)."""
    import torch
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def mfma_ceiling(blocks=1024, iters=4096):
    """Measured MFMA issue ceiling (TFLOP/s) of the fp16 32x32x16 and 16x16x32 instructions:
    ne_k_mfma_ceiling, 4 waves per block x 8 independent chains, no memory traffic."""
    import ctypes
    import torch
    L = ne.lib()
    out = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
    res = {}
    for shape, name, fl in ((0, "mfma_32x32x16_tflops", 2 * 32 * 32 * 16), (1, "mfma_16x16x32_tflops", 2 * 16 * 16 * 32)):
        def go():
            rc = L.ne_k_mfma_ceiling(ne.NE_FP16, shape, blocks, iters, ctypes.c_void_p(out.data_ptr()), None)
            if rc != 0:
                raise ne.NEError(L.ne_last_error().decode())
        go()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(3):
            go()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / 3
        res[name] = blocks * 4 * 8 * iters * fl / (ms / 1e3) / 1e12
    del out
    return res


def _om_config(w):
    from oracle import model as om
    return om.Config(dim=w["dim"], hidden=w["hidden"], n_heads=w["n_heads"], kv_heads=w["kv_heads"],
                     head_dim=w["head_dim"], n_layers=w["n_layers"], vocab=w["vocab"], seq=w["seq"],
                     rope_theta=w["rope_theta"], qk_norm=w["qk_norm"],
                     res_alpha=1.0 / math.sqrt(2.0 * w["n_layers"]))


def _median_s(fn, n_runs):
    """fn() once as a warm-up, then the median wall time of n_runs calls."""
    fn()
    ts = []
    for _ in range(n_runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def _train_leg(w, n_runs, P=None):
    """Median s/step of the oracle's fwd + bwd + AdamW on fresh batches of workload w
    (P is updated in place)."""
    from oracle import model as om
    cfg = _om_config(w)
    P = om.init_params(cfg, seed=0, std=0.02) if P is None else P
    M = {k: np.zeros_like(v) for k, v in P.items()}
    V = {k: np.zeros_like(v) for k, v in P.items()}
    toks, it = batches(w, n_runs + 1), iter(range(n_runs + 1))

    def step():
        i = next(it)
        _, cache = om.forward(cfg, P, toks[i], loss_scale=256.0)
        G = om.backward(cfg, P, cache)
        del cache
        om.optimizer_step(P, G, M, V, i + 1, 3e-4, grad_scale=1.0 / 256, clip=1.0)
    return _median_s(step, n_runs)


def cpu_baseline(wname, w, n_runs=5, legs=True):
    """The numpy oracle on this host's cores, each timing the median of n_runs after one
    warm-up.  The headline value is the full training step (fwd + bwd + AdamW) of the
    benchmarked workload (about 20 s for Qwen3-0.6B, S=256).  `legs` adds the other CPU
    timings of the same plan: the Stories110M forward + cross-entropy (B=1, S=256) and its
    full training step, and the Qwen3-0.6B token loop at batch 1 and 32 (bf16-rounded
    weights held in fp32, every position one full pass with the LM head, as the oracle's
    token loop runs it) on a short sample: an 8-token prompt and 4 new tokens."""
    import dataclasses
    from oracle import model as om
    P = om.init_params(_om_config(w), seed=0, std=0.02)
    # the token loop's weights: the same seed-0 draw rounded to bf16, taken before AdamW moves P
    Pd = {k: om.round_bf16(v) for k, v in P.items()} if legs and wname.startswith("qwen3") else None
    step_s = _train_leg(w, n_runs, P=P)
    del P
    threads, blas = int(os.environ["OPENBLAS_NUM_THREADS"]), "unknown"
    try:
        from threadpoolctl import threadpool_info
        info = [d for d in threadpool_info() if d.get("user_api") == "blas"]
        if info:
            threads, blas = info[0]["num_threads"], f"{info[0]['internal_api']} {info[0].get('version')}"
    except Exception:
        pass
    out = {"value": w["batch"] * w["seq"] / step_s, "unit": "tokens/s", "cores": threads, "kind": "port",
           "host_cpus": os.cpu_count(), "blas_threads": threads,
           "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
           "sample": f"median of {n_runs} full steps (fwd+bwd+AdamW, after 1 warm-up) of {wname} on the numpy "
                     f"oracle: {step_s:.2f} s/step; numpy BLAS {blas} on {threads} threads (OMP_NUM_THREADS and "
                     f"OPENBLAS_NUM_THREADS = {os.environ.get('OMP_NUM_THREADS')}: the environment's value where it "
                     f"sets one, as the GPU box's harness does for a process's CPU share, else all "
                     f"{os.cpu_count()} host CPUs); host CPU {platform.processor() or platform.machine()}"}
    if not legs:
        return out
    res = []
    ws = WORKLOADS["stories110m-s256-b1"]
    cfg_s = _om_config(ws)
    Ps = om.init_params(cfg_s, seed=0, std=0.02)
    tok = batches(ws, 1)[0]
    fwd_s = _median_s(lambda: om.forward(cfg_s, Ps, tok, want_grad_cache=False), n_runs)
    res.append({"leg": "stories110m-s256-b1 forward + cross-entropy", "value": ws["seq"] / fwd_s,
                "unit": "tokens/s", "s_per_run": fwd_s})
    st_s = _train_leg(ws, n_runs, P=Ps)
    res.append({"leg": "stories110m-s256-b1 training step (fwd+bwd+AdamW)", "value": ws["seq"] / st_s,
                "unit": "tokens/s", "s_per_run": st_s})
    del Ps
    if wname.startswith("qwen3"):
        cfg_d = dataclasses.replace(_om_config({**w, "seq": 64}), res_alpha=1.0)
        p0, n_new = 8, 4
        for B in (1, 32):
            prompt = np.random.default_rng(2).integers(0, w["vocab"], (B, p0)).astype(np.int32)
            d_s = _median_s(lambda: om.decode(cfg_d, Pd, prompt, n_new), n_runs)
            npos = p0 + n_new - 1
            res.append({"leg": f"{wname.split('-s')[0]} token loop, batch {B} (greedy)",
                        "value": B * npos / d_s, "unit": "tokens/s (sequence positions processed)",
                        "s_per_run": d_s,
                        "sample": f"prompt {p0} + {n_new} new tokens = {npos} positions per sequence"})
    out["legs"] = res
    return out


def roofline_step(w, ms):
    """The step against its floor on one MI355X: the algorithmic FLOPs of fwd + bwd (3 x forward,
    causal attention counted once) at the dense 16-bit MFMA peak plus the AdamW pass's algorithmic
    bytes (30 B per parameter: p, g, m, v read, p, m, v and the 16-bit copy written) at the HBM
    peak, as if nothing else moved a byte and the two did not overlap."""
    fl = flops(w)["total"]
    mfma_ms = fl / PEAK_MFMA_16 * 1e3
    adam_ms = 30 * n_params(w) / PEAK_HBM * 1e3
    return {"floor_ms": mfma_ms + adam_ms, "mfma_floor_ms": mfma_ms, "adam_floor_ms": adam_ms,
            "frac": (mfma_ms + adam_ms) / ms}


def train_summary(w, r, ceiling=None):
    """Throughput, per-family kernel time and MFMA utilisation of one run_train result (against
    the datasheet peak and, when given, the measured 32x32x16 issue ceiling in TFLOP/s)."""
    fl = flops(w)
    fam_ms = {k: v[0] / 2 for k, v in r["fam"].items()}   # ms per step (2 profiled steps)
    mm_ms = sum(fam_ms.get(k, 0.0) for k in ("gemm_fwd", "gemm_bwd", "attn_fwd", "attn_bwd", "ce"))
    T = w["batch"] * w["seq"]
    return {"tokens_per_s": T / (r["ms"] / 1e3), "ms_per_step": r["ms"],
            "roofline_step": roofline_step(w, r["ms"]),
            "kernel_ms_per_step": {k: round(v, 4) for k, v in fam_ms.items()},
            "mfma_util": {"flops_per_step": fl["total"], "gemm_attn_ms_per_step": mm_ms,
                          "achieved_tflops": fl["total"] / (mm_ms / 1e3) / 1e12 if mm_ms else None,
                          "frac_of_dense_peak": fl["total"] / (mm_ms / 1e3) / PEAK_MFMA_16 if mm_ms else None,
                          "frac_of_measured_ceiling": (fl["total"] / (mm_ms / 1e3) / (ceiling * 1e12)
                                                       if mm_ms and ceiling else None),
                          "step_tflops": fl["total"] / (r["ms"] / 1e3) / 1e12}}


def _short(name):
    """Kernel name without its return type, namespace and argument list."""
    n = name.replace("(anonymous namespace)::", "")
    if n.startswith("void "):
        n = n[5:]
    if n.endswith(")"):  # drop the trailing balanced (...) group: the argument list
        depth = 0
        for i in range(len(n) - 1, -1, -1):
            depth += {")": 1, "(": -1}.get(n[i], 0)
            if depth == 0:
                n = n[:i]
                break
    return n


def counters_run(child_args, outdir, timeout_s=900):
    """The per-kernel counter report of one benchmark invocation, for the training step of its
    workload: this process never touches the GPU; it runs the benchmark as child processes under
    rocprofv3, eager launches on one stream, no decode, no CPU leg: a kernel trace with statistics, one pass
    each of the FETCH_SIZE and WRITE_SIZE counters (their bytes scaled by three plain 1 GiB
    device copies run first in the same process) and one of MfmaUtil with the fp16/bf16 MFMA
    op count.  Returns the trace run's JSON result with a `counters` object added."""
    import csv
    import subprocess
    me = [sys.executable, os.path.abspath(__file__)]
    os.makedirs(outdir, exist_ok=True)
    # one stream, eager: every kernel runs alone, so a row's duration, counters and rates belong
    # to that kernel (with the second stream, overlapping kernels stretch each other's durations)
    run = me + child_args + ["--no-graphs", "--no-overlap", "--no-cpu", "--no-decode", "--no-scale"]
    pmc_run = run + ["--steps", "3", "--warmup", "1"]

    def prof(key, what):
        return ["rocprofv3"] + what + ["-f", "csv", "-d", os.path.join(outdir, key), "-o", "run", "--"]
    cmds = {
        "trace": prof("trace", ["--kernel-trace", "--stats"]) + run,
        "fetch": prof("fetch", ["--pmc", "FETCH_SIZE"]) + pmc_run + ["--calib-copy"],
        "write": prof("write", ["--pmc", "WRITE_SIZE"]) + pmc_run + ["--calib-copy"],
        "mfma": prof("mfma", ["--pmc", "MfmaUtil", "SQ_INSTS_VALU_MFMA_MOPS_F16"]) + pmc_run,
    }
    result = None
    for key, cmd in cmds.items():
        print(f"[counters] {key}: {' '.join(cmd)}", file=sys.stderr, flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout_s)
        lines = [l for l in r.stdout.splitlines() if l.startswith("{")]
        if not lines:
            raise RuntimeError(f"rocprofv3 {key} pass printed no result (rc {r.returncode}): {r.stderr[-2000:]}")
        if key == "trace":
            result = json.loads(lines[-1])
    shown = {k: " ".join(v).replace(me[1], "bench.py").replace(sys.executable, "python3") for k, v in cmds.items()}
    return counters_collect(outdir, result, shown)


def counters_collect(outdir, result, commands):
    """Join the trace and counter passes under outdir into result["counters"] (see counters_run)."""
    import csv
    stats = []
    with open(os.path.join(outdir, "trace", "run_kernel_stats.csv")) as f:
        for row in csv.DictReader(f):
            stats.append({"kernel": _short(row["Name"]), "calls": int(row["Calls"]),
                          "avg_us": float(row["AverageNs"]) / 1e3, "total_ms": float(row["TotalDurationNs"]) / 1e6,
                          "pct": float(row["Percentage"])})
    stats.sort(key=lambda d: -d["total_ms"])
    avg_us = {d["kernel"]: d["avg_us"] for d in stats}
    # launches per step: the dispatches from one embedding lookup to the next (a training step and
    # its optimizer step), without the runtime's copies and the MFMA-ceiling measurement
    with open(os.path.join(outdir, "trace", "run_kernel_trace.csv")) as f:
        disp = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    names = [_short(r["Kernel_Name"]) for r in disp]
    starts = [i for i, n in enumerate(names) if n.startswith("embed_fwd")]
    per_step = [sum(1 for n in names[a:b] if not n.startswith(("__amd_rocclr", "mfma_ceiling")))
                for a, b in zip(starts, starts[1:])]

    def pmc(key):
        """{kernel: {counter: (sum over dispatches, dispatches)}} of a counter pass, and the
        per-dispatch values of the device copies."""
        per, copies = {}, []
        for r in csv.DictReader(open(os.path.join(outdir, key, "run_counter_collection.csv"))):
            k = _short(r["Kernel_Name"])
            c = per.setdefault(k, {})
            s_, n_ = c.get(r["Counter_Name"], (0.0, 0))
            c[r["Counter_Name"]] = (s_ + float(r["Counter_Value"]), n_ + 1)
            if "copyBuffer" in k:
                copies.append(float(r["Counter_Value"]))
        return per, copies

    def copy_scale(copies):
        """Bytes per counter unit: the three 1 GiB copies are the three largest copy dispatches."""
        vals = sorted(copies, reverse=True)[:3]
        return (1 << 30) / (sum(vals) / len(vals)) if len(vals) == 3 else None
    (fetch, fc), (write, wc), (mfma, _) = pmc("fetch"), pmc("write"), pmc("mfma")
    fs, wsc = copy_scale(fc), copy_scale(wc)
    rows = []
    for d in stats:
        k = d["kernel"]
        row = dict(d)
        if k in fetch and "FETCH_SIZE" in fetch[k] and fs:
            v, n = fetch[k]["FETCH_SIZE"]
            row["read_MB_per_launch"] = v / n * fs / 1e6
        if k in write and "WRITE_SIZE" in write[k] and wsc:
            v, n = write[k]["WRITE_SIZE"]
            row["write_MB_per_launch"] = v / n * wsc / 1e6
        if k in mfma and "MfmaUtil" in mfma[k]:
            v, n = mfma[k]["MfmaUtil"]
            row["mfma_util_pct"] = v / n
            if "SQ_INSTS_VALU_MFMA_MOPS_F16" in mfma[k]:
                v, n = mfma[k]["SQ_INSTS_VALU_MFMA_MOPS_F16"]
                row["mfma_tflops"] = v / n * 512 / (avg_us[k] * 1e-6) / 1e12
        if "read_MB_per_launch" in row and "write_MB_per_launch" in row:
            gbs = (row["read_MB_per_launch"] + row["write_MB_per_launch"]) * 1e6 / (d["avg_us"] * 1e-6) / 1e9
            row["hbm_GBps"] = gbs
            row["hbm_frac"] = gbs * 1e9 / PEAK_HBM
        rows.append(row)
    result["counters"] = {"kernels": rows[:40],
                          "launches_per_step": sorted(per_step)[len(per_step) // 2] if per_step else None,
                          "steps_traced": len(per_step),
                          "calibration": {"fetch_bytes_per_unit": fs, "write_bytes_per_unit": wsc,
                                          "how": "three 1 GiB device copies (__amd_rocclr_copyBuffer) in the "
                                                 "byte-counter passes"},
                          "commands": commands}
    # the roofline kernel's HBM traffic per pass, from the counter passes
    rk = result["roofline"]["kernel"].split(" ")[0]
    for row in rows:
        if row["kernel"].split("<")[0] == rk and "read_MB_per_launch" in row and "write_MB_per_launch" in row:
            result["roofline"]["traffic"] = (row["read_MB_per_launch"] + row["write_MB_per_launch"]) * 1e6 * \
                result["roofline"]["launches_per_pass"]
            result["roofline"]["traffic_source"] = ("rocprofv3 FETCH_SIZE + WRITE_SIZE of this invocation's counter "
                                                    "passes, copy-calibrated, mean per launch x launches per pass")
    return result


def counters_markdown(res, made_by):
    """A short text summary of a counters_run result (for profiles/); made_by: the command."""
    c = res["counters"]
    cal = c["calibration"]
    out = [f"# rocprofv3 per-kernel report: training step of {res['config']['workload']}", "",
           f"Made by `{made_by}` (one run: its child processes below).", "",
           f"Traced run (eager launches on one stream: each kernel runs alone, so its duration, counters and "
           f"rates are its own): {res['ms_per_step']:.3f} ms per step, {c['launches_per_step']} kernel launches per "
           f"step (a training step and its optimizer step; median over {c['steps_traced']} traced steps, the runtime's "
           "copies not counted; the two-stream schedule runs the same kernels with the AdamW pass in "
           f"{res['roofline'].get('update_launches', 'L + 1 + P')} launches instead of one).", "",
           "Commands of the child processes:", ""]
    out += [f"    {v}" for v in c["commands"].values()]
    out += ["", "Durations from the kernel trace; HBM bytes per launch from FETCH_SIZE and WRITE_SIZE scaled by "
            f"{cal['fetch_bytes_per_unit']:.0f} and {cal['write_bytes_per_unit']:.0f} bytes per counter unit (the "
            "factors that make three 1 GiB device copies read and write 1 GiB each); MfmaUtil as rocprofv3 derives "
            "it; MFMA TFLOP/s = SQ_INSTS_VALU_MFMA_MOPS_F16 x 512 / average duration; HBM GB/s = (read + write) / "
            "average duration, and its fraction of the 8 TB/s peak.", "",
            "| kernel | calls | avg µs | total ms | % | read MB | write MB | HBM GB/s | of peak | MfmaUtil % | "
            "MFMA TFLOP/s |",
            "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]

    def f(d, k, fmt):
        return format(d[k], fmt) if k in d else "–"
    out += [f"| `{d['kernel']}` | {d['calls']} | {d['avg_us']:.2f} | {d['total_ms']:.2f} | {d['pct']:.2f} | "
            f"{f(d, 'read_MB_per_launch', '.2f')} | {f(d, 'write_MB_per_launch', '.2f')} | "
            f"{f(d, 'hbm_GBps', '.0f')} | {f(d, 'hbm_frac', '.2f')} | "
            f"{f(d, 'mfma_util_pct', '.1f')} | {f(d, 'mfma_tflops', '.0f')} |" for d in c["kernels"]]
    r = res["roofline"]
    out += ["", f"Roofline kernel `{r['kernel'].split(' ')[0]}`: {r['achieved']:.0f} GB/s of {r['peak']:.0f} "
            f"(frac {r['frac']:.3f}) in the traced run; HBM traffic per pass "
            f"{r['traffic'] / 1e9 if r['traffic'] else float('nan'):.2f} GB against {r['bytes_per_pass'] / 1e9:.2f} GB "
            "algorithmic.", ""]
    return "\n".join(out)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="qwen3-0.6b-s256-b1", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-scale", action="store_true",
                    help="skip the extra Qwen3-0.6B batch 8 x seq 2048 step measurement")
    ap.add_argument("--no-graphs", action="store_true",
                    help="launch the step's kernels one by one instead of replaying a captured HIP graph "
                         "(for tracers that do not follow graph launches)")
    ap.add_argument("--no-overlap", action="store_true",
                    help="run the weight-gradient GEMMs in order on the step's stream instead of on a "
                         "second stream beside the activation-gradient chain")
    ap.add_argument("--counters", metavar="DIR",
                    help="run this benchmark under rocprofv3 as child processes (kernel statistics and HBM byte "
                         "counters, written under DIR) and add the per-kernel report to the result")
    ap.add_argument("--counters-md", metavar="FILE", help="with --counters: also write the report as text to FILE")
    ap.add_argument("--calib-copy", action="store_true",
                    help="first run three plain 1 GiB device copies (a known-size kernel that scales "
                         "the FETCH_SIZE / WRITE_SIZE counters of a --pmc run)")
    a = ap.parse_args()
    if a.counters:
        child, skip = [], False
        for x in sys.argv[1:]:
            if skip:
                skip = False
                continue
            if x in ("--counters", "--counters-md"):
                skip = True
                continue
            if x.startswith(("--counters=", "--counters-md=")):
                continue
            child.append(x)
        res = counters_run(child, a.counters)
        if a.counters_md:
            with open(a.counters_md, "w") as f:
                f.write(counters_markdown(res, " ".join(["python3", "bench.py"] + sys.argv[1:])))
        print(json.dumps(res), flush=True)
        return
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(data-parallel sharding is a design note); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    w = WORKLOADS[a.workload]
    T = w["batch"] * w["seq"]
    # torch (its own HIP runtime) must initialise the device before the library does
    if a.calib_copy:
        calib_copy()
    ceil = mfma_ceiling()
    r = run_train(w, a.steps, a.warmup, graphs=not a.no_graphs, overlap=not a.no_overlap)
    summ = train_summary(w, r, ceil["mfma_32x32x16_tflops"])
    npar = n_params(w)
    fam_ms = summ["kernel_ms_per_step"]
    dom = max(fam_ms, key=fam_ms.get)
    # One AdamW pass per step, run by the next step beside its forward on the second stream in
    # ne_update_launches launches (the gains, one per layer, the embedding's rows in the
    # classifier's vocabulary pieces; capped at 384 work-groups each), between one event pair (a
    # pair per launch cost the step 0.22 ms); the last pass of the timed steps runs after them in
    # one launch.  Pass time: the pair's span, gaps included.
    passes = max(r["adam"][1], 1)
    adam_launches = 1 if a.no_overlap else r["upd_launches"]   # one stream: the pass in one launch
    adam_ms = r["adam"][0] / passes
    adam_bytes = 30 * npar                                 # read p,g,m,v; write p,m,v + 16-bit shadow
    roofline = {"bound": "hbm",
                "kernel": ("adam_kernel (fused AdamW; one pass over all parameters per step, in one launch after "
                           "the step on one stream)" if a.no_overlap else
                           "adam_kernel (fused AdamW; one pass over all parameters per step, run beside the next "
                           f"step's forward in {adam_launches} launches: the gains, one per layer, the embedding's "
                           "rows in the classifier's vocabulary pieces, each capped at 384 work-groups; timed by "
                           "one event pair around the pass)"),
                "achieved": adam_bytes / (adam_ms / 1e3) / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                "frac": adam_bytes / (adam_ms / 1e3) / PEAK_HBM,
                "traffic": ADAM_TRAFFIC_B_PER_PARAM * npar,
                "traffic_source": ADAM_TRAFFIC_SOURCE,
                "bytes_per_pass": adam_bytes, "pass_ms": adam_ms, "launches_per_pass": adam_launches,
                "bytes_per_launch": adam_bytes / adam_launches, "avg_launch_ms": adam_ms / adam_launches,
                "update_launches": r["upd_launches"]}
    out = {
        "metric": "Qwen3-0.6B train tokens/s + step ms on 1 MI355X; MFMA util %; decode tok/s",
        "value": summ["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": r["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: N(0,0.02) weights from seed 0, uniform token ids (fresh batch per step)",
        "config": {"workload": a.workload, "global_batch": w["batch"], "seq_len": w["seq"],
                   "tokens_per_step": w["batch"] * w["seq"], "params": npar, "parallelism": "single GPU",
                   "precision": "fp32 master weights + AdamW state, fp16 activations/operands, fp32 accumulate "
                                "(fp16 is the training format; bf16 operands are supported, with their Wq/Wk/QK-norm "
                                "gradients tested at 4e-2 relative L2 instead of 1e-2)"},
        "roofline": roofline,
        "dominant_family": dom,
        "kernel_ms_per_step": fam_ms,
        "mfma_util": summ["mfma_util"],
        "mfma_ceiling": {**ceil, "datasheet_tflops": PEAK_MFMA_16 / 1e12,
                         "how": "ne_k_mfma_ceiling: 1024 blocks x 4 waves x 8 independent fp16 MFMA chains, "
                                "no memory traffic"},
        "grad_scale": r["scale"], "skipped_steps": r["skipped"], "overflow_sites": r["sites"],
        "loss_last": r["loss"],
    }
    out["roofline_step"] = summ["roofline_step"]
    if not a.no_scale and a.workload == "qwen3-0.6b-s256-b1":
        ws = WORKLOADS["qwen3-0.6b-s2048-b8"]
        rs = run_train(ws, 3, 1, graphs=not a.no_graphs, overlap=not a.no_overlap)
        out["at_scale"] = {"workload": "qwen3-0.6b-s2048-b8", "tokens_per_step": ws["batch"] * ws["seq"],
                           **train_summary(ws, rs, ceil["mfma_32x32x16_tflops"])}
    if not a.no_decode and a.workload.startswith("qwen3"):
        P, n_new = 32, 200
        d1, t1 = run_decode(w, 1, n_new, P, graphs=not a.no_graphs)
        d32, t32 = run_decode(w, 32, n_new, P, graphs=not a.no_graphs)
        gains = w["n_layers"] * (2 * w["dim"] + (2 * w["head_dim"] if w["qk_norm"] else 0)) + w["dim"]
        wbytes = 2 * (npar - gains)                          # bf16 matrices read once per position
        lm = 2 * w["vocab"] * w["dim"]                       # the LM head: generated positions only
        npos = P - 1 + n_new                                 # positions run one at a time

        def loop_bytes(B):
            """HBM bytes of one decode call: the weights once per position (all sequences share
            them), plus each sequence's fp32 K and V cache rows read by attention."""
            kv_row = 2 * w["n_layers"] * w["kv_heads"] * w["head_dim"] * 4
            kv = B * kv_row * sum(p + 1 for p in range(npos))
            return (P - 1) * (wbytes - lm) + n_new * wbytes + kv

        def roof(B, dt):
            byt = loop_bytes(B)
            return {"bound": "hbm", "bytes_per_call": byt, "positions": npos, "us_per_position": dt / npos * 1e6,
                    "achieved_GBps": byt / dt / 1e9, "frac": byt / dt / PEAK_HBM}
        out["decode"] = {"tokens_per_s_b1": d1, "tokens_per_s_b32": d32, "prompt": P, "new_tokens": n_new,
                         "weights": "bf16", "roofline_b1": roof(1, t1), "roofline_b32": roof(32, t32)}
    if not a.no_cpu:
        out["cpu_baseline"] = cpu_baseline(a.workload, w)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
