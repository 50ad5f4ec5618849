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

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "neural-engine_amd"))

import ne  # noqa: E402

PEAK_HBM = 8.0e12          # MI355X HBM3E, bytes/s
PEAK_MFMA_16 = 2.5e15      # MI355X dense fp16/bf16 MFMA, flop/s
# AdamW HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE (copy-calibrated)
# on Qwen3-0.6B: equal to its algorithmic 30 B/param (profiles/adam_hbm_counters_qwen3-0.6b.md)
ADAM_TRAFFIC_B_PER_PARAM = 30.0

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
    m.close()
    return dict(ms=ms, adam=(adam_ms, adam_n), fam=fam, skipped=skipped, scale=scale, loss=loss, sites=sites)


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


def cpu_baseline(wname, w, n_runs=5):
    """The numpy oracle (fwd + bwd + AdamW) on this host's cores: one warm-up step, then the
    median of n_runs full steps of the same workload (about 20 s for Qwen3-0.6B, S=256)."""
    from oracle import model as om
    cfg = om.Config(dim=w["dim"], hidden=w["hidden"], n_heads=w["n_heads"], kv_heads=w["kv_heads"],
                    head_dim=w["head_dim"], n_layers=w["n_layers"], vocab=w["vocab"], seq=w["seq"],
                    rope_theta=w["rope_theta"], qk_norm=w["qk_norm"], res_alpha=1.0 / math.sqrt(2.0 * w["n_layers"]))
    P = om.init_params(cfg, seed=0, std=0.02)
    M = {k: np.zeros_like(v) for k, v in P.items()}
    V = {k: np.zeros_like(v) for k, v in P.items()}
    times = []
    for i, tok in enumerate(batches(w, n_runs + 1)):
        t0 = time.perf_counter()
        _, cache = om.forward(cfg, P, tok, loss_scale=256.0)
        G = om.backward(cfg, P, cache)
        del cache
        om.optimizer_step(P, G, M, V, i + 1, 3e-4, grad_scale=1.0 / 256, clip=1.0)
        if i > 0:
            times.append(time.perf_counter() - t0)
        del G
    step_s = float(np.median(times))
    threads, blas = os.cpu_count() or 1, "unknown"
    try:
        from threadpoolctl import threadpool_info
        info = [d for d in threadpool_info() if d.get("user_api") == "blas"]
        if info:
            threads, blas = info[0]["num_threads"], f"{info[0]['internal_api']} {info[0].get('version')}"
    except Exception:
        pass
    return {"value": w["batch"] * w["seq"] / step_s, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"median of {n_runs} full steps (fwd+bwd+AdamW, after 1 warm-up) of {wname} on the numpy "
                      f"oracle: {step_s:.2f} s/step; numpy BLAS {blas}, {threads} threads; "
                      f"host CPU {platform.processor() or platform.machine()}"}


def train_summary(w, r, ceiling=None):
    """Throughput, per-family kernel time and MFMA utilisation of one run_train result (against
    the datasheet peak and, when given, the measured 32x32x16 issue ceiling in TFLOP/s)."""
    fl = flops(w)
    fam_ms = {k: v[0] / 2 for k, v in r["fam"].items()}   # ms per step (2 profiled steps)
    mm_ms = sum(fam_ms.get(k, 0.0) for k in ("gemm_fwd", "gemm_bwd", "attn_fwd", "attn_bwd", "ce"))
    T = w["batch"] * w["seq"]
    return {"tokens_per_s": T / (r["ms"] / 1e3), "ms_per_step": r["ms"],
            "kernel_ms_per_step": {k: round(v, 4) for k, v in fam_ms.items()},
            "mfma_util": {"flops_per_step": fl["total"], "gemm_attn_ms_per_step": mm_ms,
                          "achieved_tflops": fl["total"] / (mm_ms / 1e3) / 1e12 if mm_ms else None,
                          "frac_of_dense_peak": fl["total"] / (mm_ms / 1e3) / PEAK_MFMA_16 if mm_ms else None,
                          "frac_of_measured_ceiling": (fl["total"] / (mm_ms / 1e3) / (ceiling * 1e12)
                                                       if mm_ms and ceiling else None),
                          "step_tflops": fl["total"] / (r["ms"] / 1e3) / 1e12}}


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
    ap.add_argument("--calib-copy", action="store_true",
                    help="first run three plain 1 GiB device copies (a known-size kernel that scales "
                         "the FETCH_SIZE / WRITE_SIZE counters of a --pmc run)")
    a = ap.parse_args()
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
    # one AdamW pass per step: 29 launches (embedding + gains, then one per layer) on the second
    # stream, each between its own event pair; the pass time is the sum of their durations
    adam_launches = max(r["adam"][1], 1) / a.steps
    adam_ms = r["adam"][0] / a.steps
    adam_bytes = 30 * npar                                 # read p,g,m,v; write p,m,v + 16-bit shadow
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
                   "precision": "fp32 master weights + AdamW state, fp16 activations/operands, fp32 accumulate"},
        "roofline": {"bound": "hbm",
                     "kernel": "adam_kernel (fused AdamW; one pass over all parameters per step, in "
                               f"{adam_launches:.0f} launches: embedding + gains, then one per layer)",
                     "achieved": adam_bytes / (adam_ms / 1e3) / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                     "frac": adam_bytes / (adam_ms / 1e3) / PEAK_HBM,
                     "traffic": ADAM_TRAFFIC_B_PER_PARAM * npar,
                     "traffic_source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, copy-calibrated "
                                       "(profiles/adam_hbm_counters_qwen3-0.6b.md)",
                     "bytes_per_pass": adam_bytes, "pass_ms": adam_ms, "launches_per_pass": adam_launches,
                     "bytes_per_launch": adam_bytes / adam_launches, "avg_launch_ms": adam_ms / adam_launches},
        "dominant_family": dom,
        "kernel_ms_per_step": fam_ms,
        "mfma_util": summ["mfma_util"],
        "mfma_ceiling": {**ceil, "datasheet_tflops": PEAK_MFMA_16 / 1e12,
                         "how": "ne_k_mfma_ceiling: 1024 blocks x 4 waves x 8 independent fp16 MFMA chains, "
                                "no memory traffic"},
        "grad_scale": r["scale"], "skipped_steps": r["skipped"], "overflow_sites": r["sites"],
        "loss_last": r["loss"],
    }
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
