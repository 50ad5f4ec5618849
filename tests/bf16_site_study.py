"""Where the bf16 step's gradient error comes from (CPU only; the oracle with the device's
16-bit rounding points, oracle.model.ROUND_SITES).

For Stories110M and Qwen3-0.6B at batch 1 x 256 tokens (N(0, 0.02) weights from seed 0), the
reference is the fp32 oracle on the weights rounded to bf16 (what the device multiplies); each
row rounds one site of the forward or backward to bf16 on top of it, and the last rows round
every site (the device's bf16 step), every site but the largest contributors, and every site
in fp16 (the backward sites at the device's internal gradient scale 256).  Reported: the
largest per-tensor gradient relative L2 against the reference, over all tensors and over
the attention-score tensors (Wq, Wk, q_norm, k_norm), each with the tensor.

    python3 tests/bf16_site_study.py [--models stories,qwen3] [--md FILE]
"""
import argparse
import os
import sys
import time

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
from oracle import model as om  # noqa: E402

BWD = {"dlogits", "dbf", "dh13", "datt", "p_bwd", "ds", "dv", "dqk"}


def rounder(sites, fmt="bf16", gs=256.0):
    sites = set(sites)

    def r(site, x):
        if site not in sites:
            return x
        if fmt == "bf16":
            return om.round_bf16(np.asarray(x, np.float32))
        s = np.float32(gs if site in BWD else 1.0)
        return ((np.asarray(x, np.float32) * s).astype(np.float16).astype(np.float32) / s).astype(np.float32)
    return r


def grads(cfg, P, tok, sites=(), fmt="bf16"):
    r = rounder(sites, fmt)
    _, cache = om.forward(cfg, P, tok, loss_scale=256.0, rnd=r)
    return om.backward(cfg, P, cache, rnd=r)


def worst(G, G0, names=None):
    best = (0.0, "")
    for n in (names or G0):
        d = float(np.linalg.norm(G[n] - G0[n]) / max(np.linalg.norm(G0[n]), 1e-30))
        best = max(best, (d, n))
    return best


def study(name, cfg):
    P = om.init_params(cfg, seed=0, std=0.02)
    Pb = {k: (v if om.is_gain(k) else om.round_bf16(v)) for k, v in P.items()}
    tok = om.tokens_for_step(cfg, 1, cfg.seq, seed=1)
    t0 = time.time()
    G0 = grads(cfg, Pb, tok)
    att = [n for n in G0 if n.split(".")[-1] in ("Wq", "Wk", "q_norm", "k_norm")]
    rows = []

    def add(label, sites, fmt="bf16"):
        G = grads(cfg, Pb, tok, sites, fmt)
        a, b = worst(G, G0), worst(G, G0, att)
        rows.append((label, a, b))
        print(f"  [{name}] {label:28s} all {a[0]:.2e} ({a[1]})  attention-score {b[0]:.2e} ({b[1]})  "
              f"{time.time() - t0:.0f}s", flush=True)
        return a[0]
    per = {s: add(s, [s]) for s in om.ROUND_SITES}
    add("every site (device bf16)", om.ROUND_SITES)
    top = sorted(per, key=per.get, reverse=True)[:3]
    for k in (1, 2, 3):
        keep = top[:k]
        add("every site but " + "+".join(keep), [s for s in om.ROUND_SITES if s not in keep])
    add("every site, fp16", om.ROUND_SITES, "fp16")
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--models", default="stories,qwen3")
    ap.add_argument("--md", help="write the tables as markdown to this file")
    a = ap.parse_args()
    cfgs = {"stories": ("Stories110M, B=1, S=256", om.stories110m(seq=256, res_alpha=om.train_alpha(12))),
            "qwen3": ("Qwen3-0.6B, B=1, S=256", om.qwen3_06b(seq=256, res_alpha=om.train_alpha(28)))}
    out = []
    for m in a.models.split(","):
        title, cfg = cfgs[m]
        rows = study(m, cfg)
        out += [f"**{title}** (reference: the fp32 oracle on bf16-rounded weights)", "",
                "| rounded to 16 bits | worst gradient rel-L2 (tensor) | worst of Wq, Wk, q/k_norm (tensor) |",
                "|---|---|---|"]
        out += [f"| {l} | {x[0]:.2e} ({x[1]}) | {y[0]:.2e} ({y[1]}) |" for l, x, y in rows]
        out.append("")
    if a.md:
        with open(a.md, "w") as f:
            f.write("\n".join(out) + "\n")
    print("\n".join(out))


if __name__ == "__main__":
    main()
