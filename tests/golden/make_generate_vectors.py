"""Writes tests/golden/generate_tiny.json from the reference's own numpy decoder.

Run in a container that holds the reference checkout (never on the GPU box):
    python tests/golden/make_generate_vectors.py /root/reference

What it does:
  1. builds a tiny v4 checkpoint with the oracle's writer (oracle/ckpt.py), with the
     GQA dims duplicated into the header slots generate.py:28 actually reads;
  2. loads the reference's TD/tools/generate.py as a module (its module-level
     imports are argparse/struct/sys/numpy/pathlib only; main() is not called,
     so no tokenizer or network is touched);
  3. reads the checkpoint back with the reference's read_checkpoint() and records
     sample values (pins the byte layout), then runs the reference's generate()
     greedily and with two sampling settings, recording the token streams.

The fixture is data (config, seeds, prompt, sampled weight values, token streams);
no reference source travels with it.
"""
import importlib.util
import io
import json
import os
import sys
import tempfile
from contextlib import redirect_stdout

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import ckpt, model as om  # noqa: E402

GEN_REL = "ane-training/training/training_dynamic/tools/generate.py"

CFG = om.Config(dim=64, hidden=128, n_heads=4, kv_heads=2, head_dim=16, n_layers=2, vocab=256,
                seq=64, rope_theta=10000.0, qk_norm=False, res_alpha=1.0)
WEIGHT_SEED, WEIGHT_STD = 21, 0.08
PROMPT = [5, 17, 99, 3, 200]
N_NEW = 24
SAMPLES = [("greedy", 0.0, 1.0, None), ("t08_p09_s11", 0.8, 0.9, 11), ("t06_p10_s3", 0.6, 1.0, 3)]
PROBES = [("layers.0.Wq", (3, 5)), ("layers.0.Wk", (31, 60)), ("layers.1.Wo", (10, 63)),
          ("layers.1.W2", (7, 100)), ("layers.1.W3", (127, 0)), ("rms_final", (9,)),
          ("embed", (255, 63)), ("embed", (0, 0))]


class _Tok:
    eos_token_id = -1

    def decode(self, ids):
        return ""


def main(ref_root):
    spec = importlib.util.spec_from_file_location("ref_generate", os.path.join(ref_root, GEN_REL))
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)

    P = om.init_params(CFG, seed=WEIGHT_SEED, std=WEIGHT_STD)
    Z = {k: np.zeros_like(v) for k, v in P.items()}
    out = {"config": {k: getattr(CFG, k) for k in ("dim", "hidden", "n_heads", "kv_heads", "head_dim",
                                                  "n_layers", "vocab", "seq", "rope_theta")},
           "weight_seed": WEIGHT_SEED, "weight_std": WEIGHT_STD, "prompt": PROMPT, "n_new": N_NEW}
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "tiny.bin")
        # generate.py:28 unpacks kv_heads/head_dim/q_dim from header fields 15:18, which
        # TD/config.h:82-91 defines as cum_steps/cum_batches/adam_t (the GQA fields are
        # 18:21).  Writing the GQA values into both slots lets the reference read this file.
        ckpt.write(path, CFG, P, Z, Z, cum_steps=CFG.kv_heads, cum_batches=CFG.head_dim,
                   adam_t=CFG.q_dim)
        with redirect_stdout(io.StringIO()):
            info, layers, rms_final, embed = gen.read_checkpoint(path)
    ref = {"rms_final": rms_final, "embed": embed}
    for l, layer in enumerate(layers):
        for k, v in layer.items():
            ref[f"layers.{l}.{k}"] = v
    out["probes"] = [[n, list(ix), float(ref[n][ix])] for n, ix in PROBES]
    out["streams"] = {}
    for name, temp, top_p, seed in SAMPLES:
        if seed is not None:
            np.random.seed(seed)
        with redirect_stdout(io.StringIO()):
            toks = gen.generate(info, layers, rms_final, embed, _Tok(), list(PROMPT), N_NEW, temp, top_p)
        out["streams"][name] = {"temp": temp, "top_p": top_p, "seed": seed,
                                "tokens": [int(t) for t in toks]}
    with open(os.path.join(HERE, "generate_tiny.json"), "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", os.path.join(HERE, "generate_tiny.json"))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
