"""Writes tests/golden/decode_qwen3_greedy.npz: the oracle's greedy token streams for the
Qwen3-0.6B token loop (200 new tokens after a 32-token prompt, batch 1 and batch 32).

    python tests/golden/make_decode_fixture.py

Workload: Qwen3-0.6B shape (dim 1024, 28 layers, GQA 16/8 heads of 128, QK-RMSNorm, RoPE theta
1e6, vocab 151936, residual scale 1 as in generate.py), N(0, 0.02) weights from
default_rng(0) in checkpoint order rounded to bf16 (the form the device holds them in),
prompts from default_rng(2) uniform in [0, vocab).  The oracle (oracle/model.py decode, a
restatement of TD/tools/generate.py:113-228) runs in fp32 with float64 RoPE angles, as
generate.py does.  Saved per batch size: the prompt, the tokens and each step's top-2 logit
margin (how close the argmax was to a tie).  The fixture is data only.
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import model as om  # noqa: E402

N_NEW, P0 = 200, 32


def main():
    cfg = om.qwen3_06b(res_alpha=1.0)
    P = {k: om.round_bf16(v) for k, v in om.init_params(cfg, seed=0, std=0.02).items()}
    out = {}
    for B in (1, 32):
        prompt = np.random.default_rng(2).integers(0, cfg.vocab, (B, P0)).astype(np.int32)
        t0 = time.time()
        tok, margins, _ = om.decode(cfg, P, prompt, N_NEW, return_logits=True)
        print(f"B={B}: {time.time() - t0:.0f} s, min top-2 margin {margins.min():.3e}", flush=True)
        out[f"prompt_b{B}"] = prompt
        out[f"tokens_b{B}"] = tok.astype(np.int32)
        out[f"margins_b{B}"] = margins.astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "decode_qwen3_greedy.npz"), **out)


if __name__ == "__main__":
    main()
