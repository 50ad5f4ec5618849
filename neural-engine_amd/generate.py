#!/usr/bin/env python3
"""generate.py - text generation from a v4 training checkpoint on one MI355X (ne_decode).

The command line of the reference's TD/tools/generate.py (TD = ane-training/training/
training_dynamic): a positional checkpoint path, --model/-m (tokenizer), --prompt/-p,
--tokens/-n (max new tokens, default 100), --temp/-t (default 0.8, 0 = greedy), --top-p
(default 0.9), --seed (generate.py:236-245), the same prints around the generated text
(generate.py:266-282), the same sampling semantics - softmax(logits/temp), the top-p mask
of generate.py:205-213, one draw of numpy's global RandomState per token
(generate.py:215, seeded by --seed as generate.py:249 does) - and the stop at the
tokenizer's EOS (generate.py:223-225).  The decode loop (KV cache, GEMVs, sampling) runs on
the GPU through the C-ABI; the weights come from the checkpoint's fp32 tensors, held in a
16-bit shadow (fp16 by default, --bf16 for bf16) with fp32 activations and KV cache.

Offline tokenizer I/O: --model takes a local tokenizer directory (loaded with
transformers' AutoTokenizer, local files only; the reference's from_pretrained(name)
needs the network).  Without --model, --prompt-ids gives the prompt as comma-separated
token ids and the generated ids are printed.  Extensions: --prompt-ids, --eos ID (stop
token when no tokenizer gives one), --rope-theta (the v4 header does not record it;
generate.py's rope uses 10000), --bf16.
"""
import argparse
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)

import ne  # noqa: E402


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description="Generate text from an ANE-format (v4) checkpoint on the GPU")
    ap.add_argument("checkpoint", help="Path to the v4 checkpoint (.bin)")
    ap.add_argument("--model", "-m", default=None, help="local tokenizer directory (offline)")
    ap.add_argument("--prompt", "-p", default="Once upon a time", help="Text prompt (needs --model)")
    ap.add_argument("--prompt-ids", default=None, help="prompt as comma-separated token ids")
    ap.add_argument("--tokens", "-n", type=int, default=100, help="Max tokens to generate (default: 100)")
    ap.add_argument("--temp", "-t", type=float, default=0.8, help="Sampling temperature (default: 0.8, 0=greedy)")
    ap.add_argument("--top-p", type=float, default=0.9, help="Top-p nucleus sampling (default: 0.9)")
    ap.add_argument("--seed", type=int, default=None, help="Random seed for reproducibility")
    ap.add_argument("--eos", type=int, default=None, help="stop token id (default: the tokenizer's EOS)")
    ap.add_argument("--rope-theta", type=float, default=10000.0, help="RoPE base (default: 10000)")
    ap.add_argument("--bf16", action="store_true", help="bf16 weight shadow instead of fp16")
    return ap.parse_args(argv)


def sampling_uniforms(n, seed):
    """The draws numpy's np.random.choice(vocab, p=probs) makes after np.random.seed(seed):
    one random_sample() per generated token."""
    return np.random.RandomState(seed).random_sample(n)


def main(argv=None):
    a = parse_args(argv)
    tok = None
    if a.model:
        try:
            from transformers import AutoTokenizer
        except ImportError:
            print("transformers is needed for --model (or give --prompt-ids)")
            return 1
        print(f"Loading tokenizer: {a.model}")
        tok = AutoTokenizer.from_pretrained(a.model, local_files_only=True, trust_remote_code=True)
    if a.prompt_ids is not None:
        prompt = [int(x) for x in a.prompt_ids.replace(" ", "").split(",") if x]
        prompt_text = tok.decode(prompt) if tok else " ".join(map(str, prompt))
    elif tok is not None:
        prompt = list(tok.encode(a.prompt))
        prompt_text = a.prompt
    else:
        print("Give --model (a local tokenizer directory) or --prompt-ids")
        return 1
    if not prompt or a.tokens < 1:
        print("Empty prompt or no tokens to generate")
        return 1
    eos = a.eos if a.eos is not None else (tok.eos_token_id if tok is not None else None)

    h = ne.read_ckpt_header(a.checkpoint)
    m = ne.Model(dim=h["dim"], hidden=h["hidden"], n_heads=h["n_heads"], kv_heads=h["kv_heads"],
                 head_dim=h["head_dim"], n_layers=h["n_layers"], vocab=h["vocab"], seq=64, batch=1,
                 qk_norm=h["qk_norm"], rope_theta=a.rope_theta, res_alpha=1.0, decode_batch=1,
                 decode_ctx=len(prompt) + a.tokens, dtype=ne.NE_BF16 if a.bf16 else ne.NE_FP16)
    try:
        m.load(a.checkpoint)
        print(f"Prompt ({len(prompt)} tokens): {prompt_text}")
        print(f"Generating {a.tokens} tokens (temp={a.temp}, top_p={a.top_p})...")
        print("---")
        u = sampling_uniforms(a.tokens, a.seed) if a.temp >= 1e-6 else None
        out = m.decode(np.array([prompt], np.int32), a.tokens, a.temp, a.top_p, u)[0].tolist()
    finally:
        m.close()
    generated = []
    for t in out:
        generated.append(t)
        print(tok.decode([t]) if tok is not None else f"{t} ", end="", flush=True)
        if eos is not None and t == eos:
            break
    print()
    print("---")
    print(f"Generated {len(generated)} tokens")
    return 0


if __name__ == "__main__":
    sys.exit(main())
