#!/usr/bin/env python3
"""convert_hf.py - Hugging Face (safetensors) weights -> v4 training checkpoint, offline.

The counterpart of the reference's TD/tools/convert_hf.py (TD = ane-training/training/
training_dynamic): the same HF -> checkpoint tensor mapping (convert_hf.py:78-99, 127-136:
q/k/v/o_proj -> Wq/Wk/Wv/Wo, gate/down/up_proj -> W1/W2/W3, input/post_attention_layernorm
-> rms_att/rms_ffn, model.norm -> rms_final, lm_head (else embed_tokens) -> embed), the same
header (seq 256, lr 3e-4, --steps as total_steps) and zeroed Adam state, and the same
default output name ane_<model_type>_dyn_ckpt.bin.  The model is a local directory
(config.json + *.safetensors) instead of a hub id, since there is no network.  Unlike the
reference, which drops Qwen3's q_norm/k_norm gains, they are kept in the checkpoint's
QK-norm trailer (read by `train --qk-norm` and generate.py here; v4 readers stop before
it); --no-qk-norm leaves them out as the reference does.
"""
import argparse
import json
import os
import struct
import sys

import numpy as np

CKPT_MAGIC = 0x424C5A54
QKN_TAG = 0x314E4B51            # trailer tag of the QK-norm gains after the v4 body
HDR = struct.Struct("<10i2f3d6i")  # TD/config.h:82-91
CHUNK = 1 << 24                 # floats per write of the zeroed Adam state


def load_local_model(path):
    """config.json and every tensor of the *.safetensors files of a local model directory."""
    from safetensors import safe_open
    with open(os.path.join(path, "config.json")) as f:
        config = json.load(f)
    files = sorted(x for x in os.listdir(path) if x.endswith(".safetensors"))
    if not files:
        raise FileNotFoundError(f"no .safetensors files in {path}")
    state = {}
    for name in files:
        with safe_open(os.path.join(path, name), framework="numpy") as f:
            for key in f.keys():
                state[key] = f.get_tensor(key)
    return state, config


def model_dims(config):
    """convert_hf.py:45-56."""
    dim = config["hidden_size"]
    heads = config["num_attention_heads"]
    kv_heads = config.get("num_key_value_heads", heads)
    hd = config.get("head_dim", dim // heads)
    return dict(dim=dim, hidden=config["intermediate_size"], heads=heads, kv_heads=kv_heads, hd=hd,
                n_layers=config["num_hidden_layers"], vocab=config["vocab_size"], q_dim=heads * hd,
                kv_dim=kv_heads * hd)


LAYER_MAP = (("Wq", "self_attn.q_proj.weight"), ("Wk", "self_attn.k_proj.weight"),
             ("Wv", "self_attn.v_proj.weight"), ("Wo", "self_attn.o_proj.weight"),
             ("W1", "mlp.gate_proj.weight"), ("W2", "mlp.down_proj.weight"), ("W3", "mlp.up_proj.weight"),
             ("rms_att", "input_layernorm.weight"), ("rms_ffn", "post_attention_layernorm.weight"))


def _write_zeros(f, n):
    z = np.zeros(min(n, CHUNK), np.float32)
    while n > 0:
        k = min(n, CHUNK)
        f.write(z[:k].tobytes())
        n -= k


def _write_param(f, a):
    """A tensor followed by its zeroed Adam m and v (rms_final, embed, the QK-norm gains)."""
    a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
    f.write(a.tobytes())
    _write_zeros(f, 2 * a.size)


def write_checkpoint(out, state, config, seq=256, total_steps=10000, qk_norm=True, log=print):
    d = model_dims(config)
    D, H, L, V = d["dim"], d["hidden"], d["n_layers"], d["vocab"]
    shapes = {"Wq": (d["q_dim"], D), "Wk": (d["kv_dim"], D), "Wv": (d["kv_dim"], D), "Wo": (D, d["q_dim"]),
              "W1": (H, D), "W2": (D, H), "W3": (H, D), "rms_att": (D,), "rms_ffn": (D,)}
    has_qkn = "model.layers.0.self_attn.q_norm.weight" in state
    log(f"Model: {config.get('model_type', 'unknown')}")
    log(f"  dim={D} q_dim={d['q_dim']} kv_dim={d['kv_dim']} hd={d['hd']} hidden={H}")
    log(f"  heads={d['heads']} kv_heads={d['kv_heads']} layers={L} vocab={V}")
    if has_qkn:
        log("  QK-norm gains: " + ("kept in the checkpoint's QK-norm trailer" if qk_norm else "skipped (--no-qk-norm)"))
    if "lm_head.weight" in state:
        embed = state["lm_head.weight"]
        log("  Using lm_head.weight for embeddings")
    else:
        embed = state["model.embed_tokens.weight"]
        log("  Using tied embed_tokens.weight for embeddings")

    def get(key, shape):
        if key not in state:
            raise KeyError(f"Missing weight: {key}")
        a = state[key]
        if a.size != int(np.prod(shape)):
            raise ValueError(f"{key}: {a.shape}, expected {shape}")
        return a

    with open(out, "wb") as f:
        f.write(HDR.pack(CKPT_MAGIC, 4, 0, total_steps, L, V, D, H, d["heads"], seq, 3e-4, 0.0, 0.0, 0.0, 0.0,
                         0, 0, 0, d["kv_heads"], d["hd"], d["q_dim"]))
        for l in range(L):
            # the layer's nine tensors, then their (m, v) pairs in the same order
            ws = [np.ascontiguousarray(get(f"model.layers.{l}.{hf}", shapes[name]), dtype=np.float32)
                  for name, hf in LAYER_MAP]
            for w in ws:
                f.write(w.tobytes())
            for w in ws:
                _write_zeros(f, 2 * w.size)
        _write_param(f, get("model.norm.weight", (D,)))
        if embed.size != V * D:
            raise ValueError(f"embedding: {embed.shape}, expected {(V, D)}")
        _write_param(f, embed)
        if has_qkn and qk_norm:
            f.write(struct.pack("<3i", QKN_TAG, L, d["hd"]))
            for l in range(L):
                for hf in ("self_attn.q_norm.weight", "self_attn.k_norm.weight"):
                    _write_param(f, get(f"model.layers.{l}.{hf}", (d["hd"],)))
    log(f"\nCheckpoint saved: {out} ({os.path.getsize(out) / 1e6:.1f} MB)")
    log("Load with: ./train --resume" + (" --qk-norm" if has_qkn and qk_norm else ""))


def main(argv=None):
    ap = argparse.ArgumentParser(description="Convert a local HF model directory to a v4 training checkpoint")
    ap.add_argument("model_dir", help="local directory with config.json and *.safetensors")
    ap.add_argument("--output", "-o", default=None, help="output checkpoint (default: ane_<model_type>_dyn_ckpt.bin)")
    ap.add_argument("--steps", type=int, default=10000, help="total training steps written to the header")
    ap.add_argument("--no-qk-norm", action="store_true", help="drop q_norm/k_norm gains (the reference's behaviour)")
    a = ap.parse_args(argv)
    print(f"Loading {a.model_dir}...")
    state, config = load_local_model(a.model_dir)
    print(f"Loaded {len(state)} tensors")
    out = a.output or f"ane_{config.get('model_type', 'model')}_dyn_ckpt.bin"
    write_checkpoint(out, state, config, total_steps=a.steps, qk_norm=not a.no_qk_norm)
    return 0


if __name__ == "__main__":
    sys.exit(main())
