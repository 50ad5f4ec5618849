#!/usr/bin/env python3
"""export_hf.py - v4 training checkpoint -> Hugging Face safetensors directory, offline.

The counterpart of the reference's TD/tools/export_hf.py: the same checkpoint reader
(export_hf.py:16-78: header, per-layer tensors, Adam state skipped), the same tensor names
(export_hf.py:90-105) in model.safetensors, config/tokenizer files copied from the original
model (a local directory here, --model) or a minimal Qwen3 config.json (export_hf.py:
140-158).  QK-norm gains found in the checkpoint's trailer are exported as
self_attn.q_norm/k_norm.  Pushing to the hub needs the network and is not offered.
"""
import argparse
import json
import os
import shutil
import struct
import sys

import numpy as np

CKPT_MAGIC = 0x424C5A54
QKN_TAG = 0x314E4B51
HDR = struct.Struct("<10i2f3d6i")
COPY_FILES = ("config.json", "tokenizer.json", "tokenizer_config.json", "special_tokens_map.json", "vocab.json",
              "merges.txt", "generation_config.json")


def read_checkpoint(path, log=print):
    """Header info, per-layer weights, rms_final, embed and (when present) the QK-norm gains."""
    with open(path, "rb") as f:
        h = HDR.unpack(f.read(HDR.size))
        magic, version, step, total_steps, L, V, D, H, heads, seq, lr, loss = h[:12]
        kv_heads, hd, q_dim = h[18:21]
        if magic != CKPT_MAGIC or version != 4:
            raise ValueError(f"{path}: not a v4 checkpoint")
        kv_dim = kv_heads * hd
        info = dict(step=step, loss=loss, lr=lr, dim=D, hidden=H, heads=heads, kv_heads=kv_heads, hd=hd,
                    q_dim=q_dim, kv_dim=kv_dim, n_layers=L, vocab=V)
        log(f"Checkpoint: step={step} loss={loss:.4f}")
        log(f"  dim={D} q_dim={q_dim} kv_dim={kv_dim} hidden={H}")
        log(f"  heads={heads} kv_heads={kv_heads} layers={L} vocab={V}")

        def read(shape):
            n = int(np.prod(shape))
            a = np.fromfile(f, np.float32, n)
            if a.size != n:
                raise ValueError(f"{path}: truncated")
            return a.reshape(shape)

        def take(shape):                       # a tensor followed by its Adam m, v
            a = read(shape)
            f.seek(2 * 4 * a.size, os.SEEK_CUR)
            return a

        shapes = (("Wq", (q_dim, D)), ("Wk", (kv_dim, D)), ("Wv", (kv_dim, D)), ("Wo", (D, q_dim)),
                  ("W1", (H, D)), ("W2", (D, H)), ("W3", (H, D)), ("rms_att", (D,)), ("rms_ffn", (D,)))
        layers = []
        for _ in range(L):                     # nine tensors, then their (m, v) pairs
            layers.append({name: read(shape) for name, shape in shapes})
            f.seek(2 * 4 * sum(int(np.prod(sh)) for _, sh in shapes), os.SEEK_CUR)
        rms_final = take((D,))
        embed = take((V, D))
        qkn = None
        tag = f.read(12)
        if len(tag) == 12:
            t, l2, hd2 = struct.unpack("<3i", tag)
            if (t, l2, hd2) != (QKN_TAG, L, hd):
                raise ValueError(f"{path}: unknown data after the v4 body")
            qkn = [(take((hd,)), take((hd,))) for _ in range(L)]
    return info, layers, rms_final, embed, qkn


def minimal_config(info, qk_norm):
    """export_hf.py:140-158."""
    return {"architectures": ["Qwen3ForCausalLM"], "model_type": "qwen3", "hidden_size": info["dim"],
            "intermediate_size": info["hidden"], "num_attention_heads": info["heads"],
            "num_key_value_heads": info["kv_heads"], "head_dim": info["hd"], "num_hidden_layers": info["n_layers"],
            "vocab_size": info["vocab"], "max_position_embeddings": 32768, "rms_norm_eps": 1e-5,
            "tie_word_embeddings": True, "torch_dtype": "float32"}


def export(out_dir, info, layers, rms_final, embed, qkn=None, model_dir=None, log=print):
    from safetensors.numpy import save_file
    os.makedirs(out_dir, exist_ok=True)
    t = {"model.embed_tokens.weight": np.ascontiguousarray(embed), "model.norm.weight": np.ascontiguousarray(rms_final)}
    names = (("Wq", "self_attn.q_proj.weight"), ("Wk", "self_attn.k_proj.weight"), ("Wv", "self_attn.v_proj.weight"),
             ("Wo", "self_attn.o_proj.weight"), ("W1", "mlp.gate_proj.weight"), ("W2", "mlp.down_proj.weight"),
             ("W3", "mlp.up_proj.weight"), ("rms_att", "input_layernorm.weight"),
             ("rms_ffn", "post_attention_layernorm.weight"))
    for l, layer in enumerate(layers):
        for ours, hf in names:
            t[f"model.layers.{l}.{hf}"] = np.ascontiguousarray(layer[ours])
        if qkn is not None:
            t[f"model.layers.{l}.self_attn.q_norm.weight"] = np.ascontiguousarray(qkn[l][0])
            t[f"model.layers.{l}.self_attn.k_norm.weight"] = np.ascontiguousarray(qkn[l][1])
    st = os.path.join(out_dir, "model.safetensors")
    save_file(t, st)
    log(f"Saved: {st} ({os.path.getsize(st) / 1e6:.1f} MB)")
    copied = []
    if model_dir:
        for name in COPY_FILES:
            src = os.path.join(model_dir, name)
            if os.path.exists(src):
                shutil.copy(src, os.path.join(out_dir, name))
                copied.append(name)
        log(f"Copied {', '.join(copied) or 'nothing'} from {model_dir}")
    if "config.json" not in copied:
        with open(os.path.join(out_dir, "config.json"), "w") as f:
            json.dump(minimal_config(info, qkn is not None), f, indent=2)
    log(f"\nModel exported to: {out_dir}/")


def main(argv=None):
    ap = argparse.ArgumentParser(description="Export a v4 training checkpoint to an HF safetensors directory")
    ap.add_argument("checkpoint")
    ap.add_argument("--model", "-m", default=None, help="local directory of the original model (config + tokenizer)")
    ap.add_argument("--output", "-o", required=True, help="output directory")
    a = ap.parse_args(argv)
    info, layers, rms_final, embed, qkn = read_checkpoint(a.checkpoint)
    export(a.output, info, layers, rms_final, embed, qkn, a.model)
    return 0


if __name__ == "__main__":
    sys.exit(main())
