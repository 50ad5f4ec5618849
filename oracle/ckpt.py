"""v4 checkpoint reader/writer (oracle side; test infrastructure only).

Byte layout restated from TD/config.h:82-91 (CkptHdr), TD/train.m:97-131
(save_checkpoint) and TD/tools/generate.py:18-78 (read_checkpoint):

  96-byte header, native alignment:
    i32 magic=0x424C5A54, version=4, step, total_steps,
    i32 n_layers, vocab, dim, hidden, n_heads, seq,
    f32 lr, loss,
    f64 cum_compile, cum_train, cum_wall,
    i32 cum_steps, cum_batches, adam_t,
    i32 kv_heads, head_dim, q_dim
  per layer: Wq Wk Wv Wo W1 W2 W3 rms_att rms_ffn (fp32), then (m, v) per tensor in
  the same order;  rms_final, m, v;  embed, m, v.

Extension (this build, only when QK-norm gains exist): after embed.v a trailer
  i32 tag=0x314E4B51 ("QKN1"), n_layers, head_dim, then per layer
  q_norm, m, v, k_norm, m, v (fp32 [head_dim] each).
v4 readers stop after embed.v (generate.py:76, TD/train.m:161-163), so the trailer
is ignored by them.
"""
from __future__ import annotations

import struct

import numpy as np

from .model import Config, LAYER_TENSORS, layer_shapes

HDR_FMT = "iiii" "iiiiii" "ff" "ddd" "iii" "iii"
HDR_SIZE = struct.calcsize(HDR_FMT)
MAGIC = 0x424C5A54
QKN_TAG = 0x314E4B51
HDR_FIELDS = ("magic", "version", "step", "total_steps", "n_layers", "vocab", "dim", "hidden",
              "n_heads", "seq", "lr", "loss", "cum_compile", "cum_train", "cum_wall", "cum_steps",
              "cum_batches", "adam_t", "kv_heads", "head_dim", "q_dim")
assert HDR_SIZE == 96


def expected_size(cfg: Config) -> int:
    D, V = cfg.dim, cfg.vocab
    per_layer = sum(int(np.prod(s)) for s in layer_shapes(cfg).values())
    n = cfg.n_layers * per_layer + D + V * D
    size = HDR_SIZE + 3 * 4 * n
    if cfg.qk_norm:
        size += 12 + cfg.n_layers * 6 * cfg.head_dim * 4
    return size


def write(path, cfg: Config, P: dict, M: dict, V: dict, **hdr):
    h = dict(magic=MAGIC, version=4, step=0, total_steps=0, n_layers=cfg.n_layers,
             vocab=cfg.vocab, dim=cfg.dim, hidden=cfg.hidden, n_heads=cfg.n_heads, seq=cfg.seq,
             lr=0.0, loss=0.0, cum_compile=0.0, cum_train=0.0, cum_wall=0.0, cum_steps=0,
             cum_batches=0, adam_t=0, kv_heads=cfg.kv_heads, head_dim=cfg.head_dim,
             q_dim=cfg.q_dim)
    h.update(hdr)
    with open(path, "wb") as f:
        f.write(struct.pack(HDR_FMT, *[h[k] for k in HDR_FIELDS]))
        for l in range(cfg.n_layers):
            names = [f"layers.{l}.{t}" for t in LAYER_TENSORS]
            for n in names:
                f.write(np.ascontiguousarray(P[n], np.float32).tobytes())
            for n in names:
                f.write(np.ascontiguousarray(M[n], np.float32).tobytes())
                f.write(np.ascontiguousarray(V[n], np.float32).tobytes())
        for n in ("rms_final", "embed"):
            for src in (P, M, V):
                f.write(np.ascontiguousarray(src[n], np.float32).tobytes())
        if cfg.qk_norm:
            f.write(struct.pack("iii", QKN_TAG, cfg.n_layers, cfg.head_dim))
            for l in range(cfg.n_layers):
                for t in ("q_norm", "k_norm"):
                    n = f"layers.{l}.{t}"
                    for src in (P, M, V):
                        f.write(np.ascontiguousarray(src[n], np.float32).tobytes())


def read(path):
    """Returns (hdr dict, P, M, V) with tensors keyed as oracle.model.tensor_list."""
    with open(path, "rb") as f:
        buf = f.read()
    vals = struct.unpack(HDR_FMT, buf[:HDR_SIZE])
    h = dict(zip(HDR_FIELDS, vals))
    if h["magic"] != MAGIC or h["version"] != 4:
        raise ValueError("not a v4 checkpoint")
    cfg = Config(dim=h["dim"], hidden=h["hidden"], n_heads=h["n_heads"], kv_heads=h["kv_heads"],
                 head_dim=h["head_dim"], n_layers=h["n_layers"], vocab=h["vocab"], seq=h["seq"])
    off = HDR_SIZE
    P, M, V = {}, {}, {}

    def take(shape):
        nonlocal off
        n = int(np.prod(shape))
        if off + 4 * n > len(buf):
            raise ValueError("truncated checkpoint")
        a = np.frombuffer(buf, np.float32, n, off).reshape(shape).copy()
        off += 4 * n
        return a

    shapes = layer_shapes(cfg)
    for l in range(cfg.n_layers):
        for t in LAYER_TENSORS:
            P[f"layers.{l}.{t}"] = take(shapes[t])
        for t in LAYER_TENSORS:
            M[f"layers.{l}.{t}"] = take(shapes[t])
            V[f"layers.{l}.{t}"] = take(shapes[t])
    for n, shp in (("rms_final", (cfg.dim,)), ("embed", (cfg.vocab, cfg.dim))):
        P[n], M[n], V[n] = take(shp), take(shp), take(shp)
    if off + 12 <= len(buf):
        tag, nl, hd = struct.unpack_from("iii", buf, off)
        if tag == QKN_TAG and nl == cfg.n_layers and hd == cfg.head_dim:
            off += 12
            for l in range(cfg.n_layers):
                for t in ("q_norm", "k_norm"):
                    n = f"layers.{l}.{t}"
                    P[n], M[n], V[n] = take((hd,)), take((hd,)), take((hd,))
    return h, P, M, V
