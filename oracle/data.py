"""Data sampling and --scratch init of the reference train CLI (oracle; test infrastructure only).

* drand48 / srand48       POSIX 48-bit linear congruential generator (a = 0x5DEECE66D,
                          c = 0xB, seed -> (seed << 16) | 0x330E), the generator the
                          reference's train.m uses; pinned against the C library's own
                          drand48 in tests/test_oracle_data.py.
* window positions        TD/train.m:389-398: srand48(42 + start_step) once, then per step
                          pos = (size_t)(drand48() * (n_tokens - SEQ - 1)); inputs are
                          data[pos : pos+SEQ], targets data[pos+1 : pos+SEQ+1].
* scratch init            TD/train.m:236-251: srand48(42), uniform +-scale per tensor in
                          the order Wq Wk Wv Wo W1 W2 W3 per layer, then the embedding
                          (scale 0.02); gains 1.
"""
from __future__ import annotations

import numpy as np

from .model import Config, LAYER_TENSORS, layer_shapes, tensor_list

F32 = np.float32


class Drand48:
    A, C, MASK = 0x5DEECE66D, 0xB, (1 << 48) - 1

    def __init__(self, seed: int):
        self.x = ((seed & 0xFFFFFFFF) << 16) | 0x330E

    def __call__(self) -> float:
        self.x = (self.A * self.x + self.C) & self.MASK
        return self.x / float(1 << 48)


def window_positions(n_tokens: int, seq: int, start_step: int, n_steps: int):
    """Start offsets of the windows train.m samples for steps start_step .. +n_steps-1."""
    r = Drand48(42 + start_step)
    max_pos = n_tokens - seq - 1
    return [int(r() * max_pos) for _ in range(n_steps)]


def scratch_init(cfg: Config) -> dict:
    """Weights of `train --scratch` (fp32, reference layout)."""
    r = Drand48(42)
    D, H, Q, L = cfg.dim, cfg.hidden, cfg.q_dim, cfg.n_layers
    # the reference computes these scales as 1.0f/sqrtf(x) in fp32
    s_d = F32(1.0) / np.sqrt(F32(D))
    s_qd = F32(1.0) / np.sqrt(F32(Q))
    s_h = F32(1.0) / np.sqrt(F32(H))
    res = F32(1.0) / np.sqrt(F32(2.0) * F32(L))
    scales = {"Wq": s_d, "Wk": s_d, "Wv": s_d, "Wo": s_qd * res, "W1": s_h, "W2": s_d * res, "W3": s_h}
    shapes = layer_shapes(cfg)

    def draw(n, sc):
        # float scale x double draw, formed in double and rounded once to float
        # (TD/train.m:246-251: `scale*(2*drand48()-1)` stored into a float array)
        u = np.fromiter((2.0 * r() - 1.0 for _ in range(n)), np.float64, n)
        return (np.float64(F32(sc)) * u).astype(F32)

    P = {}
    for l in range(L):
        for t in LAYER_TENSORS[:7]:
            shp = shapes[t]
            P[f"layers.{l}.{t}"] = draw(int(np.prod(shp)), scales[t]).reshape(shp)
    P["embed"] = draw(cfg.vocab * D, F32(0.02)).reshape(cfg.vocab, D)
    for name, shp in tensor_list(cfg):
        if name not in P:
            P[name] = np.ones(shp, F32)
    return P
