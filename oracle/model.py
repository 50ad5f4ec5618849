"""fp32 numpy restatement of the training_dynamic step (oracle; test infrastructure only).

Reference files followed (paths relative to the reference repo,
TD = ane-training/training/training_dynamic):

* forward math            TD/tools/generate.py:81-110 (rmsnorm, softmax, silu, rope),
                          generate.py:133-195 (layer loop, tied LM head), batched over
                          B sequences of S tokens; residual scale alpha as in
                          TD/train.m:181 and TD/io.h:25-37 (alpha=1 reproduces
                          generate.py literally)
* GQA head mapping        kv head = q head // (heads/kv_heads)  (generate.py:168,
                          TD/io.h:423-430)
* interleaved RoPE        pairs (2i, 2i+1), freq = theta^(-2i/hd)  (generate.py:97-110,
                          TD/cpu_ops.h:456-475); theta is a parameter (reference: 1e4)
* causal softmax attention, scale 1/sqrt(hd)  (TD/mil_dynamic.h:57-234)
* SwiGLU fwd/bwd          TD/mil_dynamic.h:238-306, 320-409
* cross-entropy           TD/cpu_ops.h:348-382: loss = mean(-log(p_tgt + 1e-10)),
                          dlogits = (softmax - onehot) * loss_scale / T
* vocab compaction        TD/cpu_ops.h:384-431, TD/train.m:286-292, 401, 497-523, 802:
                          optional; the classifier and the softmax cover only the ids
                          present in the data (ascending full id = compact id), and the
                          compact embedding gradient is scattered back to its rows
* RMSNorm bwd             exact gradient of TD/cpu_ops.h:20-60 (the reference's
                          TD/cpu_ops.h:108-261 carries an extra gain factor on the
                          projection term; identical while gains are 1.0); that formula
                          as an option (backward(norm_bwd_ref=True))
* grad scale/norm/clip    TD/train.m:785-849
* LR schedule             TD/train.m:851-858
* AdamW                   TD/cpu_ops.h:266-303, wd=0 for norm gains (TD/train.m:861-897)
* token loop              generate.py:113-228 (KV cache, greedy / temperature / top-p)

Optional Qwen3 switch: per-head QK-RMSNorm (gain [head_dim], applied to q and k
before RoPE).  The reference has no QK-norm; with qk_norm=False the math is the
reference's.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, replace

import numpy as np

F32 = np.float32


@dataclass(frozen=True)
class Config:
    dim: int
    hidden: int
    n_heads: int
    kv_heads: int
    head_dim: int
    n_layers: int
    vocab: int
    seq: int
    rope_theta: float = 10000.0
    qk_norm: bool = False
    res_alpha: float = 1.0
    eps: float = 1e-5

    @property
    def q_dim(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.kv_heads * self.head_dim

    @property
    def gqa_ratio(self) -> int:
        return self.n_heads // self.kv_heads

    def with_(self, **kw) -> "Config":
        return replace(self, **kw)


def stories110m(**kw) -> Config:
    """TD/models/stories110m.h:6-19."""
    return Config(dim=768, hidden=2048, n_heads=12, kv_heads=12, head_dim=64, n_layers=12,
                  vocab=32000, seq=256).with_(**kw)


def qwen3_06b(**kw) -> Config:
    """TD/models/qwen3_06b.h:6-19, plus the Qwen3 QK-norm / theta=1e6 switches."""
    base = Config(dim=1024, hidden=3072, n_heads=16, kv_heads=8, head_dim=128, n_layers=28,
                  vocab=151936, seq=256, rope_theta=1e6, qk_norm=True)
    return base.with_(**kw)


def tiny(**kw) -> Config:
    """A small GQA model whose dims are multiples of 64 (GPU tile constraint)."""
    return Config(dim=128, hidden=256, n_heads=4, kv_heads=2, head_dim=64, n_layers=2,
                  vocab=512, seq=64).with_(**kw)


def train_alpha(n_layers: int) -> float:
    """Residual scale of TD/train.m:181."""
    return float(np.float32(1.0) / np.sqrt(np.float32(2.0 * n_layers)))


# ----------------------------------------------------------------------------------------
# parameters

LAYER_TENSORS = ("Wq", "Wk", "Wv", "Wo", "W1", "W2", "W3", "rms_att", "rms_ffn")


def layer_shapes(cfg: Config) -> dict:
    D, H, Q, KV = cfg.dim, cfg.hidden, cfg.q_dim, cfg.kv_dim
    return {"Wq": (Q, D), "Wk": (KV, D), "Wv": (KV, D), "Wo": (D, Q), "W1": (H, D),
            "W2": (D, H), "W3": (H, D), "rms_att": (D,), "rms_ffn": (D,)}


def tensor_list(cfg: Config):
    """Checkpoint tensor order (TD/train.m:111-129), then the QK-norm gains extension.

    Returns [(name, shape)] where name is "layers.{l}.{Wq..rms_ffn}", "rms_final",
    "embed", and (qk_norm only) "layers.{l}.q_norm" / "layers.{l}.k_norm".
    """
    out = []
    shapes = layer_shapes(cfg)
    for l in range(cfg.n_layers):
        for t in LAYER_TENSORS:
            out.append((f"layers.{l}.{t}", shapes[t]))
    out.append(("rms_final", (cfg.dim,)))
    out.append(("embed", (cfg.vocab, cfg.dim)))
    if cfg.qk_norm:
        for l in range(cfg.n_layers):
            out.append((f"layers.{l}.q_norm", (cfg.head_dim,)))
            out.append((f"layers.{l}.k_norm", (cfg.head_dim,)))
    return out


def is_gain(name: str) -> bool:
    return name.endswith(("rms_att", "rms_ffn", "rms_final", "q_norm", "k_norm"))


def init_params(cfg: Config, seed: int = 0, std: float = 0.02, zero: bool = False) -> dict:
    """N(0, std) weights drawn per tensor in checkpoint order from default_rng(seed); gains 1."""
    rng = np.random.default_rng(seed)
    P = {}
    for name, shape in tensor_list(cfg):
        if is_gain(name):
            P[name] = np.ones(shape, F32)
        elif zero:
            P[name] = np.zeros(shape, F32)
        else:
            n = int(np.prod(shape))
            P[name] = (rng.standard_normal(n, dtype=F32) * F32(std)).reshape(shape)
    return P


def round_bf16(a: np.ndarray) -> np.ndarray:
    """Round fp32 to the nearest bf16 (ties to even), returned as fp32."""
    u = np.ascontiguousarray(a, F32).view(np.uint32)
    r = ((u.astype(np.uint64) + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(F32).reshape(a.shape)


def tokens_for_step(cfg: Config, B: int, S: int, seed: int) -> np.ndarray:
    """Token ids uniform in [0, V) from default_rng(seed), shape [B, S+1] int32."""
    return np.random.default_rng(seed).integers(0, cfg.vocab, size=(B, S + 1)).astype(np.int32)


# ----------------------------------------------------------------------------------------
# primitive ops


def rmsnorm(x, w, eps):
    """generate.py:81-84 vectorised over leading axes: (x / rms) * w."""
    rms = np.sqrt(np.mean(x * x, axis=-1, keepdims=True, dtype=F32) + F32(eps)).astype(F32)
    return ((x / rms) * w).astype(F32), (F32(1.0) / rms).astype(F32)


def rmsnorm_bwd(dy, x, w, r, ref: bool = False):
    """Exact gradient of y = x*r*w, r = (mean(x^2)+eps)^-1/2.  Returns (dx, dw).

    ref=True gives the reference's formula instead (TD/cpu_ops.h:146-153, 188-189 rmsnorm_bwd;
    255-256 rmsnorm_bwd_add, whose residual the caller adds here): dot = sum(dy*x*w)*r^2/D,
    dx = (dy - x*dot)*r*w.  Its projection term carries one more factor w than the exact
    gradient; the two agree at w = 1.  dw (TD/cpu_ops.h:153, 192) is the same under both."""
    D = x.shape[-1]
    dot = np.sum(dy * x * w, axis=-1, keepdims=True, dtype=F32)
    if ref:
        dx = (dy - x * (dot * (r * r) / F32(D))) * r * w
    else:
        dx = r * (w * dy) - x * (r * r * r) * dot / F32(D)
    dw = np.sum((dy * x * r).reshape(-1, D), axis=0, dtype=F32)
    return dx.astype(F32), dw.astype(F32)


def silu(x):
    return (x * (F32(1.0) / (F32(1.0) + np.exp(-x)))).astype(F32)


def rope_tables(S: int, hd: int, theta: float, pos0: int = 0):
    """cos/sin [S, hd/2] in float64: angle = pos / theta^(2i/hd) (generate.py:101-105)."""
    i = np.arange(hd // 2, dtype=np.float64)
    freq = 1.0 / (float(theta) ** (2.0 * i / hd))
    pos = np.arange(pos0, pos0 + S, dtype=np.float64)[:, None]
    ang = pos * freq[None, :]
    return np.cos(ang), np.sin(ang)


def rope_apply(x, cos, sin):
    """Interleaved-pair rotation of x [..., S, nh, hd] with float64 tables [S, hd/2]."""
    x0 = x[..., 0::2].astype(np.float64)
    x1 = x[..., 1::2].astype(np.float64)
    c = cos[:, None, :]
    s = sin[:, None, :]
    out = np.empty_like(x)
    out[..., 0::2] = (x0 * c - x1 * s).astype(F32)
    out[..., 1::2] = (x0 * s + x1 * c).astype(F32)
    return out


def rope_bwd(dy, cos, sin):
    """Transpose of rope_apply: (v0*c + v1*s, v1*c - v0*s)  (TD/cpu_ops.h:510-537)."""
    d0 = dy[..., 0::2].astype(np.float64)
    d1 = dy[..., 1::2].astype(np.float64)
    c = cos[:, None, :]
    s = sin[:, None, :]
    out = np.empty_like(dy)
    out[..., 0::2] = (d0 * c + d1 * s).astype(F32)
    out[..., 1::2] = (d1 * c - d0 * s).astype(F32)
    return out


def softmax_rows(x):
    m = np.max(x, axis=-1, keepdims=True)
    e = np.exp(x - m)
    return (e / np.sum(e, axis=-1, keepdims=True, dtype=F32)).astype(F32)


# ----------------------------------------------------------------------------------------
# training step


def vocab_map_build(data: np.ndarray, vocab: int) -> np.ndarray:
    """Compact vocabulary of a token stream (TD/cpu_ops.h:391-414): the distinct ids in
    ascending order; compact id c stands for full id ids[c]."""
    used = np.zeros(vocab, bool)
    used[np.asarray(data, np.int64).reshape(-1)] = True
    return np.flatnonzero(used).astype(np.int32)


# Sites of the device's 16-bit roundings (the operands its GEMMs and attention read in 16 bits),
# for forward(rnd=...) / backward(rnd=...): rnd(site, array) returns the array as the device
# holds it there (default: unchanged, the fp32 oracle).  Forward: xn, x2n, xf (RMSNorm outputs),
# qkv (the QKV GEMM's output), qkr (q, k after QK-norm and RoPE), p_fwd (attention
# probabilities in P.V), att (attention output), h13, gate, dlogits.  Backward: dbf (alpha * dx
# into the FFN and attention blocks), dh13, datt (dO), p_bwd (P in dV), ds (dS), dv, dqk (dq,
# dk after the RoPE / QK-norm backward).
ROUND_SITES = ("xn", "qkv", "qkr", "p_fwd", "att", "x2n", "h13", "gate", "xf", "dlogits",
               "dbf", "dh13", "datt", "p_bwd", "ds", "dv", "dqk")


def _keep(site, t):
    return t


def forward(cfg: Config, P: dict, tokens: np.ndarray, loss_scale: float = 1.0, want_grad_cache=True,
            vocab_ids: np.ndarray | None = None, rnd=None):
    """Batched forward + CE.  tokens [B, S+1] int: inputs [:, :S], targets [:, 1:].

    vocab_ids (optional, from vocab_map_build): the classifier and the softmax run over
    those embedding rows only and the targets are mapped to their compact ids
    (TD/train.m:401, 497-503).  rnd (optional): see ROUND_SITES.  Returns (loss, cache).
    cache carries everything the backward needs.
    """
    R = rnd or _keep
    B, S1 = tokens.shape
    S = S1 - 1
    inp, tgt = tokens[:, :S], tokens[:, 1:]
    D, NH, NKV, HD = cfg.dim, cfg.n_heads, cfg.kv_heads, cfg.head_dim
    r_gqa = cfg.gqa_ratio
    a = F32(cfg.res_alpha)
    scale = F32(1.0 / math.sqrt(HD))
    cos, sin = rope_tables(S, HD, cfg.rope_theta)
    mask = np.triu(np.full((S, S), -np.inf, F32), 1)

    x = P["embed"][inp].astype(F32)                       # [B,S,D]
    layers = []
    for l in range(cfg.n_layers):
        p = lambda t: P[f"layers.{l}.{t}"]
        c = {"x_in": x}
        xn, r1 = rmsnorm(x, p("rms_att"), cfg.eps)
        xn = R("xn", xn)
        q = R("qkv", (xn @ p("Wq").T).reshape(B, S, NH, HD))
        k = R("qkv", (xn @ p("Wk").T).reshape(B, S, NKV, HD))
        v = R("qkv", (xn @ p("Wv").T).reshape(B, S, NKV, HD))
        c.update(xn=xn, r1=r1, q_raw=q, k_raw=k, v=v)
        if cfg.qk_norm:
            qn, rq = rmsnorm(q, p("q_norm"), cfg.eps)
            kn, rk = rmsnorm(k, p("k_norm"), cfg.eps)
            c.update(rq=rq, rk=rk, qn=qn, kn=kn)
        else:
            qn, kn = q, k
        qr = R("qkr", rope_apply(qn, cos, sin))
        kr = R("qkr", rope_apply(kn, cos, sin))
        att = np.empty((B, S, NH, HD), F32)
        probs = np.empty((B, NH, S, S), F32)
        for b in range(B):
            for h in range(NH):
                kh = h // r_gqa
                s = (qr[b, :, h, :] @ kr[b, :, kh, :].T) * scale + mask
                pr = softmax_rows(s)
                probs[b, h] = pr
                att[b, :, h, :] = R("p_fwd", pr) @ v[b, :, kh, :]
        attf = R("att", att.reshape(B, S, NH * HD))
        o = attf @ p("Wo").T
        x2 = (x + a * o).astype(F32)
        x2n, r2 = rmsnorm(x2, p("rms_ffn"), cfg.eps)
        x2n = R("x2n", x2n)
        h1 = R("h13", x2n @ p("W1").T)
        h3 = R("h13", x2n @ p("W3").T)
        gate = R("gate", (silu(h1) * h3).astype(F32))
        f = gate @ p("W2").T
        x = (x2 + a * f).astype(F32)
        c.update(qr=qr, kr=kr, probs=probs, att=attf, x2=x2, x2n=x2n, r2=r2, h1=h1, h3=h3,
                 gate=gate)
        layers.append(c)
    xL = x
    xf, rf = rmsnorm(xL, P["rms_final"], cfg.eps)
    xf = R("xf", xf)
    E_cls = P["embed"] if vocab_ids is None else P["embed"][vocab_ids]
    logits = xf @ E_cls.T                                 # [B,S,V] (or [B,S,CV])
    T = B * S
    lg = logits.reshape(T, -1)
    m = np.max(lg, axis=1, keepdims=True)
    e = np.exp(lg - m)
    ssum = np.sum(e, axis=1, keepdims=True, dtype=F32)
    probs_v = (e / ssum).astype(F32)
    t_flat = tgt.reshape(T)
    if vocab_ids is not None:
        pos = np.searchsorted(vocab_ids, t_flat)
        if np.any(pos >= len(vocab_ids)) or np.any(vocab_ids[np.minimum(pos, len(vocab_ids) - 1)] != t_flat):
            raise ValueError("target id outside the compact vocabulary")
        t_flat = pos
    p_tgt = probs_v[np.arange(T), t_flat]
    losses = -np.log(p_tgt + F32(1e-10))
    loss = float(np.sum(losses, dtype=F32) / F32(T))
    cache = None
    if want_grad_cache:
        dlog = probs_v * F32(loss_scale / T)
        dlog[np.arange(T), t_flat] -= F32(loss_scale / T)
        cache = dict(inp=inp, tgt=tgt, layers=layers, xL=xL, xf=xf, rf=rf, dlogits=R("dlogits", dlog.astype(F32)),
                     cos=cos, sin=sin, B=B, S=S, vocab_ids=vocab_ids)
    return loss, cache


def backward(cfg: Config, P: dict, cache: dict, norm_bwd_ref: bool = False, rnd=None) -> dict:
    """Analytic fp32 backward of forward(); returns grads keyed like P (loss_scale included).

    norm_bwd_ref: the attention, FFN and final RMSNorms use the reference's backward formula
    (rmsnorm_bwd(ref=True); TD/train.m:527, 603, 751); the QK-norms stay exact.  rnd: see
    ROUND_SITES."""
    R = rnd or _keep
    B, S = cache["B"], cache["S"]
    D, NH, NKV, HD = cfg.dim, cfg.n_heads, cfg.kv_heads, cfg.head_dim
    r_gqa = cfg.gqa_ratio
    a = F32(cfg.res_alpha)
    scale = F32(1.0 / math.sqrt(HD))
    cos, sin = cache["cos"], cache["sin"]
    G = {k: np.zeros_like(v) for k, v in P.items()}

    dlog = cache["dlogits"].reshape(B, S, -1)
    xf = cache["xf"]
    ids = cache.get("vocab_ids")
    dE_cls = (dlog.reshape(B * S, -1).T @ xf.reshape(B * S, D)).astype(F32)
    if ids is None:
        G["embed"] += dE_cls
        dxf = dlog @ P["embed"]
    else:                                                 # vocab_scatter_grads, TD/cpu_ops.h:425-431
        G["embed"][ids] += dE_cls
        dxf = dlog @ P["embed"][ids]
    dx, dg = rmsnorm_bwd(dxf, cache["xL"], P["rms_final"], cache["rf"], norm_bwd_ref)
    G["rms_final"] += dg

    for l in reversed(range(cfg.n_layers)):
        c = cache["layers"][l]
        p = lambda t: P[f"layers.{l}.{t}"]
        g = lambda t: f"layers.{l}.{t}"
        # FFN
        dffn = R("dbf", a * dx)                            # grad of f
        G[g("W2")] += (dffn.reshape(-1, D).T @ c["gate"].reshape(B * S, -1)).astype(F32)
        dgate = dffn @ p("W2")
        h1, h3 = c["h1"], c["h3"]
        sig = (F32(1.0) / (F32(1.0) + np.exp(-h1))).astype(F32)
        dh3 = R("dh13", dgate * (h1 * sig))
        dh1 = R("dh13", dgate * h3 * sig * (F32(1.0) + h1 * (F32(1.0) - sig)))
        x2n = c["x2n"].reshape(B * S, D)
        G[g("W1")] += (dh1.reshape(B * S, -1).T @ x2n).astype(F32)
        G[g("W3")] += (dh3.reshape(B * S, -1).T @ x2n).astype(F32)
        dx2n = dh1 @ p("W1") + dh3 @ p("W3")
        dxr, dg = rmsnorm_bwd(dx2n, c["x2"], p("rms_ffn"), c["r2"], norm_bwd_ref)
        G[g("rms_ffn")] += dg
        dx2 = (dx + dxr).astype(F32)
        # attention
        do = R("dbf", a * dx2)
        G[g("Wo")] += (do.reshape(-1, D).T @ c["att"].reshape(B * S, -1)).astype(F32)
        datt = R("datt", (do @ p("Wo")).reshape(B, S, NH, HD))
        qr, kr, v, probs = c["qr"], c["kr"], c["v"], c["probs"]
        dqr = np.zeros_like(qr)
        dkr = np.zeros_like(kr)
        dv = np.zeros_like(v)
        for b in range(B):
            for h in range(NH):
                kh = h // r_gqa
                pr = probs[b, h]
                do_h = datt[b, :, h, :]
                dv[b, :, kh, :] += R("p_bwd", pr).T @ do_h
                dp = do_h @ v[b, :, kh, :].T
                ds = R("ds", pr * (dp - np.sum(dp * pr, axis=1, keepdims=True, dtype=F32)))
                dqr[b, :, h, :] = (ds @ kr[b, :, kh, :]) * scale
                dkr[b, :, kh, :] += (ds.T @ qr[b, :, h, :]) * scale
        dv = R("dv", dv)
        dqn = rope_bwd(dqr, cos, sin)
        dkn = rope_bwd(dkr, cos, sin)
        if cfg.qk_norm:
            dq, dgq = rmsnorm_bwd(dqn, c["q_raw"], p("q_norm"), c["rq"])
            dk, dgk = rmsnorm_bwd(dkn, c["k_raw"], p("k_norm"), c["rk"])
            G[g("q_norm")] += dgq
            G[g("k_norm")] += dgk
        else:
            dq, dk = dqn, dkn
        dq, dk = R("dqk", dq), R("dqk", dk)
        dq = dq.reshape(B * S, -1)
        dk = dk.reshape(B * S, -1)
        dvf = dv.reshape(B * S, -1)
        xn = c["xn"].reshape(B * S, D)
        G[g("Wq")] += (dq.T @ xn).astype(F32)
        G[g("Wk")] += (dk.T @ xn).astype(F32)
        G[g("Wv")] += (dvf.T @ xn).astype(F32)
        dxn = (dq @ p("Wq") + dk @ p("Wk") + dvf @ p("Wv")).reshape(B, S, D)
        dxr, dg = rmsnorm_bwd(dxn, c["x_in"], p("rms_att"), c["r1"], norm_bwd_ref)
        G[g("rms_att")] += dg
        dx = (dx2 + dxr).astype(F32)

    np.add.at(G["embed"], cache["inp"].reshape(-1), dx.reshape(-1, D))
    return G


# ----------------------------------------------------------------------------------------
# optimizer


def grad_norm(G: dict) -> float:
    """Global L2 norm over every gradient (TD/train.m:786-806), fp64 accumulation."""
    return float(math.sqrt(sum(float(np.sum(g.astype(np.float64) ** 2)) for g in G.values())))


def clip_scale(gnorm: float, clip: float) -> float:
    """TD/train.m:813-815: scale = clip/norm when clip > 0 and norm > clip, else 1."""
    return clip / gnorm if (clip > 0 and gnorm > clip) else 1.0


def lr_at(step: int, max_lr: float, warmup: int, total: int, min_frac: float = 0.1) -> float:
    """Warmup + cosine schedule (TD/train.m:851-858), computed in fp32 as the reference."""
    if step < warmup:
        return float(F32(max_lr) * F32(step + 1) / F32(warmup))
    ratio = F32(step - warmup) / F32(total - warmup)
    mn = F32(max_lr) * F32(min_frac)
    return float(mn + F32(0.5) * (F32(1.0) + F32(math.cos(math.pi * float(ratio)))) * (F32(max_lr) - mn))


def adam_update(w, g, m, v, t, lr, b1, b2, eps, wd):
    """In-place AdamW of TD/cpu_ops.h:266-303 (fp32)."""
    b1, b2, eps, lr, wd = F32(b1), F32(b2), F32(eps), F32(lr), F32(wd)
    bc1 = F32(1.0) - F32(b1 ** t)
    bc2 = F32(1.0) - F32(b2 ** t)
    m *= b1
    m += (F32(1.0) - b1) * g
    v *= b2
    v += (F32(1.0) - b2) * (g * g)
    mh = m * (F32(1.0) / bc1)
    vh = v * (F32(1.0) / bc2)
    upd = mh / (np.sqrt(vh) + eps) + wd * w
    w -= lr * upd


def optimizer_step(P, G, M, V, t, lr, b1=0.9, b2=0.95, eps=1e-8, wd=0.1, grad_scale=1.0, clip=1.0):
    """Scale grads, global norm, clip, AdamW (wd=0 for gains).  Mutates P, G, M, V.

    Returns the pre-clip global gradient norm (after grad_scale).
    """
    for k in G:
        G[k] *= F32(grad_scale)
    gn = grad_norm(G)
    cs = clip_scale(gn, clip)
    if cs != 1.0:
        for k in G:
            G[k] *= F32(cs)
    for k in P:
        adam_update(P[k], G[k], M[k], V[k], t, lr, b1, b2, eps, 0.0 if is_gain(k) else wd)
    return gn


# ----------------------------------------------------------------------------------------
# KV-cached token loop (generate.py:113-228), batched over B sequences


def decode(cfg: Config, P: dict, prompt: np.ndarray, n_new: int, temperature: float = 0.0,
           top_p: float = 1.0, uniforms=None, return_logits=False, forced=None):
    """Autoregressive generation.  prompt [B, P0] int.  Returns tokens [B, n_new] int32.

    Greedy when temperature < 1e-6 (generate.py:198-199).  Otherwise logits/temp ->
    softmax -> optional top-p mask -> inverse-CDF sample in vocabulary order with
    uniforms[b, step] (np.random.choice's own method, generate.py:215).
    Residual scale cfg.res_alpha (1.0 = generate.py literal).  Per-step top-2 logit
    margins are returned when return_logits is set (for near-tie diagnostics).

    forced [B, n_new] (sampling only): the tokens fed back are forced[b, step] instead of the
    oracle's own picks, and the call returns (picks, dist) where dist[b, step] is how far the
    uniform lies from the cumulative-probability boundary between the oracle's pick o and
    forced[b, step] = f (0 when they agree): u - cdf[f] when f < o, cdf[f - 1] - u when f > o.
    """
    B, P0 = prompt.shape
    D, NH, NKV, HD, L = cfg.dim, cfg.n_heads, cfg.kv_heads, cfg.head_dim, cfg.n_layers
    r_gqa = cfg.gqa_ratio
    a = F32(cfg.res_alpha)
    max_seq = P0 + n_new
    kc = np.zeros((L, B, NKV, max_seq, HD), F32)
    vc = np.zeros((L, B, NKV, max_seq, HD), F32)
    out = np.zeros((B, n_new), np.int32)
    margins = []
    logit_rows = []
    dist = np.zeros((B, n_new)) if forced is not None else None
    cur = prompt[:, 0].copy()
    scale = 1.0 / np.sqrt(HD)
    n_out = 0
    for pos in range(P0 + n_new - 1):
        tok = prompt[:, pos] if pos < P0 else cur
        x = P["embed"][tok].astype(F32)                   # [B, D]
        cos, sin = rope_tables(1, HD, cfg.rope_theta, pos0=pos)
        for l in range(L):
            p = lambda t: P[f"layers.{l}.{t}"]
            xn, _ = rmsnorm(x, p("rms_att"), cfg.eps)
            q = (xn @ p("Wq").T).reshape(B, 1, NH, HD)
            k = (xn @ p("Wk").T).reshape(B, 1, NKV, HD)
            v = (xn @ p("Wv").T).reshape(B, NKV, HD)
            if cfg.qk_norm:
                q, _ = rmsnorm(q, p("q_norm"), cfg.eps)
                k, _ = rmsnorm(k, p("k_norm"), cfg.eps)
            q = rope_apply(q, cos, sin).reshape(B, NH, HD)
            k = rope_apply(k, cos, sin).reshape(B, NKV, HD)
            kc[l, :, :, pos] = k
            vc[l, :, :, pos] = v
            att = np.zeros((B, NH, HD), F32)
            for h in range(NH):
                kh = h // r_gqa
                s = np.einsum("bd,btd->bt", q[:, h], kc[l, :, kh, :pos + 1])
                s = (s.astype(np.float64) * scale).astype(F32)
                w = softmax_rows(s)
                att[:, h] = np.einsum("bt,btd->bd", w, vc[l, :, kh, :pos + 1])
            x = (x + a * (att.reshape(B, -1) @ p("Wo").T)).astype(F32)
            xn, _ = rmsnorm(x, p("rms_ffn"), cfg.eps)
            h1 = xn @ p("W1").T
            h3 = xn @ p("W3").T
            x = (x + a * ((silu(h1) * h3) @ p("W2").T)).astype(F32)
        xf, _ = rmsnorm(x, P["rms_final"], cfg.eps)
        logits = (xf @ P["embed"].T).astype(F32)          # [B, V]
        if pos >= P0 - 1:
            if temperature < 1e-6:
                nxt = np.argmax(logits, axis=1)
            else:
                nxt = np.empty(B, np.int64)
                for b in range(B):
                    pr = softmax_rows((logits[b] / F32(temperature))[None])[0]
                    if top_p < 1.0:
                        idx = np.argsort(-pr, kind="stable")
                        cum = np.cumsum(pr[idx])
                        cut = int(np.searchsorted(cum, top_p)) + 1
                        mk = np.zeros_like(pr)
                        mk[idx[:cut]] = pr[idx[:cut]]
                        pr = mk / mk.sum()
                    cdf = np.cumsum(pr.astype(np.float64))
                    cdf /= cdf[-1]
                    u = uniforms[b, n_out]
                    nxt[b] = int(np.searchsorted(cdf, u, side="right"))
                    if forced is not None:
                        f = int(forced[b, n_out])
                        if f < nxt[b]:
                            dist[b, n_out] = u - cdf[f]
                        elif f > nxt[b]:
                            dist[b, n_out] = cdf[f - 1] - u
            if return_logits:
                srt = np.sort(logits, axis=1)
                margins.append(srt[:, -1] - srt[:, -2])
                logit_rows.append(logits.copy())
            out[:, n_out] = nxt
            cur = (forced[:, n_out] if forced is not None else nxt).astype(np.int32)
            n_out += 1
    if forced is not None:
        return out, dist
    if return_logits:
        return out, np.array(margins).T, np.array(logit_rows)
    return out
