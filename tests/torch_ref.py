"""Independent float64 torch restatement of the training step, used to pin the oracle's
backward through autograd (test helper; CPU only).

Written separately from oracle/model.py: RoPE by complex multiplication of
interleaved pairs, GQA by repeat_interleave, attention with an explicit causal
mask, CE through log_softmax.
"""
import math

import numpy as np
import torch


def loss_fn(cfg, params: dict, tokens: np.ndarray, loss_scale: float = 1.0, vocab_ids=None):
    """params: name -> float64 torch tensor (requires_grad as the caller wishes).  With
    vocab_ids the classifier is the sub-matrix of those embedding rows and each target is
    replaced by its position in vocab_ids (found with a dictionary)."""
    tok = torch.as_tensor(tokens, dtype=torch.long)
    inp, tgt = tok[:, :-1], tok[:, 1:]
    B, S = inp.shape
    HD, NH, NKV = cfg.head_dim, cfg.n_heads, cfg.kv_heads
    a = cfg.res_alpha

    def norm(x, w):
        return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + cfg.eps) * w

    i = torch.arange(HD // 2, dtype=torch.float64)
    freq = cfg.rope_theta ** (-2.0 * i / HD)
    ang = torch.arange(S, dtype=torch.float64)[:, None] * freq[None, :]
    rot = torch.polar(torch.ones_like(ang), ang)            # [S, HD/2]

    def rope(x):                                            # [B,S,h,HD]
        xc = torch.view_as_complex(x.reshape(*x.shape[:-1], HD // 2, 2).contiguous())
        return torch.view_as_real(xc * rot[None, :, None, :]).reshape(x.shape)

    causal = torch.ones(S, S, dtype=torch.bool).tril()
    x = params["embed"][inp]
    for l in range(cfg.n_layers):
        p = lambda t: params[f"layers.{l}.{t}"]
        xn = norm(x, p("rms_att"))
        q = (xn @ p("Wq").T).view(B, S, NH, HD)
        k = (xn @ p("Wk").T).view(B, S, NKV, HD)
        v = (xn @ p("Wv").T).view(B, S, NKV, HD)
        if cfg.qk_norm:
            q = norm(q, p("q_norm"))
            k = norm(k, p("k_norm"))
        q, k = rope(q), rope(k)
        rep = NH // NKV
        k = k.repeat_interleave(rep, dim=2)
        v = v.repeat_interleave(rep, dim=2)
        s = torch.einsum("bqhd,bkhd->bhqk", q, k) / math.sqrt(HD)
        s = s.masked_fill(~causal, float("-inf"))
        att = torch.einsum("bhqk,bkhd->bqhd", s.softmax(-1), v).reshape(B, S, NH * HD)
        x = x + a * (att @ p("Wo").T)
        xn = norm(x, p("rms_ffn"))
        h1 = xn @ p("W1").T
        h3 = xn @ p("W3").T
        x = x + a * ((torch.nn.functional.silu(h1) * h3) @ p("W2").T)
    xf = norm(x, params["rms_final"])
    if vocab_ids is None:
        logits = xf @ params["embed"].T
    else:
        where = {int(v): i for i, v in enumerate(vocab_ids)}
        tgt = torch.tensor([[where[int(t)] for t in row] for row in tgt.tolist()], dtype=torch.long)
        logits = xf @ params["embed"][torch.as_tensor(np.asarray(vocab_ids), dtype=torch.long)].T
    logp = logits.log_softmax(-1)
    nll = -logp.gather(-1, tgt[..., None]).squeeze(-1)
    return nll.mean() * loss_scale


def grads(cfg, P: dict, tokens, loss_scale=1.0, vocab_ids=None):
    params = {k: torch.tensor(v, dtype=torch.float64, requires_grad=True) for k, v in P.items()}
    loss = loss_fn(cfg, params, tokens, loss_scale, vocab_ids)
    loss.backward()
    return float(loss) / loss_scale, {k: t.grad.numpy() for k, t in params.items()}
