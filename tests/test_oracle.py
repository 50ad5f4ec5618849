"""Pins the numpy oracle (CPU only): closed forms, autograd, finite differences,
batched-vs-token-loop consistency and the checkpoint byte layout."""
import math
import struct

import numpy as np
import pytest

from oracle import ckpt, model as om


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


# ---------------------------------------------------------------- primitives

def test_rmsnorm_closed_form():
    D = 64
    for c in (0.5, 3.0, -2.0):
        x = np.full((3, D), c, np.float32)
        w = np.linspace(0.5, 1.5, D).astype(np.float32)
        y, r = om.rmsnorm(x, w, 1e-5)
        np.testing.assert_allclose(y, w * c / math.sqrt(c * c + 1e-5) * np.ones((3, 1)), rtol=1e-6)
        np.testing.assert_allclose(r[:, 0], 1 / math.sqrt(c * c + 1e-5), rtol=1e-6)


def test_rope_identity_at_pos0_and_norm_preserved():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, 5, 3, 16)).astype(np.float32)
    cos, sin = om.rope_tables(5, 16, 10000.0)
    y = om.rope_apply(x, cos, sin)
    np.testing.assert_array_equal(y[:, 0], x[:, 0])
    # a rotation keeps each pair's norm
    n0 = x[..., 0::2] ** 2 + x[..., 1::2] ** 2
    n1 = y[..., 0::2] ** 2 + y[..., 1::2] ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-5, atol=1e-6)
    # closed-form angle of pair i at position p: p * theta^(-2i/hd); pair (1, 0) -> (cos, sin)
    e = np.zeros((1, 5, 1, 16), np.float32)
    e[..., 6] = 1.0                                   # pair i=3, first channel
    y = om.rope_apply(e, cos, sin)
    ang = np.arange(5) * 10000.0 ** (-6.0 / 16)
    np.testing.assert_allclose(y[0, :, 0, 6], np.cos(ang), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(y[0, :, 0, 7], np.sin(ang), rtol=1e-6, atol=1e-7)
    # backward is the transpose: <rope(x), g> == <x, rope_bwd(g)>
    g = rng.standard_normal(x.shape).astype(np.float32)
    lhs = np.sum(om.rope_apply(x, cos, sin).astype(np.float64) * g)
    rhs = np.sum(x.astype(np.float64) * om.rope_bwd(g, cos, sin))
    assert abs(lhs - rhs) < 1e-4 * abs(lhs) + 1e-5


@pytest.mark.parametrize("V", [512, 32000])
def test_ce_zero_weights_is_ln_vocab(V):
    cfg = om.tiny(vocab=V, n_layers=1)
    P = om.init_params(cfg, zero=True)
    tok = om.tokens_for_step(cfg, 2, 16, seed=1)
    loss, cache = om.forward(cfg, P, tok)
    assert abs(loss - (-math.log(1.0 / V + 1e-10))) < 1e-5
    assert abs(loss - math.log(V)) < 1e-4
    # dlogits rows sum to zero (softmax minus one-hot)
    assert np.abs(cache["dlogits"].sum(axis=1)).max() < 1e-6


def test_adam_closed_form_t1():
    rng = np.random.default_rng(3)
    w0 = rng.standard_normal(1000).astype(np.float32) * 0.02
    g = rng.standard_normal(1000).astype(np.float32) * 1e-3
    w, m, v = w0.copy(), np.zeros_like(w0), np.zeros_like(w0)
    lr, wd, eps = 3e-4, 0.1, 1e-8
    om.adam_update(w, g, m, v, 1, lr, 0.9, 0.95, eps, wd)
    expect = w0 - lr * (g / (np.abs(g) + eps) + wd * w0)
    np.testing.assert_allclose(w, expect, rtol=1e-5, atol=1e-9)


@pytest.mark.parametrize("grad_scale,clip", [(1.0, 0.0), (1 / 256, 0.0), (1.0, 1e-3)])
def test_optimizer_step_constant_gradient_closed_form(grad_scale, clip):
    """AdamW of TD/cpu_ops.h:266-303 over several steps with the wd rules of
    TD/train.m:861-897.  With the same gradient g every step, the bias-corrected moments are
    exactly m^ = g and v^ = g^2 at every t (m_t = (1 - b1^t) g, v_t = (1 - b2^t) g^2), so each
    step moves w by -lr * (g/(|g| + eps) + wd * w): after n steps
    w_n = k^n w_0 - lr * s * (1 - k^n) / (1 - k), k = 1 - lr * wd, s = g/(|g| + eps), and
    wd = 0 for the norm gains (w_n = w_0 - n * lr * s).  A wrong bias-correction exponent,
    weight decay applied to a gain or left off a matrix, or the clip factor applied to only
    part of the gradients each break it.  The clip scales g by clip/||g|| (s is
    scale-invariant up to eps, which the small gradients here make matter)."""
    rng = np.random.default_rng(7)
    P0 = {"layers.0.Wq": (rng.standard_normal(300) * 0.02).astype(np.float32),
          "layers.0.rms_att": (1 + rng.standard_normal(40) * 0.1).astype(np.float32),
          "embed": (rng.standard_normal(200) * 0.02).astype(np.float32)}
    G0 = {k: (rng.standard_normal(v.shape) * 1e-6 / grad_scale).astype(np.float32) for k, v in P0.items()}
    lr, b1, b2, eps, wd, n = 3e-4, 0.9, 0.95, 1e-8, 0.1, 6
    P = {k: v.copy() for k, v in P0.items()}
    M = {k: np.zeros_like(v) for k, v in P0.items()}
    V = {k: np.zeros_like(v) for k, v in P0.items()}
    norm = math.sqrt(sum(float(np.sum((g.astype(np.float64) * grad_scale) ** 2)) for g in G0.values()))
    cs = clip / norm if (clip > 0 and norm > clip) else 1.0
    for t in range(1, n + 1):
        gn = om.optimizer_step(P, {k: v.copy() for k, v in G0.items()}, M, V, t, lr, b1, b2, eps, wd,
                               grad_scale=grad_scale, clip=clip)
        assert gn == pytest.approx(norm, rel=1e-6)
    for k in P0:
        g = G0[k].astype(np.float64) * grad_scale * cs
        s = g / (np.abs(g) + eps)
        w0 = P0[k].astype(np.float64)
        if om.is_gain(k):
            want = w0 - n * lr * s
        else:
            kk = 1 - lr * wd
            want = kk ** n * w0 - lr * s * (1 - kk ** n) / (1 - kk)
        # one fp32 rounding of w per step: n ulps of the largest element
        np.testing.assert_allclose(P[k], want, rtol=0, atol=n * 2.0 ** -23 * np.abs(w0).max(), err_msg=k)
        # the moments themselves: m_t = (1 - b1^t) g, v_t = (1 - b2^t) g^2
        np.testing.assert_allclose(M[k], (1 - b1 ** n) * g, rtol=2e-6, atol=1e-30, err_msg=k)
        np.testing.assert_allclose(V[k], (1 - b2 ** n) * g * g, rtol=2e-6, atol=1e-37, err_msg=k)


def test_optimizer_step_decay_only_on_matrices():
    """A zero gradient isolates weight decay: the matrices and the embedding shrink by
    exactly lr*wd*w (m = v = 0 gives a zero Adam direction), the gains stay put."""
    P = {"layers.0.W2": np.full(8, 0.5, np.float32), "rms_final": np.full(8, 1.5, np.float32),
         "layers.0.q_norm": np.full(8, 2.0, np.float32), "embed": np.full(8, -0.25, np.float32)}
    G = {k: np.zeros_like(v) for k, v in P.items()}
    M = {k: np.zeros_like(v) for k, v in P.items()}
    V = {k: np.zeros_like(v) for k, v in P.items()}
    om.optimizer_step(P, G, M, V, 3, 1e-2, wd=0.1, clip=1.0)
    assert np.all(P["layers.0.W2"] == np.float32(0.5 - 1e-2 * 0.1 * 0.5))
    assert np.all(P["embed"] == np.float32(-0.25 + 1e-2 * 0.1 * 0.25))
    assert np.all(P["rms_final"] == 1.5) and np.all(P["layers.0.q_norm"] == 2.0)


def test_lr_schedule_and_clip_closed_form():
    assert om.lr_at(0, 3e-4, 100, 1000) == pytest.approx(3e-6, rel=1e-6)
    assert om.lr_at(99, 3e-4, 100, 1000) == pytest.approx(3e-4, rel=1e-6)
    assert om.lr_at(100, 3e-4, 100, 1000) == pytest.approx(3e-4, rel=1e-6)
    assert om.lr_at(1000, 3e-4, 100, 1000) == pytest.approx(3e-5, rel=1e-5)
    mid = om.lr_at(550, 3e-4, 100, 1000)
    assert mid == pytest.approx(3e-5 + 0.5 * 2.7e-4, rel=1e-5)
    assert om.clip_scale(2.0, 1.0) == 0.5
    assert om.clip_scale(0.5, 1.0) == 1.0
    assert om.clip_scale(5.0, 0.0) == 1.0


def test_bf16_rounding():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -9, -3.14159, 1e-30], np.float32)
    r = om.round_bf16(x)
    assert r[0] == 1.0
    assert r[1] == 1.0                       # tie -> even
    assert r[2] == 1.0 + 2 ** -7             # above half -> up
    assert abs(r[3] + 3.140625) < 1e-7


# ---------------------------------------------------------------- backward

CASES = [
    dict(qk_norm=False, res_alpha=1.0, rope_theta=1e4),
    dict(qk_norm=True, res_alpha=om.train_alpha(2), rope_theta=1e6),
]


@pytest.mark.parametrize("kw", CASES)
def test_backward_matches_float64_autograd(kw):
    torch = pytest.importorskip("torch")
    import torch_ref
    cfg = om.tiny(**kw, dim=64, hidden=128, head_dim=16, vocab=97)
    P = om.init_params(cfg, seed=5, std=0.1)
    rng = np.random.default_rng(9)
    for n in P:                                   # gains away from 1 exercise the exact bwd
        if om.is_gain(n):
            P[n] = (1 + 0.3 * rng.standard_normal(P[n].shape)).astype(np.float32)
    tok = om.tokens_for_step(cfg, 2, 12, seed=4)
    loss, cache = om.forward(cfg, P, tok, loss_scale=256.0)
    G = om.backward(cfg, P, cache)
    tl, TG = torch_ref.grads(cfg, P, tok, loss_scale=256.0)
    assert abs(loss - tl) < 1e-5 * abs(tl)
    for n in P:
        assert rel_l2(G[n], TG[n]) < 2e-4, n


def _ref_rmsnorm_bwd_loops(dy, x, w, resid=None):
    """The reference's rmsnorm_bwd / rmsnorm_bwd_add as its scalar loops run them, on its
    channel-major [d, S] layout, in float64 (TD/cpu_ops.h:108-192, 198-261): ss and dot over
    channels, rrms recomputed from x with eps 1e-5, dot scaled by rrms^2/d, then per channel
    tmp = (dy - x*dot)*rrms, dx = tmp*w (+ residual), dw += sum_s dy*x*rrms."""
    d, S = x.shape
    ss = [0.0] * S
    dot = [0.0] * S
    for i in range(d):
        for s in range(S):
            ss[s] += float(x[i, s]) * float(x[i, s])
            dot[s] += float(dy[i, s]) * float(x[i, s]) * float(w[i])
    rrms = [1.0 / math.sqrt(ss[s] / d + 1e-5) for s in range(S)]
    dot = [dot[s] * rrms[s] * rrms[s] / d for s in range(S)]
    dx = np.zeros((d, S))
    dw = np.zeros(d)
    for i in range(d):
        for s in range(S):
            tmp = (float(dy[i, s]) - float(x[i, s]) * dot[s]) * rrms[s]
            dx[i, s] = tmp * float(w[i]) + (float(resid[i, s]) if resid is not None else 0.0)
            dw[i] += float(dy[i, s]) * float(x[i, s]) * rrms[s]
    return dx, dw


def test_rmsnorm_bwd_reference_formula_matches_reference_loops():
    """backward's norm_bwd_ref option (the reference's formula) against the reference's loops
    on the transposed layout, with and without the fused residual; and at unit gains both
    formulas agree (the exact one is pinned by autograd above)."""
    rng = np.random.default_rng(21)
    S, d = 5, 12
    x = rng.standard_normal((S, d)).astype(np.float32)
    dy = rng.standard_normal((S, d)).astype(np.float32)
    res = rng.standard_normal((S, d)).astype(np.float32)
    w = (1 + 0.4 * rng.standard_normal(d)).astype(np.float32)
    _, r = om.rmsnorm(x, w, 1e-5)
    dx, dw = om.rmsnorm_bwd(dy, x, w, r, ref=True)
    for resid in (None, res):
        want, want_dw = _ref_rmsnorm_bwd_loops(dy.T, x.T, w, None if resid is None else resid.T)
        got = dx + (0 if resid is None else resid)
        np.testing.assert_allclose(got, want.T, rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(dw, want_dw, rtol=1e-5, atol=1e-6)
    # the gain placement matters: with non-unit gains the exact gradient differs
    dx_exact, dw_exact = om.rmsnorm_bwd(dy, x, w, r)
    assert rel_l2(dx_exact, dx) > 1e-2
    np.testing.assert_array_equal(dw_exact, dw)
    one = np.ones(d, np.float32)
    _, r1 = om.rmsnorm(x, one, 1e-5)
    np.testing.assert_allclose(om.rmsnorm_bwd(dy, x, one, r1, ref=True)[0], om.rmsnorm_bwd(dy, x, one, r1)[0],
                               rtol=1e-5, atol=1e-6)


def test_backward_reference_norm_formula_threads_through_the_model():
    """norm_bwd_ref reaches the final, FFN and attention norms: equal to the exact backward at
    unit gains; with trained gains the final gain's gradient (above every norm) is unchanged
    and the gradients below it move."""
    cfg = om.tiny(qk_norm=True, dim=64, hidden=128, head_dim=16, vocab=97)
    P = om.init_params(cfg, seed=5, std=0.1)
    tok = om.tokens_for_step(cfg, 2, 12, seed=4)
    _, cache = om.forward(cfg, P, tok, loss_scale=256.0)
    G0, G1 = om.backward(cfg, P, cache), om.backward(cfg, P, cache, norm_bwd_ref=True)
    for n in P:
        assert rel_l2(G1[n], G0[n]) < 1e-5, n
    rng = np.random.default_rng(9)
    for n in P:
        if om.is_gain(n):
            P[n] = (1 + 0.3 * rng.standard_normal(P[n].shape)).astype(np.float32)
    _, cache = om.forward(cfg, P, tok, loss_scale=256.0)
    G0, G1 = om.backward(cfg, P, cache), om.backward(cfg, P, cache, norm_bwd_ref=True)
    np.testing.assert_array_equal(G1["rms_final"], G0["rms_final"])
    for n in ("layers.1.W1", "layers.1.rms_ffn", "layers.1.Wq", "layers.0.rms_att", "embed"):
        assert rel_l2(G1[n], G0[n]) > 1e-3, n


def test_compact_vocab_backward_matches_float64_autograd():
    """Vocab compaction (TD/cpu_ops.h:384-431): classifier over the ids present in the data,
    gradient scattered back to those embedding rows; pinned by autograd of the sub-matrix."""
    pytest.importorskip("torch")
    import torch_ref
    cfg = om.tiny(qk_norm=True, res_alpha=om.train_alpha(2), rope_theta=1e6, dim=64, hidden=128,
                  head_dim=16, vocab=97)
    P = om.init_params(cfg, seed=5, std=0.1)
    rng = np.random.default_rng(3)
    tok = rng.choice(np.arange(10, 60, 3), size=(2, 13)).astype(np.int32)   # 17 distinct ids
    ids = om.vocab_map_build(tok, cfg.vocab)
    assert list(ids) == sorted(set(tok.reshape(-1).tolist()))
    loss, cache = om.forward(cfg, P, tok, loss_scale=256.0, vocab_ids=ids)
    G = om.backward(cfg, P, cache)
    tl, TG = torch_ref.grads(cfg, P, tok, loss_scale=256.0, vocab_ids=ids)
    assert abs(loss - tl) < 1e-5 * abs(tl)
    for n in P:
        assert rel_l2(G[n], TG[n]) < 2e-4, n
    # rows outside the compact vocabulary and never used as inputs get no gradient
    unused = np.setdiff1d(np.arange(cfg.vocab), ids)
    assert np.abs(G["embed"][unused]).max() == 0


def test_compact_vocab_known_answers():
    cfg = om.tiny(vocab=300)
    tok = om.tokens_for_step(cfg, 2, 16, seed=7) % 50 + 100
    ids = om.vocab_map_build(tok, cfg.vocab)
    # zero weights: every logit is 0, so the loss is ln(CV)
    P0 = om.init_params(cfg, seed=0, zero=True)
    l0, _ = om.forward(cfg, P0, tok, vocab_ids=ids)
    assert abs(l0 - np.log(len(ids))) < 1e-5
    # the identity map is the full-vocabulary path
    P = om.init_params(cfg, seed=1, std=0.05)
    lf, cf = om.forward(cfg, P, tok, loss_scale=4.0)
    li, ci = om.forward(cfg, P, tok, loss_scale=4.0, vocab_ids=np.arange(cfg.vocab, dtype=np.int32))
    assert abs(lf - li) <= 1e-6 * abs(lf)
    Gf, Gi = om.backward(cfg, P, cf), om.backward(cfg, P, ci)
    for n in P:
        np.testing.assert_allclose(Gi[n], Gf[n], rtol=1e-5, atol=1e-7)
    # a target outside the map is an error
    with pytest.raises(ValueError):
        om.forward(cfg, P, tok, vocab_ids=ids[1:])


def test_torch_ref_matches_finite_differences():
    torch = pytest.importorskip("torch")
    import torch_ref
    cfg = om.tiny(dim=32, hidden=64, head_dim=8, vocab=31, n_layers=1, qk_norm=True,
                  res_alpha=0.5, rope_theta=1e6)
    P = om.init_params(cfg, seed=2, std=0.2)
    tok = om.tokens_for_step(cfg, 1, 6, seed=8)
    _, TG = torch_ref.grads(cfg, P, tok)
    params = {k: torch.tensor(v, dtype=torch.float64) for k, v in P.items()}
    rng = np.random.default_rng(1)
    for n in ("layers.0.Wq", "layers.0.Wk", "layers.0.W2", "layers.0.q_norm", "layers.0.rms_att",
              "rms_final", "embed"):
        flat = params[n].view(-1)
        for idx in rng.choice(flat.numel(), 3, replace=False):
            h = 1e-6
            old = float(flat[idx])
            flat[idx] = old + h
            lp = float(torch_ref.loss_fn(cfg, params, tok))
            flat[idx] = old - h
            lm = float(torch_ref.loss_fn(cfg, params, tok))
            flat[idx] = old
            fd = (lp - lm) / (2 * h)
            an = TG[n].reshape(-1)[idx]
            assert abs(fd - an) < 1e-6 + 1e-4 * abs(an), (n, idx, fd, an)


# ---------------------------------------------------------------- forward consistency

@pytest.mark.parametrize("kw", CASES)
def test_batched_forward_equals_token_loop(kw):
    cfg = om.tiny(**kw, vocab=300)
    P = om.init_params(cfg, seed=0, std=0.05)
    tok = om.tokens_for_step(cfg, 2, 10, seed=3)
    _, cache = om.forward(cfg, P, tok)
    xf = cache["xf"]
    logits = xf @ P["embed"].T
    for k in (1, 4, 10):
        _, _, rows = om.decode(cfg, P, tok[:, :k], 1, return_logits=True)
        np.testing.assert_allclose(rows[0], logits[:, k - 1], rtol=2e-4, atol=2e-5)


def test_decode_sampling_matches_numpy_choice():
    """Inverse-CDF sampling with a supplied uniform equals RandomState.choice's draw."""
    cfg = om.tiny(vocab=200, n_layers=1)
    P = om.init_params(cfg, seed=1, std=0.3)
    prompt = np.array([[3, 7, 11]], np.int32)
    u = np.random.RandomState(5).random_sample((1, 6))
    toks, _, rows = om.decode(cfg, P, prompt, 6, temperature=0.6, uniforms=u, return_logits=True)
    rs = np.random.RandomState(5)
    for j in range(6):
        pr = om.softmax_rows((rows[j, 0] / np.float32(0.6))[None])[0]
        assert toks[0, j] == rs.choice(200, p=pr)


# ---------------------------------------------------------------- checkpoint

def test_ckpt_header_offsets_and_roundtrip(tmp_path):
    cfg = om.tiny(n_layers=1, qk_norm=True)
    P = om.init_params(cfg, seed=1)
    M = {k: v * 0.5 for k, v in P.items()}
    V = {k: v * 0.25 for k, v in P.items()}
    path = tmp_path / "c.bin"
    ckpt.write(path, cfg, P, M, V, step=7, total_steps=100, lr=1e-3, loss=2.5, adam_t=3,
               cum_train=1.5)
    raw = path.read_bytes()
    assert len(raw) == ckpt.expected_size(cfg)
    # hand-decoded offsets of the 96-byte header (TD/config.h:82-91)
    assert struct.unpack_from("<i", raw, 0)[0] == 0x424C5A54
    assert struct.unpack_from("<i", raw, 4)[0] == 4
    assert struct.unpack_from("<i", raw, 8)[0] == 7
    assert struct.unpack_from("<i", raw, 16)[0] == 1          # n_layers
    assert struct.unpack_from("<i", raw, 20)[0] == cfg.vocab
    assert struct.unpack_from("<f", raw, 44)[0] == 2.5        # loss
    assert struct.unpack_from("<d", raw, 56)[0] == 1.5        # cum_train
    assert struct.unpack_from("<i", raw, 80)[0] == 3          # adam_t
    assert struct.unpack_from("<iii", raw, 84) == (cfg.kv_heads, cfg.head_dim, cfg.q_dim)
    # first tensor (Wq) starts right after the header
    np.testing.assert_array_equal(np.frombuffer(raw, np.float32, 4, 96), P["layers.0.Wq"].reshape(-1)[:4])
    h, P2, M2, V2 = ckpt.read(path)
    assert h["step"] == 7 and h["adam_t"] == 3
    for k in P:
        np.testing.assert_array_equal(P2[k], P[k])
        np.testing.assert_array_equal(M2[k], M[k])
        np.testing.assert_array_equal(V2[k], V[k])


def test_ckpt_reference_sizes():
    """Byte counts of the reference checkpoints computed from TD/train.m:97-131."""
    assert ckpt.expected_size(om.stories110m()) == 1_314_358_368
    assert ckpt.expected_size(om.qwen3_06b(qk_norm=False)) == 7_152_513_120


def test_rounding_hooks_pass_values_through_and_reach_every_site():
    """The oracle's 16-bit rounding hooks (used only by the bf16 site study): an identity hook
    leaves the loss and every gradient bit-identical to no hook, and the forward and backward
    visit every site of ROUND_SITES; rounding one backward site (dlogits) to bf16 moves the
    gradients, rounding the final norm's output moves the loss."""
    cfg = om.tiny(qk_norm=True, n_layers=2)
    P = om.init_params(cfg, seed=0, std=0.02)
    tok = om.tokens_for_step(cfg, 2, cfg.seq, seed=1)
    seen = set()

    def ident(site, x):
        seen.add(site)
        return x

    l0, c0 = om.forward(cfg, P, tok, loss_scale=256.0)
    g0 = om.backward(cfg, P, c0)
    l1, c1 = om.forward(cfg, P, tok, loss_scale=256.0, rnd=ident)
    g1 = om.backward(cfg, P, c1, rnd=ident)
    assert l1 == l0
    for n in g0:
        np.testing.assert_array_equal(g1[n], g0[n], err_msg=n)
    assert seen == set(om.ROUND_SITES)

    def only(name):
        return lambda site, x: om.round_bf16(np.asarray(x, np.float32)) if site == name else x

    _, c2 = om.forward(cfg, P, tok, loss_scale=256.0, rnd=only("dlogits"))
    g2 = om.backward(cfg, P, c2, rnd=only("dlogits"))
    assert any(not np.array_equal(g2[n], g0[n]) for n in g0)
    l3, _ = om.forward(cfg, P, tok, loss_scale=256.0, rnd=only("xf"))
    assert l3 != l0
