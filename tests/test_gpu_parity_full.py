"""Parity of the training step and the token loop against the fp32 numpy oracle at the
benchmarked shapes.

* Stories110M, B=1, S=256: ten consecutive steps of fwd + bwd + AdamW on fresh token batches
  (default_rng(1000 + step)).  At every step the loss and every gradient are checked against
  the oracle run from the same weights, and the update against the oracle's AdamW fed the
  same gradients and moments.
* Qwen3-0.6B (QK-norm, theta=1e6), B=1 x S=256 and S=512: loss and gradients.
* Qwen3-0.6B at B x S = 2 x 2048 (2 layers, full vocabulary) and 8 x 2048 (1 layer): loss and
  gradients; at the full B=8 x S=2048 size the loss against the oracle's forward and
  size-independent properties of the gradient.
* The Qwen3-0.6B token loop: 200 greedy tokens at batch 1 and 32 against the committed oracle
  streams, and 200 temperature-0.6 samples against the oracle run on the same prefixes.

Tolerances: loss relative error <= 1e-3, per-tensor gradient relative L2 <= 1e-2, post-AdamW
weights and moments within 1e-5 relative (an fp32-ulp floor at the tensor's scale), greedy
tokens identical.  These are the bars of the fp16 training format.  The bf16 step is compared
with the oracle run on the bf16-rounded matrices it multiplies (as the token loop is), with
the bf16 gradient bar of gpu_util.grad_tol (4e-2; fp16 is the parity-qualified format).
"""
import functools
import os
import time

import numpy as np
import pytest

from gpu_util import as_multiplied, grad_tol, need_gpu, rel_l2
import ne
from oracle import model as om

pytestmark = pytest.mark.gpu

LOSS_RTOL = 1e-3
ADAM_RTOL = 1e-5
# Roundings in one moment update: g times the clip scale, the (1 - b) g product, the square
# for v, the fused multiply-add, plus one for the oracle's own order of operations.
MOMENT_ULPS = 6


def _within(got, want, bound, what):
    """|got - want| <= bound elementwise (bound >= 0, same shape)."""
    err = np.abs(got.astype(np.float64) - want)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {err.size} outside the bound; "
                             f"worst at {i}: got {got[i]!r} want {want[i]!r} bound {bound[i]!r}")
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DTYPES = {"fp16": ne.NE_FP16, "bf16": ne.NE_BF16}


@pytest.fixture(autouse=True)
def _gpu():
    need_gpu()


@functools.lru_cache(maxsize=2)
def _qwen3_params(bf16=False):
    """N(0, 0.02) weights of the full Qwen3-0.6B from default_rng(0) (read-only: shared)."""
    P = om.init_params(om.qwen3_06b(), seed=0, std=0.02)
    return {k: om.round_bf16(v) for k, v in P.items()} if bf16 else P


def _check_grads(label, loss, lo, G, Go, dtype=ne.NE_FP16):
    errs = sorted(((rel_l2(G[n], Go[n]), n) for n in Go), reverse=True)
    print(f"[{label}] loss gpu={loss:.6f} oracle={lo:.6f} rel={abs(loss - lo) / lo:.2e}; worst grad rel-L2: "
          + ", ".join(f"{n}={e:.2e}" for e, n in errs[:4]), flush=True)
    assert abs(loss - lo) <= LOSS_RTOL * abs(lo), (loss, lo)
    for e, n in errs:
        assert e <= grad_tol(n, dtype), (n, e)


def _compare_grads(cfg, P, tok, label, vocab_ids=None, dtype=ne.NE_FP16):
    m = ne.Model.from_oracle(cfg, batch=tok.shape[0], dtype=dtype)
    m.set_params(P)
    if vocab_ids is not None:
        m.set_vocab_map(vocab_ids)
    t0 = time.time()
    loss = m.train_step(tok, 256.0)
    G = m.get_all(dict(om.tensor_list(cfg)), ne.NE_GRAD)
    t1 = time.time()
    Pm = as_multiplied(P, dtype)
    lo, cache = om.forward(cfg, Pm, tok, loss_scale=256.0, vocab_ids=vocab_ids)
    Go = om.backward(cfg, Pm, cache)
    del cache
    print(f"\n[{label}] gpu {t1 - t0:.1f}s oracle {time.time() - t1:.1f}s", flush=True)
    _check_grads(label, loss, lo, G, Go, dtype)
    return m


# ------------------------------------------------------------------- Stories110M, 10 steps

@pytest.mark.timeout(600)
@pytest.mark.parametrize("dtype", list(DTYPES))
def test_stories110m_ten_steps(dtype):
    """Ten steps of fwd + bwd + AdamW (lr 3e-4, betas 0.9/0.95, eps 1e-8, wd 0.1, clip 1.0,
    loss scale 256) on fresh batches (TD/train.m:391-918).  Each step's loss and gradients are
    checked against the oracle run from the weights that step used, and each update against
    the oracle's AdamW on the same gradients and moments.  The state is read after each
    step, whose forward ran beside the update enqueued by the optimizer step before it."""
    cfg = om.stories110m(res_alpha=om.train_alpha(12))
    sh = dict(om.tensor_list(cfg))
    P = om.init_params(cfg, seed=0, std=0.02)
    m = ne.Model.from_oracle(cfg, batch=1, dtype=DTYPES[dtype])
    m.set_params(P)
    prev = None

    def check_update(prev, step):
        Pp, Gp, Mp, Vp = prev
        M0 = {n: np.abs(x) for n, x in Mp.items()}
        V0 = {n: x.copy() for n, x in Vp.items()}
        gno = om.optimizer_step(Pp, Gp, Mp, Vp, step, 3e-4, grad_scale=1 / 256, clip=1.0)
        P2, M2, V2 = m.get_all(sh), m.get_all(sh, ne.NE_ADAM_M), m.get_all(sh, ne.NE_ADAM_V)
        for n in Pp:
            np.testing.assert_allclose(P2[n], Pp[n], rtol=ADAM_RTOL, atol=2 ** -23 * np.abs(Pp[n]).max(), err_msg=n)
            # 1e-5 relative (the two sides' clip scales differ by their gradient norms'
            # summation order) plus, where m = b1 m + (1 - b1) g nearly cancels, a few float32
            # roundings of the terms themselves rather than of the result.
            g = np.abs(Gp[n])
            _within(M2[n], Mp[n], ADAM_RTOL * np.abs(Mp[n]) + MOMENT_ULPS * 2 ** -24 * (0.9 * M0[n] + 0.1 * g),
                    n + " (m)")
            _within(V2[n], Vp[n], ADAM_RTOL * Vp[n] + MOMENT_ULPS * 2 ** -24 * (0.95 * V0[n] + 0.05 * g * g),
                    n + " (v)")
        return gno, P2, M2, V2

    for step in range(10):
        tok = om.tokens_for_step(cfg, 1, 256, seed=1000 + step)
        loss = m.train_step(tok, 256.0)
        if prev is None:
            Pg, Mg, Vg = m.get_all(sh), m.get_all(sh, ne.NE_ADAM_M), m.get_all(sh, ne.NE_ADAM_V)
        else:
            gno, Pg, Mg, Vg = check_update(prev, step)
            assert abs(gn - gno) <= 1e-5 * gno, (gn, gno)
        G = m.get_all(sh, ne.NE_GRAD)
        Pm = as_multiplied(Pg, DTYPES[dtype])
        lo, cache = om.forward(cfg, Pm, tok, loss_scale=256.0)
        Go = om.backward(cfg, Pm, cache)
        del cache, Pm
        _check_grads(f"{dtype} step {step}", loss, lo, G, Go, DTYPES[dtype])
        gn = m.optimizer_step(3e-4, 0.9, 0.95, 1e-8, 0.1, grad_scale=1 / 256, clip=1.0)
        prev = (Pg, G, Mg, Vg)
    gno, *_ = check_update(prev, 10)
    assert abs(gn - gno) <= 1e-5 * gno, (gn, gno)
    assert m.state().adam_t == 10 and m.grad_scale_info()[1] == 0
    m.close()


def test_stories110m_compact_vocab_step_parity():
    """Vocabulary compaction at the Stories110M shape: the classifier over the ~3k distinct
    ids of a data stream drawn from 3500 of the 32000 ids (TD/train.m:286-292)."""
    cfg = om.stories110m(res_alpha=om.train_alpha(12))
    P = om.init_params(cfg, seed=0, std=0.02)
    rng = np.random.default_rng(11)
    data = rng.choice(rng.choice(cfg.vocab, 3500, replace=False), 20000).astype(np.int32)
    ids = om.vocab_map_build(data, cfg.vocab)
    tok = data[1000:1000 + cfg.seq + 1][None]
    _compare_grads(cfg, P, tok, f"stories110m compact vocab {len(ids)}", vocab_ids=ids).close()


# ------------------------------------------------------------------------- Qwen3-0.6B

@pytest.mark.timeout(300)
@pytest.mark.parametrize("dtype", list(DTYPES))
def test_qwen3_step_parity(dtype):
    cfg = om.qwen3_06b(res_alpha=om.train_alpha(28))
    P = _qwen3_params()
    tok = om.tokens_for_step(cfg, 1, 256, seed=1)
    _compare_grads(cfg, P, tok, f"qwen3-0.6b B=1 S=256 {dtype}", dtype=DTYPES[dtype]).close()


@pytest.mark.timeout(300)
def test_qwen3_seq512_step_parity():
    """The SEQ=512 model (TD/models/qwen3_06b_seq512.h) at reduced depth: two layers of
    Qwen3-0.6B at S=512 with the full vocabulary."""
    cfg = om.qwen3_06b(res_alpha=om.train_alpha(28), n_layers=2, seq=512)
    P = om.init_params(cfg, seed=0, std=0.02)
    tok = om.tokens_for_step(cfg, 1, 512, seed=5)
    _compare_grads(cfg, P, tok, "qwen3-0.6b 2 layers B=1 S=512").close()


@pytest.mark.timeout(600)
@pytest.mark.parametrize("B,L,V", [(2, 2, 151936), (8, 1, 32000)])
def test_qwen3_s2048_reduced_depth(B, L, V):
    """The at-scale shape at reduced depth against the oracle: sequences of 2048 tokens through
    the flash attention forward / backward (GQA partial sums, XCD block order at B=8), the
    16k-token GEMM tiles, the split-K weight gradients over 16384 tokens and the vocabulary
    seams of 151,936 columns."""
    cfg = om.qwen3_06b(res_alpha=om.train_alpha(28), n_layers=L, seq=2048, vocab=V)
    P = om.init_params(cfg, seed=0, std=0.02)
    tok = om.tokens_for_step(cfg, B, 2048, seed=3)
    _compare_grads(cfg, P, tok, f"qwen3-0.6b {L} layers B={B} S=2048 V={V}").close()


@pytest.mark.timeout(900)
def test_qwen3_s2048_b8_full_size():
    """The full at-scale step, Qwen3-0.6B at B=8 x S=2048 (16384 tokens): the loss against the
    oracle's forward of the same 8 sequences (each sequence is independent under causal
    attention, so the oracle runs them one at a time); the update is not skipped; the norm the
    optimizer computes from the step's partials equals the float64 norm of the gradients read
    back; the two-stream schedule gives gradients bit-identical to the in-order one."""
    cfg = om.qwen3_06b(res_alpha=om.train_alpha(28), seq=2048)
    sh = dict(om.tensor_list(cfg))
    P = _qwen3_params()
    tok = om.tokens_for_step(cfg, 8, 2048, seed=1)
    m = ne.Model.from_oracle(cfg, batch=8)
    m.set_params(P)
    t0 = time.time()
    m.overlap_weight_grads(False)
    loss_inorder = m.train_step(tok, 256.0)
    G_inorder = m.get_all(sh, ne.NE_GRAD)
    m.zero_grads()
    m.overlap_weight_grads(True)
    loss = m.train_step(tok, 256.0)
    G = m.get_all(sh, ne.NE_GRAD)
    print(f"\n[qwen3 B=8 S=2048] gpu steps + read-back {time.time() - t0:.1f}s", flush=True)
    assert loss == loss_inorder
    for n in G:
        np.testing.assert_array_equal(G[n], G_inorder[n], err_msg=n)
    del G_inorder
    want = float(np.sqrt(sum(np.sum(g.astype(np.float64) ** 2) for g in G.values()))) / 256
    gn = m.optimizer_step(3e-4, 0.9, 0.95, 1e-8, 0.1, grad_scale=1 / 256, clip=1.0)
    assert np.isfinite(gn) and m.grad_scale_info()[1] == 0
    assert abs(gn - want) <= 1e-5 * want, (gn, want)
    m.close()
    del G
    t1 = time.time()
    los = [om.forward(cfg, P, tok[b:b + 1], want_grad_cache=False)[0] for b in range(8)]
    lo = float(np.mean(los))
    print(f"[qwen3 B=8 S=2048] loss gpu={loss:.6f} oracle={lo:.6f} (ln V = {np.log(cfg.vocab):.4f}); "
          f"oracle {time.time() - t1:.0f}s; grad norm {gn:.4f}", flush=True)
    assert abs(loss - lo) <= LOSS_RTOL * lo


# ------------------------------------------------------------------------ token loop

def _decode_setup(B):
    cfg = om.qwen3_06b(res_alpha=1.0)
    P = _qwen3_params(bf16=True)
    prompt = np.random.default_rng(2).integers(0, cfg.vocab, (B, 32)).astype(np.int32)
    m = ne.Model.from_oracle(cfg, batch=1, decode_batch=B, decode_ctx=232, dtype=ne.NE_BF16)
    m.set_params(P)
    return cfg, P, prompt, m


@pytest.mark.timeout(300)
@pytest.mark.parametrize("B", [1, 32])
def test_qwen3_decode_greedy_200_tokens(B):
    """The Qwen3-0.6B token loop: bf16-held N(0, 0.02) weights from seed 0, a 32-token prompt
    of uniform ids, 200 greedy tokens, token-identical to the oracle's generate path on the
    same bf16 weights (fp32 activations and KV cache on both sides).  The oracle streams are
    committed (tests/golden/make_decode_fixture.py)."""
    gold = np.load(os.path.join(GOLDEN, "decode_qwen3_greedy.npz"))
    cfg, P, prompt, m = _decode_setup(B)
    np.testing.assert_array_equal(prompt, gold[f"prompt_b{B}"])
    t0 = time.time()
    got = m.decode(prompt, 200)
    print(f"\n[decode B={B}] gpu {time.time() - t0:.2f}s; min top-2 margin of the oracle "
          f"{gold[f'margins_b{B}'].min():.3e}", flush=True)
    m.close()
    np.testing.assert_array_equal(got, gold[f"tokens_b{B}"])


@pytest.mark.timeout(600)
@pytest.mark.parametrize("B", [1, 32])
def test_qwen3_decode_sampling_200_tokens(B):
    """200 tokens sampled at temperature 0.6 with the uniforms of numpy's RandomState(3)
    (the draws generate.py's np.random.choice makes after np.random.seed(3),
    TD/tools/generate.py:198-215 and 248-249).  The oracle runs on the device's own token
    prefixes and draws with the same uniform: a token either equals the oracle's, or the
    uniform lies within TOL of the cumulative-probability boundary between the two tokens
    (the device and the oracle sum the same probabilities in different orders, and with
    151,936 tokens the boundaries are ~1e-5 apart)."""
    TOL = 1e-5
    cfg, P, prompt, m = _decode_setup(B)
    u = np.random.RandomState(3).random_sample((B, 200))
    t0 = time.time()
    got = m.decode(prompt, 200, temperature=0.6, uniforms=u)
    t1 = time.time()
    m.close()
    picks, dist = om.decode(cfg, P, prompt, 200, temperature=0.6, uniforms=u, forced=got)
    n_diff, worst = 0, 0.0
    for b in range(B):
        for j in range(200):
            if picks[b, j] != got[b, j]:
                n_diff += 1
                worst = max(worst, dist[b, j])
                assert 0 <= dist[b, j] < TOL, (b, j, picks[b, j], got[b, j], dist[b, j])
    print(f"\n[decode sampling B={B}] gpu {t1 - t0:.2f}s oracle {time.time() - t1:.0f}s; "
          f"{n_diff} of {B * 200} draws on a boundary within {worst:.1e}", flush=True)
    assert n_diff <= max(2, B * 200 // 50)
