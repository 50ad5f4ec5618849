"""Model-level parity through the C-ABI (ne_train_step / ne_optimizer_step / ne_decode /
checkpoints) against the numpy oracle, at small shapes the oracle runs in seconds."""
import numpy as np
import pytest

from gpu_util import as_multiplied, grad_tol, need_gpu, rel_l2
import ne
from oracle import ckpt, model as om

pytestmark = pytest.mark.gpu

# Tolerances of the step (fp32 master weights and accumulation, 16-bit activations and GEMM
# operands: fp16 by default, bf16 compared with the oracle on the bf16-rounded matrices)
LOSS_RTOL = 1e-3
GRAD_RL2 = 1e-2
ADAM_RTOL = 1e-5

CASES = {
    "ref": dict(qk_norm=False, rope_theta=1e4, res_alpha=1.0),
    "train_alpha": dict(qk_norm=False, rope_theta=1e4, res_alpha=om.train_alpha(2)),
    "qwen3": dict(qk_norm=True, rope_theta=1e6, res_alpha=1.0),
}


@pytest.fixture(autouse=True)
def _gpu():
    need_gpu()


def shapes(cfg):
    return dict(om.tensor_list(cfg))


def run_step(cfg, P, tok, loss_scale=256.0, dtype=ne.NE_FP16):
    m = ne.Model.from_oracle(cfg, batch=tok.shape[0], dtype=dtype)
    m.set_params(P)
    loss = m.train_step(tok, loss_scale)
    G = m.get_all(shapes(cfg), ne.NE_GRAD)
    return m, loss, G


@pytest.mark.parametrize("dtype", [ne.NE_FP16, ne.NE_BF16])
@pytest.mark.parametrize("case", list(CASES))
def test_train_step_matches_oracle(case, dtype):
    cfg = om.tiny(**CASES[case])
    P = om.init_params(cfg, seed=0, std=0.02)
    tok = om.tokens_for_step(cfg, 2, cfg.seq, seed=1)
    print(f"\n[case {case} dtype {dtype}] tiny model B=2 S={cfg.seq}", flush=True)
    m, loss, G = run_step(cfg, P, tok, dtype=dtype)
    Pm = as_multiplied(P, dtype)
    lo, cache = om.forward(cfg, Pm, tok, loss_scale=256.0)
    Go = om.backward(cfg, Pm, cache)
    assert abs(loss - lo) <= LOSS_RTOL * abs(lo), (loss, lo)
    errs = sorted(((rel_l2(G[n], Go[n]), n) for n in P), reverse=True)
    print(f"  loss gpu={loss:.6f} oracle={lo:.6f}; worst grad rel-L2: "
          + ", ".join(f"{n}={e:.2e}" for e, n in errs[:6]))
    for n in P:
        assert rel_l2(G[n], Go[n]) <= grad_tol(n, dtype), (n, rel_l2(G[n], Go[n]))
    m.close()


@pytest.mark.parametrize("dtype", [ne.NE_FP16, ne.NE_BF16])
def test_gqa_step_on_long_sequences_matches_oracle(dtype):
    """GQA at 4 x 1024 tokens with 8 KV heads: the KV heads alone give the attention backward
    512 dK/dV blocks, so each block loops over the query heads of its KV head and writes dK and
    dV itself (shorter steps, as in the other cases here, take per-query-head partials that the
    QK-prep backward sums)."""
    cfg = om.tiny(**CASES["qwen3"], n_layers=1, dim=256, hidden=512, n_heads=16, kv_heads=8, head_dim=64,
                  vocab=512, seq=1024)
    P = om.init_params(cfg, seed=0, std=0.02)
    tok = om.tokens_for_step(cfg, 4, cfg.seq, seed=1)
    m, loss, G = run_step(cfg, P, tok, dtype=dtype)
    Pm = as_multiplied(P, dtype)
    lo, cache = om.forward(cfg, Pm, tok, loss_scale=256.0)
    Go = om.backward(cfg, Pm, cache)
    assert abs(loss - lo) <= LOSS_RTOL * abs(lo), (loss, lo)
    errs = sorted(((rel_l2(G[n], Go[n]), n) for n in P), reverse=True)
    print("\n  worst grad rel-L2: " + ", ".join(f"{n}={e:.2e}" for e, n in errs[:6]))
    for n in P:
        assert rel_l2(G[n], Go[n]) <= grad_tol(n, dtype), (n, rel_l2(G[n], Go[n]))
    m.close()


@pytest.mark.parametrize("dtype", [ne.NE_FP16, ne.NE_BF16])
def test_reference_norm_formula_step_matches_oracle(dtype):
    """ne_rmsnorm_bwd_formula: with trained (non-unit) gains the step follows the oracle's
    reference-formula backward when switched on and the exact one when switched off again; the
    one-stream step replays a captured graph, so the switch must drop it."""
    cfg = om.tiny(**CASES["qwen3"])
    P = om.init_params(cfg, seed=0, std=0.02)
    rng = np.random.default_rng(3)
    for n in P:
        if om.is_gain(n):
            P[n] = (1 + 0.5 * rng.standard_normal(P[n].shape)).astype(np.float32)
    tok = om.tokens_for_step(cfg, 2, cfg.seq, seed=1)
    print(f"\n[dtype {dtype}] tiny qwen3 model B=2 S={cfg.seq}, gains 1 +- 0.5", flush=True)
    m = ne.Model.from_oracle(cfg, batch=2, dtype=dtype)
    m.set_params(P)
    m.overlap_weight_grads(False)
    Pm = as_multiplied(P, dtype)
    lo, cache = om.forward(cfg, Pm, tok, loss_scale=256.0)
    for ref in (False, True, False):
        m.rmsnorm_bwd_formula(ref)
        m.zero_grads()
        loss = m.train_step(tok, 256.0)
        G = m.get_all(shapes(cfg), ne.NE_GRAD)
        Go = om.backward(cfg, Pm, cache, norm_bwd_ref=ref)
        Gx = om.backward(cfg, Pm, cache, norm_bwd_ref=not ref)
        assert abs(loss - lo) <= LOSS_RTOL * abs(lo), (loss, lo)
        worst = max((rel_l2(G[n], Go[n]) / grad_tol(n, dtype), n) for n in P)
        other = max((rel_l2(G[n], Gx[n]) / grad_tol(n, dtype), n) for n in P)
        print(f"  ref={ref}: worst grad rel-L2 / tol {worst[0]:.2f} ({worst[1]}); "
              f"against the other formula {other[0]:.2f} ({other[1]})", flush=True)
        assert worst[0] <= 1.0, worst
        assert other[0] > 1.0, other
    m.close()


def test_step_with_ragged_vocab_tiles():
    """A vocabulary that is not a multiple of 256 (65,664 = 256.5 tiles) with 256 tokens: the
    classifier / CE GEMMs and the embedding-gradient GEMM take tiles that divide it.  A store
    past the last embedding row would land in the gain gradients that follow it in G, which
    the comparison with the oracle covers."""
    cfg = om.tiny(**CASES["qwen3"], vocab=65664)
    P = om.init_params(cfg, seed=0, std=0.02)
    tok = om.tokens_for_step(cfg, 4, cfg.seq, seed=1)
    lo, cache = om.forward(cfg, P, tok, loss_scale=256.0)
    Go = om.backward(cfg, P, cache)
    m, loss, G = run_step(cfg, P, tok)
    m.close()
    assert abs(loss - lo) <= LOSS_RTOL * abs(lo), (loss, lo)
    for n in P:
        assert rel_l2(G[n], Go[n]) <= GRAD_RL2, (n, rel_l2(G[n], Go[n]))


def test_grads_accumulate_and_zero():
    cfg = om.tiny()
    P = om.init_params(cfg, seed=0, std=0.02)
    tok = om.tokens_for_step(cfg, 1, cfg.seq, seed=2)
    m = ne.Model.from_oracle(cfg, batch=1)
    m.set_params(P)
    m.train_step(tok, 1.0)
    g1 = m.get("layers.1.W2", ne.NE_GRAD)
    m.train_step(tok, 1.0)
    g2 = m.get("layers.1.W2", ne.NE_GRAD)
    assert rel_l2(g2, 2 * g1) < 1e-5
    m.zero_grads()
    assert np.abs(m.get("layers.1.W2", ne.NE_GRAD)).max() == 0
    m.close()


@pytest.mark.parametrize("overlap", [True, False])
def test_overflowed_window_skips_the_update(overlap):
    """A 16-bit overflow in the accumulation window (a final-norm gain of 1e6 takes the 16-bit
    final hidden state past the fp16 range) skips the update: the optimizer reports a NaN norm,
    parameters and moments stay as they were bit for bit, Adam's step count does not advance, the
    internal gradient scale halves and an overflow site is named; the next clean window updates
    as usual."""
    cfg = om.tiny(qk_norm=True)
    sh = shapes(cfg)
    P = om.init_params(cfg, seed=3, std=0.02)
    tok = om.tokens_for_step(cfg, 1, cfg.seq, seed=4)
    m = ne.Model.from_oracle(cfg, batch=1)
    m.overlap_weight_grads(overlap)
    m.set_params(P)
    m.train_step(tok, 256.0)
    assert np.isfinite(m.optimizer_step(3e-4, grad_scale=1 / 256, clip=1.0))
    m.set("rms_final", m.get("rms_final") * np.float32(1e6))
    before = {k: m.get_all(sh, k) for k in (ne.NE_PARAM, ne.NE_ADAM_M, ne.NE_ADAM_V)}
    t0, (scale0, skipped0, _) = m.state().adam_t, m.grad_scale_info()
    m.train_step(tok, 256.0)
    assert np.isnan(m.optimizer_step(3e-4, grad_scale=1 / 256, clip=1.0))
    scale, skipped, sites = m.grad_scale_info()
    assert skipped == skipped0 + 1 and sites and scale == scale0 / 2, (skipped, sites, scale)
    assert m.state().adam_t == t0
    for k, want in before.items():
        got = m.get_all(sh, k)
        for n in want:
            np.testing.assert_array_equal(got[n], want[n], err_msg=f"kind {k} {n}")
    m.set("rms_final", before[ne.NE_PARAM]["rms_final"] / np.float32(1e6))
    m.train_step(tok, 256.0)
    assert np.isfinite(m.optimizer_step(3e-4, grad_scale=1 / 256, clip=1.0))
    assert m.state().adam_t == t0 + 1 and m.grad_scale_info()[1] == skipped
    after = m.get_all(sh, ne.NE_PARAM)
    assert any(not np.array_equal(after[n], before[ne.NE_PARAM][n]) for n in after if n != "rms_final")
    m.close()


@pytest.mark.parametrize("clip", [1.0, 1e-3])
def test_optimizer_step_matches_oracle(clip):
    """Same grads in -> AdamW out within 1e-5 (isolates the update from bf16 gradients)."""
    cfg = om.tiny(qk_norm=True)
    rng = np.random.default_rng(5)
    P = om.init_params(cfg, seed=3, std=0.02)
    G = {k: (rng.standard_normal(v.shape) * 1e-2 * 256).astype(np.float32) for k, v in P.items()}
    M = {k: (rng.standard_normal(v.shape) * 1e-3).astype(np.float32) for k, v in P.items()}
    V = {k: (np.abs(rng.standard_normal(v.shape)) * 1e-5).astype(np.float32) for k, v in P.items()}
    m = ne.Model.from_oracle(cfg)
    m.set_params(P)
    m.set_params(G, ne.NE_GRAD)
    m.set_params(M, ne.NE_ADAM_M)
    m.set_params(V, ne.NE_ADAM_V)
    st = m.state()
    st.adam_t = 4
    m.set_state(st)
    gn = m.optimizer_step(3e-4, 0.9, 0.95, 1e-8, 0.1, grad_scale=1 / 256, clip=clip)
    Po = {k: v.copy() for k, v in P.items()}
    Go = {k: v.copy() for k, v in G.items()}
    gno = om.optimizer_step(Po, Go, M, V, 5, 3e-4, grad_scale=1 / 256, clip=clip)
    assert abs(gn - gno) < 1e-5 * gno
    sh = shapes(cfg)
    Pg = m.get_all(sh)
    # per element within 1e-5 relative; absolute floor = one fp32 ulp at the tensor's scale
    for n in P:
        np.testing.assert_allclose(Pg[n], Po[n], rtol=ADAM_RTOL, atol=1e-7 * np.abs(Po[n]).max(), err_msg=n)
    Mg = m.get_all(sh, ne.NE_ADAM_M)
    for n in P:
        np.testing.assert_allclose(Mg[n], M[n], rtol=ADAM_RTOL, atol=1e-7 * np.abs(M[n]).max(), err_msg=n)
    assert max(np.abs(m.get(n, ne.NE_GRAD)).max() for n in P) == 0
    assert m.state().adam_t == 5
    m.close()


@pytest.mark.parametrize("compact", [False, True])
@pytest.mark.parametrize("overlap", [False, True])
def test_grad_norm_from_step_partials(compact, overlap):
    """The optimizer's gradient norm comes from sum-of-squares partials the step leaves as each
    part of G becomes final (per layer, the embedding before the input-embedding scatter plus
    the change the scatter makes to each row, the gains).  Over two accumulating micro-steps
    (repeated token ids, so the scatter updates rows that already hold gradient) it equals the
    float64 norm of the gradients read back; after a direct gradient write the optimizer sums
    G itself."""
    cfg = om.tiny(**CASES["qwen3"])
    P = om.init_params(cfg, seed=0, std=0.02)
    toks = [om.tokens_for_step(cfg, 2, cfg.seq, seed=s) for s in (1, 2)]
    sh = shapes(cfg)
    m = ne.Model.from_oracle(cfg, batch=2)
    m.overlap_weight_grads(overlap)
    if compact:
        m.set_vocab_map(np.unique(np.concatenate([t.ravel() for t in toks])).astype(np.int32))
    m.set_params(P)

    def norm64(G):
        return float(np.sqrt(sum(np.sum(g.astype(np.float64) ** 2) for g in G.values())))

    for t in toks:
        m.train_step(t, 256.0)
    want = norm64(m.get_all(sh, ne.NE_GRAD)) / 256
    gn = m.optimizer_step(3e-4, 0.9, 0.95, 1e-8, 0.1, grad_scale=1 / 256, clip=0.0)
    print(f"\n[compact={compact} overlap={overlap}] norm {gn:.7f} float64 {want:.7f}", flush=True)
    assert abs(gn - want) <= 1e-6 * want, (gn, want)
    m.train_step(toks[1], 256.0)
    G = m.get_all(sh, ne.NE_GRAD)
    G["layers.1.Wq"] = G["layers.1.Wq"] * 3.0
    m.set("layers.1.Wq", G["layers.1.Wq"], ne.NE_GRAD)
    want = norm64(G) / 256
    gn = m.optimizer_step(3e-4, 0.9, 0.95, 1e-8, 0.1, grad_scale=1 / 256, clip=0.0)
    assert abs(gn - want) <= 1e-6 * want, (gn, want)
    # no micro-step since the update: all-zero gradients
    assert m.optimizer_step(3e-4, 0.9, 0.95, 1e-8, 0.1, grad_scale=1 / 256, clip=0.0) == 0.0
    m.close()


def _held_params(cfg, dtype, seed=0, std=0.02):
    """Weights rounded to the context's 16-bit format, so the decode's weight shadow and the
    fp32 oracle see identical values."""
    P = om.init_params(cfg, seed=seed, std=std)
    if dtype == ne.NE_BF16:
        return {k: om.round_bf16(v) for k, v in P.items()}
    return {k: v.astype(np.float16).astype(np.float32) for k, v in P.items()}


@pytest.mark.parametrize("dtype", [ne.NE_BF16, ne.NE_FP16])
@pytest.mark.parametrize("case", ["ref", "qwen3"])
def test_decode_greedy_matches_oracle(case, dtype):
    cfg = om.tiny(**CASES[case], vocab=1024)
    P = _held_params(cfg, dtype, std=0.05)
    prompt = np.random.default_rng(2).integers(0, cfg.vocab, (3, 8)).astype(np.int32)
    m = ne.Model.from_oracle(cfg, decode_batch=3, decode_ctx=64, dtype=dtype)
    m.set_params(P)
    got = m.decode(prompt, 24)
    want, margins, _ = om.decode(cfg, P, prompt, 24, return_logits=True)
    print(f"\n  min top-2 margin {margins.min():.3e}")
    np.testing.assert_array_equal(got, want)
    m.close()


def test_four_query_heads_per_kv_head():
    """GQA with four query heads per KV head (the other tests run two and one): the training
    step's gradients against the oracle, and greedy decoding token-identical to it on the
    small-batch path (one query head per attention block) and the batched bf16 path (all four
    query heads of a KV head per block)."""
    cfg = om.tiny(**CASES["qwen3"], n_heads=8, kv_heads=2, vocab=1024)
    P = om.init_params(cfg, seed=0, std=0.02)
    tok = om.tokens_for_step(cfg, 2, cfg.seq, seed=1)
    m, loss, G = run_step(cfg, P, tok)
    Pm = as_multiplied(P, ne.NE_FP16)
    lo, cache = om.forward(cfg, Pm, tok, loss_scale=256.0)
    Go = om.backward(cfg, Pm, cache)
    m.close()
    assert abs(loss - lo) <= LOSS_RTOL * abs(lo), (loss, lo)
    for n in P:
        assert rel_l2(G[n], Go[n]) <= grad_tol(n, ne.NE_FP16), (n, rel_l2(G[n], Go[n]))
    Pd = _held_params(cfg, ne.NE_BF16, std=0.05)
    for B in (1, 6):
        prompt = np.random.default_rng(B).integers(0, cfg.vocab, (B, 8)).astype(np.int32)
        md = ne.Model.from_oracle(cfg, decode_batch=B, decode_ctx=64, dtype=ne.NE_BF16)
        md.set_params(Pd)
        got = md.decode(prompt, 24)
        md.close()
        want = om.decode(cfg, Pd, prompt, 24)
        want = want[0] if isinstance(want, tuple) else want
        np.testing.assert_array_equal(got, want, err_msg=f"B={B}")


@pytest.mark.parametrize("B", [3, 6])
def test_decode_long_cache_splits_match_oracle(B):
    """A cache of 4200 positions (scores of every position in LDS) with a 150-token prompt:
    B=3 takes the VALU GEMVs, B=6 the MFMA GEMVs."""
    cfg = om.tiny(**CASES["qwen3"], vocab=1024)
    P = _held_params(cfg, ne.NE_BF16, std=0.05)
    prompt = np.random.default_rng(5).integers(0, cfg.vocab, (B, 150)).astype(np.int32)
    m = ne.Model.from_oracle(cfg, decode_batch=B, decode_ctx=4200, dtype=ne.NE_BF16)
    m.set_params(P)
    got = m.decode(prompt, 40)
    want, margins, _ = om.decode(cfg, P, prompt, 40, return_logits=True)
    print(f"\n  min top-2 margin {margins.min():.3e}")
    np.testing.assert_array_equal(got, want)
    m.close()


def test_decode_seeded_matches_generate_draws():
    """ne_decode_seeded: the tokens of the oracle's token loop on the draws generate.py makes
    after np.random.seed(seed), one RandomState.random_sample per sampled token (B = 1), and,
    with B = 2, position by position, the sequences of a position in order; greedy draws
    nothing and equals ne_decode's greedy tokens."""
    cfg = om.tiny(**CASES["qwen3"], vocab=1024)
    P = _held_params(cfg, ne.NE_BF16, std=0.3)
    prompt = np.random.default_rng(5).integers(0, cfg.vocab, (2, 5)).astype(np.int32)
    m = ne.Model.from_oracle(cfg, decode_batch=2, decode_ctx=32, dtype=ne.NE_BF16)
    m.set_params(P)
    n = 12
    for seed, temp, top_p in ((3, 0.6, 1.0), (11, 0.8, 0.9)):
        got1 = m.decode_seeded(prompt[:1], n, temp, top_p, seed)
        u1 = np.random.RandomState(seed).random_sample((1, n))
        want1 = om.decode(cfg, P, prompt[:1], n, temperature=temp, top_p=top_p, uniforms=u1)
        np.testing.assert_array_equal(got1, want1, err_msg=f"B=1 seed={seed}")
        got2 = m.decode_seeded(prompt, n, temp, top_p, seed)
        u2 = np.random.RandomState(seed).random_sample((n, 2)).T   # position-major draws
        want2 = om.decode(cfg, P, prompt, n, temperature=temp, top_p=top_p, uniforms=u2)
        np.testing.assert_array_equal(got2, want2, err_msg=f"B=2 seed={seed}")
    np.testing.assert_array_equal(m.decode_seeded(prompt, n, 0.0, 1.0, 9), m.decode(prompt, n))
    m.close()


def test_decode_sampling_matches_oracle():
    cfg = om.tiny(**CASES["qwen3"], vocab=1024)
    P = _held_params(cfg, ne.NE_BF16, std=0.3)
    prompt = np.random.default_rng(3).integers(0, cfg.vocab, (2, 5)).astype(np.int32)
    u = np.random.RandomState(3).random_sample((2, 16))
    m = ne.Model.from_oracle(cfg, decode_batch=2, decode_ctx=32, dtype=ne.NE_BF16)
    m.set_params(P)
    for temp, top_p in ((0.6, 1.0), (0.8, 0.9)):
        got = m.decode(prompt, 16, temperature=temp, top_p=top_p, uniforms=u)
        want = om.decode(cfg, P, prompt, 16, temperature=temp, top_p=top_p, uniforms=u)
        np.testing.assert_array_equal(got, want, err_msg=f"temp={temp} top_p={top_p}")
    m.close()


def test_checkpoint_roundtrip_with_oracle_reader(tmp_path):
    cfg = om.tiny(qk_norm=True, n_layers=1)
    P = om.init_params(cfg, seed=4, std=0.02)
    rng = np.random.default_rng(0)
    M = {k: rng.standard_normal(v.shape).astype(np.float32) for k, v in P.items()}
    V = {k: rng.standard_normal(v.shape).astype(np.float32) for k, v in P.items()}
    m = ne.Model.from_oracle(cfg)
    m.set_params(P)
    m.set_params(M, ne.NE_ADAM_M)
    m.set_params(V, ne.NE_ADAM_V)
    st = ne.TrainState(step=100, total_steps=1000, lr=2e-4, loss=5.5, adam_t=10, cum_steps=100)
    path = tmp_path / "c.bin"
    m.save(path, st)
    assert path.stat().st_size == ckpt.expected_size(cfg)
    h, P2, M2, V2 = ckpt.read(path)
    assert h["step"] == 100 and h["adam_t"] == 10 and abs(h["loss"] - 5.5) < 1e-6
    for n in P:
        np.testing.assert_array_equal(P2[n], P[n])
        np.testing.assert_array_equal(M2[n], M[n])
        np.testing.assert_array_equal(V2[n], V[n])
    # oracle-written file loads back into a fresh context
    path2 = tmp_path / "d.bin"
    ckpt.write(path2, cfg, P2, V2, M2, step=3, adam_t=2)
    m2 = ne.Model.from_oracle(cfg)
    st2 = m2.load(path2)
    assert st2.step == 3 and st2.adam_t == 2
    for n in P:
        np.testing.assert_array_equal(m2.get(n).reshape(P[n].shape), P[n])
        np.testing.assert_array_equal(m2.get(n, ne.NE_ADAM_M).reshape(P[n].shape), V[n])
    # truncated file is rejected with a size error
    raw = path2.read_bytes()
    (tmp_path / "t.bin").write_bytes(raw[:-4])
    with pytest.raises(ne.NEError, match="size"):
        m2.load(tmp_path / "t.bin")
    m.close()
    m2.close()


def test_graph_replay_matches_eager_launches():
    """The captured-graph step and the eagerly launched step give the same loss and grads,
    for the overwrite (first micro-step) and the accumulate variants."""
    cfg = om.tiny(**CASES["qwen3"])
    P = om.init_params(cfg, seed=0, std=0.02)
    toks = [om.tokens_for_step(cfg, 2, cfg.seq, seed=s) for s in (1, 2)]
    out = []
    for graphs in (True, False):
        m = ne.Model.from_oracle(cfg, batch=2)
        m.use_graphs(graphs)
        m.overlap_weight_grads(False)  # the two-stream step is never captured
        m.set_params(P)
        losses = [m.train_step(t, 256.0) for t in toks] + [m.train_step(toks[0], 256.0)]
        out.append((losses, m.get_all(shapes(cfg), ne.NE_GRAD)))
        m.close()
    (l1, g1), (l2, g2) = out
    assert l1 == l2
    for n in g1:
        np.testing.assert_allclose(g1[n], g2[n], rtol=1e-6, atol=1e-9, err_msg=n)


@pytest.mark.parametrize("B", [1, 2, 4, 5, 16, 32])
def test_decode_batch_sizes_match_oracle(B):
    """Greedy decode through both GEMV paths (VALU for batch <= 4, split-K MFMA above), with
    the per-position HIP graphs reused across calls of the same batch size and rebuilt for a
    new one."""
    cfg = om.tiny(**CASES["qwen3"], vocab=1024)
    P = _held_params(cfg, ne.NE_BF16, std=0.05)
    prompt = np.random.default_rng(10 + B).integers(0, cfg.vocab, (B, 6)).astype(np.int32)
    m = ne.Model.from_oracle(cfg, decode_batch=32, decode_ctx=64, dtype=ne.NE_BF16)
    m.set_params(P)
    want = om.decode(cfg, P, prompt, 20)
    for _ in range(2):  # second call replays the cached graphs
        np.testing.assert_array_equal(m.decode(prompt, 20), want)
    # a different batch size and prompt length on the same context
    p2 = prompt[:1, :3]
    np.testing.assert_array_equal(m.decode(p2, 12), om.decode(cfg, P, p2, 12))
    m.close()


def test_decode_sampling_mfma_path():
    cfg = om.tiny(**CASES["qwen3"], vocab=1024)
    P = _held_params(cfg, ne.NE_BF16, std=0.3)
    prompt = np.random.default_rng(4).integers(0, cfg.vocab, (8, 5)).astype(np.int32)
    u = np.random.RandomState(5).random_sample((8, 12))
    m = ne.Model.from_oracle(cfg, decode_batch=8, decode_ctx=32, dtype=ne.NE_BF16)
    m.set_params(P)
    got = m.decode(prompt, 12, temperature=0.6, top_p=0.95, uniforms=u)
    want = om.decode(cfg, P, prompt, 12, temperature=0.6, top_p=0.95, uniforms=u)
    np.testing.assert_array_equal(got, want)
    m.close()


@pytest.mark.parametrize("B", [6, 32])
def test_decode_stories_widths_batched(B):
    """Stories110M widths (dim 768, hidden 2048, 12 heads of 64, vocab 32000; two layers) with
    bf16 weights at batch 6 and 32: the batched GEMVs split K = 768 and 2048 three and eight
    ways, and the SwiGLU gate and the LM head take K = 768 in one split."""
    cfg = om.stories110m(n_layers=2)
    P = _held_params(cfg, ne.NE_BF16, std=0.05)
    prompt = np.random.default_rng(30 + B).integers(0, cfg.vocab, (B, 4)).astype(np.int32)
    print(f"\n[B={B}] stories widths, 2 layers", flush=True)
    m = ne.Model.from_oracle(cfg, decode_batch=B, decode_ctx=32, dtype=ne.NE_BF16)
    m.set_params(P)
    got = m.decode(prompt, 12)
    want, margins, _ = om.decode(cfg, P, prompt, 12, return_logits=True)
    print(f"  min top-2 margin {margins.min():.3e}")
    np.testing.assert_array_equal(got, want)
    m.close()


@pytest.mark.parametrize("compact", [False, True])
def test_step_identical_across_launch_modes(compact):
    """The step gives bit-identical losses and gradients over two accumulating micro-steps
    whether its kernels are launched eagerly with the weight-gradient GEMMs and the optimizer
    update on a second stream (two_streams, the default: the update overlaps the next step's
    forward), in order on one stream with per-kernel profiling events between them
    (profiled), or in order replayed from a HIP graph (graph); the same holds for the
    weights after two updates and the gradients of the steps that follow them."""
    cfg = om.tiny(**CASES["qwen3"], n_layers=2, dim=1024, hidden=4096, vocab=4096, seq=256)
    P = om.init_params(cfg, seed=0, std=0.02)
    toks = [om.tokens_for_step(cfg, 2, cfg.seq, seed=s) for s in (1, 2)]
    ids = np.unique(np.concatenate([t.ravel() for t in toks])).astype(np.int32)
    out = []
    for mode in ("profiled", "two_streams", "graph"):
        print(f"\n[compact={compact}] mode {mode}", flush=True)
        m = ne.Model.from_oracle(cfg, batch=2)
        m.use_graphs(mode == "graph")
        m.overlap_weight_grads(mode == "two_streams")
        if mode == "profiled":
            m.prof_enable()
        if compact:
            m.set_vocab_map(ids)
        m.set_params(P)
        losses = [m.train_step(t, 256.0) for t in toks]
        g_acc = m.get_all(shapes(cfg), ne.NE_GRAD)
        # an update, then a step whose forward overlaps it (two_streams), then another update
        gn = [m.optimizer_step(3e-4, 0.9, 0.95, 1e-8, 0.1, grad_scale=1 / 256, clip=1.0)]
        losses.append(m.train_step(toks[0], 256.0))
        gn.append(m.optimizer_step(3e-4, 0.9, 0.95, 1e-8, 0.1, grad_scale=1 / 256, clip=1.0))
        losses.append(m.train_step(toks[1], 256.0))
        out.append((losses, gn, g_acc, m.get_all(shapes(cfg), ne.NE_GRAD), m.get_all(shapes(cfg))))
        m.close()
    (l0, n0, *t0) = out[0]
    for li, ni, *ti in out[1:]:
        assert li == l0
        assert ni == n0
        for a, b in zip(ti, t0):
            for n in b:
                np.testing.assert_array_equal(a[n], b[n], err_msg=n)


def test_update_sequences_identical_across_launch_modes():
    """At Qwen3-0.6B's layer shapes and 256 tokens (the weight-gradient GEMMs of a short step),
    sequences of accumulating micro-steps, optimizer updates (each deferred to the next step's
    forward on two streams), zero_grads, a gradient read and a switch to one stream and back
    leave the losses, gradient norms, gradients and weights bit-identical between in-order
    launches on one stream and the two-stream schedule."""
    cfg = om.tiny(**CASES["qwen3"], n_layers=2, dim=1024, hidden=3072, n_heads=16, kv_heads=8,
                  head_dim=128, vocab=4096, seq=128)
    P = om.init_params(cfg, seed=0, std=0.02)
    toks = [om.tokens_for_step(cfg, 2, cfg.seq, seed=s) for s in (1, 2, 3)]
    opt = dict(lr=3e-4, b1=0.9, b2=0.95, eps=1e-8, wd=0.1, grad_scale=1 / 256, clip=1.0)
    out = []
    for mode in ("profiled", "two_streams"):
        print(f"\nmode {mode}", flush=True)
        m = ne.Model.from_oracle(cfg, batch=2)
        m.overlap_weight_grads(mode == "two_streams")
        if mode == "profiled":
            m.prof_enable()
        m.set_params(P)
        rec = []
        # two accumulating micro-steps, then an update over the accumulated sum
        rec += [m.train_step(toks[0], 256.0), m.train_step(toks[1], 256.0)]
        rec.append(m.optimizer_step(**opt))
        # one micro-step (the update above beside its forward), an update of its fresh sum
        rec.append(m.train_step(toks[2], 256.0))
        rec.append(m.optimizer_step(**opt))
        # a micro-step whose gradients are dropped, then one whose gradients are read
        rec.append(m.train_step(toks[0], 256.0))
        m.zero_grads()
        rec.append(m.train_step(toks[1], 256.0))
        g1 = m.get_all(shapes(cfg), ne.NE_GRAD)
        rec.append(m.optimizer_step(**opt))
        # a micro-step left pending across a switch to one stream and back
        rec.append(m.train_step(toks[2], 256.0))
        m.overlap_weight_grads(False)
        m.overlap_weight_grads(mode == "two_streams")
        rec.append(m.train_step(toks[0], 256.0))
        rec.append(m.optimizer_step(**opt))
        rec.append(m.train_step(toks[1], 256.0))
        out.append((rec, g1, m.get_all(shapes(cfg), ne.NE_GRAD), m.get_all(shapes(cfg))))
        m.close()
    (r0, *t0), (r1, *t1) = out
    assert r1 == r0
    for a, b in zip(t1, t0):
        for n in b:
            np.testing.assert_array_equal(a[n], b[n], err_msg=n)


def test_step_timeline():
    """ne_step_timeline: the phases of the last step (HIP events at its phase boundaries on
    the step stream) are non-negative and add up to no more than the step, each layer's
    forward and backward time is positive and their sums stay inside their phases; the
    timeline changes no result (the losses of the same steps with it off are identical)."""
    cfg = om.tiny(**CASES["qwen3"], n_layers=3)
    P = om.init_params(cfg, seed=0, std=0.02)
    toks = [om.tokens_for_step(cfg, 2, cfg.seq, seed=s) for s in (1, 2, 3)]
    runs = []
    for on in (False, True):
        m = ne.Model.from_oracle(cfg, batch=2)
        m.set_params(P)
        m.timeline(on)
        if on:
            with pytest.raises(ne.NEError):
                m.step_timeline()      # no step with the timeline on yet
        losses = []
        for t in toks:
            losses.append(m.train_step(t, 256.0))
            m.optimizer_step(3e-4, 0.9, 0.95, 1e-8, 0.1, grad_scale=1 / 256, clip=1.0)
        losses.append(m.train_step(toks[0], 256.0))
        if on:
            ph, lf, lb = m.step_timeline(layers=True)
            print("\n[timeline]", ph, lf, lb, flush=True)
            parts = ("wait", "fwd", "cls", "bwd", "dwait", "tail")
            assert all(ph[k] >= 0 for k in parts + ("opt", "update")), ph
            assert sum(ph[k] for k in parts) <= ph["step"] * (1 + 1e-3) + 1e-3
            assert ph["fwd"] > 0 and ph["bwd"] > 0 and ph["update"] > 0
            assert (lf > 0).all() and (lb > 0).all()
            assert lf.sum() <= ph["fwd"] * (1 + 1e-3) + 1e-3 and lb.sum() <= ph["bwd"] * (1 + 1e-3) + 1e-3
        runs.append(losses)
        m.close()
    assert runs[0] == runs[1]


def _compact_case(vocab=1024, seed=5):
    cfg = om.tiny(qk_norm=True, rope_theta=1e6, res_alpha=om.train_alpha(2), vocab=vocab)
    rng = np.random.default_rng(seed)
    data = rng.choice(np.arange(100, 900, 7), size=4096).astype(np.int32)   # 115 distinct ids
    ids = om.vocab_map_build(data, cfg.vocab)
    starts = rng.integers(0, len(data) - cfg.seq - 1, 2)
    tok = np.stack([data[s:s + cfg.seq + 1] for s in starts]).astype(np.int32)
    return cfg, data, ids, tok


@pytest.mark.parametrize("dtype", [ne.NE_FP16, ne.NE_BF16])
def test_compact_vocab_step_matches_oracle(dtype):
    """Vocabulary compaction (TD/cpu_ops.h:384-431): classifier and softmax over the ids of
    the data (115 of 1024, padded to 128 columns), compact gradient added back to its rows;
    two accumulated micro-steps, then back to the full vocabulary.  The bf16 step is compared
    with the oracle on the bf16-rounded matrices it multiplies."""
    cfg, data, ids, tok = _compact_case()
    P = om.init_params(cfg, seed=0, std=0.02)
    m = ne.Model.from_oracle(cfg, batch=2, dtype=dtype)
    m.set_params(P)
    m.set_vocab_map(ids)
    tok2 = np.roll(tok, 7, axis=1)
    loss = m.train_step(tok, 256.0)
    loss2 = m.train_step(tok2, 256.0)
    G = m.get_all(shapes(cfg), ne.NE_GRAD)
    Pm = as_multiplied(P, dtype)
    lo, cache = om.forward(cfg, Pm, tok, loss_scale=256.0, vocab_ids=ids)
    Go = om.backward(cfg, Pm, cache)
    lo2, cache2 = om.forward(cfg, Pm, tok2, loss_scale=256.0, vocab_ids=ids)
    Go2 = om.backward(cfg, Pm, cache2)
    print(f"\n  compact loss gpu={loss:.6f}/{loss2:.6f} oracle={lo:.6f}/{lo2:.6f} (ln CV = {np.log(len(ids)):.4f})")
    assert abs(loss - lo) <= LOSS_RTOL * abs(lo) and abs(loss2 - lo2) <= LOSS_RTOL * abs(lo2)
    for n in P:
        assert rel_l2(G[n], Go[n] + Go2[n]) <= grad_tol(n, dtype), (n, rel_l2(G[n], Go[n] + Go2[n]))
    unused = np.setdiff1d(np.arange(cfg.vocab), ids)
    assert np.abs(G["embed"].reshape(cfg.vocab, -1)[unused]).max() == 0
    # the map is fixed inside an accumulation window
    with pytest.raises(ne.NEError):
        m.set_vocab_map(None)
    m.zero_grads()
    m.set_vocab_map(None)
    loss_f = m.train_step(tok, 256.0)
    lf, _ = om.forward(cfg, Pm, tok, loss_scale=256.0, want_grad_cache=False)
    assert abs(loss_f - lf) <= LOSS_RTOL * abs(lf)
    m.close()


def test_classifier_pieces_match_whole():
    """With the full 151,936-entry vocabulary at 256 tokens the classifier's logits GEMM runs
    in vocabulary pieces, each after the AdamW chunk of its embedding rows (on two streams,
    beside the previous update's tail).  An identity vocabulary map runs the same GEMM whole
    after the entire update: over two micro-steps and updates both give bit-identical losses,
    gradients and weights (the pieces change neither the tiles nor their sums, and each waits
    for its rows' update).  The gradient norm is summed by different kernels in the two
    forms (the embedding gradient's GEMM tiles against a pass over the scattered compact
    gradient), so it is compared to 1e-6 and the updates run unclipped."""
    cfg = om.tiny(**CASES["qwen3"], n_layers=1, dim=1024, hidden=3072, n_heads=16, kv_heads=8,
                  head_dim=128, vocab=151936, seq=256)
    P = om.init_params(cfg, seed=0, std=0.02)
    toks = [om.tokens_for_step(cfg, 1, cfg.seq, seed=s) for s in (1, 2)]
    opt = dict(lr=3e-4, b1=0.9, b2=0.95, eps=1e-8, wd=0.1, grad_scale=1 / 256, clip=1e9)
    out = []
    for mapped in (False, True):
        print(f"\nidentity map {mapped}", flush=True)
        m = ne.Model.from_oracle(cfg, batch=1)
        # the pass beside the forward: the gains, the layer, the embedding in the 4 pieces of
        # 256, 256, 256 and 419 work-groups of 256 x 128 logits tiles
        assert m.update_launches() == 1 + cfg.n_layers + 4
        m.set_params(P)
        if mapped:
            m.set_vocab_map(np.arange(cfg.vocab, dtype=np.int32))
        losses, norms = [m.train_step(toks[0], 256.0)], [m.optimizer_step(**opt)]
        losses.append(m.train_step(toks[1], 256.0))
        g = m.get_all(shapes(cfg), ne.NE_GRAD)
        norms.append(m.optimizer_step(**opt))
        losses.append(m.train_step(toks[0], 256.0))
        out.append((losses, norms, g, m.get_all(shapes(cfg))))
        m.close()
    (l0, n0, *t0), (l1, n1, *t1) = out
    assert l1 == l0
    np.testing.assert_allclose(n1, n0, rtol=1e-6)
    for a, b in zip(t1, t0):
        for n in b:
            np.testing.assert_array_equal(a[n], b[n], err_msg=n)


def test_compact_vocab_rejects_bad_maps_and_targets():
    cfg, data, ids, tok = _compact_case()
    m = ne.Model.from_oracle(cfg, batch=2)
    with pytest.raises(ne.NEError):
        m.set_vocab_map(np.array([3, 5, 3], np.int32))        # repeated id
    with pytest.raises(ne.NEError):
        m.set_vocab_map(np.array([3, cfg.vocab], np.int32))   # out of range
    m.set_vocab_map(ids[1:])
    bad = tok.copy()
    bad[0, 5] = ids[0]                                       # a target outside the map
    with pytest.raises(ne.NEError):
        m.train_step(bad, 256.0)
    m.close()


def test_step_stats_and_grad_norm_parts():
    """The step line's ranges (TD/train.m:770-777): x = the last layer's output, dy = the
    gradient of loss * loss_scale with respect to the first layer's input, in the reference's
    scale; with every input token distinct, dy's rows are the embedding-gradient rows of those
    tokens in the oracle.  The grad-norm line's groups (TD/train.m:786-830) equal the float64
    norms of the gradients read back, scaled by grad_scale."""
    cfg = om.tiny(**CASES["qwen3"])
    P = om.init_params(cfg, seed=0, std=0.02)
    tok = np.random.default_rng(4).permutation(cfg.vocab)[: 2 * (cfg.seq + 1)].reshape(2, cfg.seq + 1)
    tok = tok.astype(np.int32)
    m = ne.Model.from_oracle(cfg, batch=2)
    m.set_params(P)
    with pytest.raises(ne.NEError):
        m.step_stats()          # no step yet
    m.train_step(tok, 256.0)
    xmn, xmx, dmn, dmx = m.step_stats()
    lo, cache = om.forward(cfg, P, tok, loss_scale=256.0)
    Go = om.backward(cfg, P, cache)
    xL = cache["xL"]
    # the tied embedding's gradient row of a (distinct) input token is the classifier's
    # dlogits^T . xf row plus the first layer's input gradient: take the classifier's part out
    T = 2 * cfg.seq
    dE_cls = (cache["dlogits"].reshape(T, -1).T @ cache["xf"].reshape(T, -1)).astype(np.float32)
    inp = tok[:, :-1].ravel()
    dy = Go["embed"][inp] - dE_cls[inp]
    print(f"\n  x [{xmn:.4f}, {xmx:.4f}] oracle [{xL.min():.4f}, {xL.max():.4f}]; "
          f"dy [{dmn:.3e}, {dmx:.3e}] oracle [{dy.min():.3e}, {dy.max():.3e}]")
    assert abs(xmn - xL.min()) <= 1e-3 * np.abs(xL).max() and abs(xmx - xL.max()) <= 1e-3 * np.abs(xL).max()
    assert abs(dmn - dy.min()) <= 1e-3 * np.abs(dy).max() and abs(dmx - dy.max()) <= 1e-3 * np.abs(dy).max()
    sh = shapes(cfg)
    G = m.get_all(sh, ne.NE_GRAD)
    with pytest.raises(ne.NEError):
        m.grad_norm_parts()     # no update yet
    gn = m.optimizer_step(3e-4, 0.9, 0.95, 1e-8, 0.1, grad_scale=1 / 256, clip=1.0)
    tot, att, ffn, emb = m.grad_norm_parts()

    def norm(names):
        return float(np.sqrt(sum(np.sum(G[n].astype(np.float64) ** 2) for n in names))) / 256

    layer = [n for n in G if n.startswith("layers.")]
    want_att = norm([n for n in layer if n.split(".")[-1] in ("Wq", "Wk", "Wv", "Wo")])
    want_ffn = norm([n for n in layer if n.split(".")[-1] in ("W1", "W2", "W3")])
    print(f"  norms {tot:.6f} {att:.6f} {ffn:.6f} {emb:.6f}; float64 {norm(G):.6f} {want_att:.6f} "
          f"{want_ffn:.6f} {norm(['embed']):.6f}")
    assert abs(tot - gn) <= 1e-6 * gn and abs(tot - norm(G)) <= 1e-5 * norm(G)
    assert abs(att - want_att) <= 1e-5 * want_att and abs(ffn - want_ffn) <= 1e-5 * want_ffn
    assert abs(emb - norm(["embed"])) <= 1e-5 * norm(["embed"])
    m.train_step(tok, 256.0)
    with pytest.raises(ne.NEError):
        m.grad_norm_parts()     # the gradients changed since
    # a diverged run: a NaN weight makes the ranges NaN, not a finite-looking subset
    Pn = dict(P)
    Pn["layers.1.W2"] = P["layers.1.W2"].copy()
    Pn["layers.1.W2"][0, 0] = np.nan
    m.set("layers.1.W2", Pn["layers.1.W2"])
    m.train_step(tok, 256.0)
    st = m.step_stats()
    assert all(np.isnan(v) for v in st), st
    m.close()

