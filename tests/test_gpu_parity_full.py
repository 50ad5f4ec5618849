"""Full-size parity of the training step against the fp32 numpy oracle on the benchmarked
shapes: Stories110M (B=1, S=256, 10 steps of fwd+bwd+AdamW on fresh batches) and
Qwen3-0.6B (B=1, S=256, QK-norm, theta=1e6).  Tolerances: loss rel err <= 1e-3, per-tensor
gradient rel-L2 <= 1e-2; the AdamW update itself is checked to 1e-5 in
test_gpu_model.py (same grads in)."""
import time

import numpy as np
import pytest

from gpu_util import need_gpu, rel_l2
import ne
from oracle import model as om

pytestmark = pytest.mark.gpu

LOSS_RTOL = 1e-3
GRAD_RL2 = 1e-2


@pytest.fixture(autouse=True)
def _gpu():
    need_gpu()


def _compare_grads(cfg, P, tok, label, vocab_ids=None):
    m = ne.Model.from_oracle(cfg, batch=tok.shape[0])
    m.set_params(P)
    if vocab_ids is not None:
        m.set_vocab_map(vocab_ids)
    t0 = time.time()
    loss = m.train_step(tok, 256.0)
    G = m.get_all(dict(om.tensor_list(cfg)), ne.NE_GRAD)
    t1 = time.time()
    lo, cache = om.forward(cfg, P, tok, loss_scale=256.0, vocab_ids=vocab_ids)
    Go = om.backward(cfg, P, cache)
    del cache
    t2 = time.time()
    errs = sorted(((rel_l2(G[n], Go[n]), n) for n in P), reverse=True)
    print(f"\n[{label}] loss gpu={loss:.6f} oracle={lo:.6f} rel={abs(loss - lo) / lo:.2e}; "
          f"gpu {t1 - t0:.1f}s oracle {t2 - t1:.1f}s; worst grad rel-L2: "
          + ", ".join(f"{n}={e:.2e}" for e, n in errs[:5]), flush=True)
    assert abs(loss - lo) <= LOSS_RTOL * abs(lo)
    assert errs[0][0] <= GRAD_RL2, errs[0]
    return m


def test_stories110m_step_parity():
    cfg = om.stories110m(res_alpha=om.train_alpha(12))
    P = om.init_params(cfg, seed=0, std=0.02)
    tok = om.tokens_for_step(cfg, 1, 256, seed=1)
    _compare_grads(cfg, P, tok, "stories110m B=1 S=256").close()


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


def test_qwen3_step_parity():
    cfg = om.qwen3_06b(res_alpha=om.train_alpha(28))
    P = om.init_params(cfg, seed=0, std=0.02)
    tok = om.tokens_for_step(cfg, 1, 256, seed=1)
    _compare_grads(cfg, P, tok, "qwen3-0.6b B=1 S=256 qk-norm theta=1e6").close()


@pytest.mark.parametrize("B", [1, 32])
def test_qwen3_decode_greedy_64_tokens(B):
    """The Qwen3-0.6B token loop: bf16-held N(0, 0.02) weights from seed 0, a 32-token
    prompt of uniform ids, 64 greedy tokens, token-identical to the oracle's generate
    path on the same bf16 weights (fp32 activations and KV cache on both sides)."""
    cfg = om.qwen3_06b(res_alpha=1.0)
    P = {k: om.round_bf16(v) for k, v in om.init_params(cfg, seed=0, std=0.02).items()}
    prompt = np.random.default_rng(2).integers(0, cfg.vocab, (B, 32)).astype(np.int32)
    m = ne.Model.from_oracle(cfg, batch=1, decode_batch=B, decode_ctx=96, dtype=ne.NE_BF16)
    m.set_params(P)
    t0 = time.time()
    got = m.decode(prompt, 64)
    t1 = time.time()
    want, margins, _ = om.decode(cfg, P, prompt, 64, return_logits=True)
    print(f"\n[decode B={B}] gpu {t1 - t0:.2f}s oracle {time.time() - t1:.1f}s; "
          f"min top-2 margin {margins.min():.3e}", flush=True)
    np.testing.assert_array_equal(got, want)
    m.close()
