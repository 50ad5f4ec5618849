"""The drop-in `train` command line (neural-engine_amd/train.c, built for models/tiny.h)
against the oracle: the reference's flags, data sampling (srand48/drand48 windows of a
uint16 token file, TD/train.m:389-398), warmup+cosine LR, loss scale 256, clip, AdamW and
its v4 checkpoint save rule (TD/train.m:782-915), and the stdout lines TR/dashboard.py
parses (TR/dashboard.py:338-360)."""
import os
import re
import subprocess

import numpy as np
import pytest

from gpu_util import need_gpu, rel_l2
from oracle import ckpt as ock
from oracle import data as od
from oracle import model as om

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "neural-engine_amd", "train_tiny")
RE_STEP = re.compile(r"step\s+(\d+)\s+loss=([\d.]+)(?:\s+lr=([\d.e+-]+))?(?:\s+([\d.]+)ms/step)?")


@pytest.fixture(autouse=True)
def _gpu():
    need_gpu()
    if not os.path.exists(CLI):
        pytest.fail(f"{CLI} is not built (make -C neural-engine_amd train MODEL=tiny)")


def tiny_cfg():
    # the CLI's semantics: residual scale 1/sqrt(2L), RoPE base 1e4, no QK-norm
    return om.tiny(res_alpha=om.train_alpha(2), rope_theta=1e4, qk_norm=False)


def run_cli(args, cwd):
    print("[cli]", " ".join(args), flush=True)
    r = subprocess.run([CLI] + args, cwd=cwd, capture_output=True, text=True, timeout=120)
    print(r.stdout[-3000:], flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    return r.stdout


def write_data(path, cfg, n=5000, seed=5, n_ids=None):
    data = np.random.default_rng(seed).integers(0, n_ids or cfg.vocab, n).astype(np.uint16)
    data.tofile(path)
    return data


@pytest.mark.parametrize("compact", [True, False])
def test_resume_one_step_matches_oracle(tmp_path, compact):
    """--resume from an oracle-written checkpoint at step 99 of 100: one sampled window,
    one AdamW step at the cosine LR of step 99, checkpoint saved at step 100.  The data use
    300 of the 512 ids: by default the classifier is compacted to them (TD/train.m:286-292);
    --full-vocab keeps the full softmax."""
    cfg = tiny_cfg()
    P = om.init_params(cfg, seed=0, std=0.02)
    M = {k: np.zeros_like(v) for k, v in P.items()}
    V = {k: np.zeros_like(v) for k, v in P.items()}
    ck = str(tmp_path / "ck.bin")
    ock.write(ck, cfg, P, M, V, step=99, total_steps=100, lr=3e-4, loss=0.0)
    data = write_data(tmp_path / "data.bin", cfg, n_ids=300)
    ids = om.vocab_map_build(data, cfg.vocab) if compact else None
    out = run_cli(["--resume", "--ckpt", ck, "--data", str(tmp_path / "data.bin"), "--accum", "1",
                   "--warmup", "1", "--lr", "3e-4"] + ([] if compact else ["--full-vocab"]), tmp_path)
    assert "[RESUMED step 99, loss=0.0000]" in out
    if compact:
        assert f"Vocab compaction: {cfg.vocab} \u2192 {len(ids)} active tokens" in out
    else:
        assert f"Vocab: full {cfg.vocab}-way softmax" in out
    m = RE_STEP.search(out)
    assert m and int(m.group(1)) == 99
    assert "[ckpt saved" in out

    (pos,) = od.window_positions(len(data), cfg.seq, 99, 1)
    tok = data[pos:pos + cfg.seq + 1].astype(np.int32)[None]
    lo, cache = om.forward(cfg, P, tok, loss_scale=256.0, vocab_ids=ids)
    G = om.backward(cfg, P, cache)
    lr = om.lr_at(99, 3e-4, 1, 100)
    Po = {k: v.copy() for k, v in P.items()}
    om.optimizer_step(Po, G, M, V, 1, lr, grad_scale=1 / 256, clip=1.0)

    assert abs(float(m.group(2)) - lo) <= 1e-3 * lo + 1e-4, (m.group(2), lo)
    h, Pg, Mg, Vg = ock.read(ck)
    assert h["step"] == 100 and h["adam_t"] == 1 and h["total_steps"] == 100
    assert abs(h["lr"] - lr) <= 1e-6 * lr
    assert abs(h["loss"] - lo) <= 1e-3 * lo
    for n in P:
        # m = (1 - b1) * clipped grad: the gradient parity bar
        assert rel_l2(Mg[n], M[n]) <= 1e-2, n
        # one AdamW step at t=1 moves each weight by lr * (g/|g| + wd*w): the two updates
        # agree wherever the gradient signs agree (all but near-zero gradients), and never
        # differ by more than 2*lr
        d = np.abs(Pg[n] - Po[n])
        assert d.max() <= 2.0 * lr * 1.01, n
        assert float(np.mean(d > 0.5 * lr)) <= 0.05, n


def test_scratch_init_and_dashboard_lines(tmp_path):
    """--scratch: srand48(42) uniform init of TD/train.m:236-251 (kept exact by lr 0), 100
    accumulated micro-steps, one update, checkpoint at step 100; stdout in the reference's
    format."""
    cfg = tiny_cfg()
    write_data(tmp_path / "data.bin", cfg)
    ck = str(tmp_path / "ck.bin")
    out = run_cli(["--scratch", "--steps", "100", "--accum", "100", "--lr", "0", "--ckpt", ck,
                   "--data", str(tmp_path / "data.bin")], tmp_path)
    assert re.search(r"ANE Dynamic Training: Tiny-GQA \(2 layers", out)
    assert re.search(r"dim=128 q_dim=256 kv_dim=128 hd=64 hidden=256 seq=64 vocab=512", out)
    assert re.search(r"Params: [\d.]+M \(transformer [\d.]+M \+ embed [\d.]+M\)", out)
    assert re.search(r"Accum 100.*LR=0", out)
    steps = [int(m.group(1)) for m in RE_STEP.finditer(out)]
    assert steps == list(range(0, 100, 10))
    losses = [float(m.group(2)) for m in RE_STEP.finditer(out)]
    assert all(abs(l - np.log(cfg.vocab)) < 0.5 for l in losses)
    assert "[ckpt saved" in out and "=== Efficiency Report ===" in out
    h, Pg, Mg, Vg = ock.read(ck)
    assert h["step"] == 100 and h["adam_t"] == 1
    want = od.scratch_init(cfg)
    for n in want:
        np.testing.assert_array_equal(Pg[n], want[n], err_msg=n)
    assert all(np.abs(Mg[n]).max() > 0 for n in want if not om.is_gain(n))


def test_resume_continues_the_run(tmp_path):
    """--resume picks up the step, Adam counter and schedule of a --scratch run's checkpoint
    (total_steps comes from the header, TD/train.m:146) and keeps training from there."""
    cfg = tiny_cfg()
    write_data(tmp_path / "data.bin", cfg)
    d = str(tmp_path / "data.bin")
    a, b = str(tmp_path / "a.bin"), str(tmp_path / "b.bin")
    run_cli(["--scratch", "--steps", "100", "--accum", "1", "--ckpt", a, "--data", d, "--warmup", "10"], tmp_path)
    ha, Pa, _, _ = ock.read(a)
    assert ha["step"] == 100 and ha["adam_t"] == 100 and ha["total_steps"] == 100
    raw = bytearray(open(a, "rb").read())
    np.frombuffer(raw, np.int32, 1, 12)[:] = 130   # total_steps field
    np.frombuffer(raw, np.float32, 1, 44)[:] = 99.0  # loss field: the next save is a new best
    open(b, "wb").write(bytes(raw))
    out = run_cli(["--resume", "--ckpt", b, "--data", d, "--accum", "10", "--warmup", "10"], tmp_path)
    assert "[RESUMED step 100, loss=99.0000]" in out
    steps = [int(m.group(1)) for m in RE_STEP.finditer(out)]
    assert steps == [100, 110, 120]
    hb, Pb, Mb, Vb = ock.read(b)
    # the last step (129) updates and, not being a multiple of 100, does not save: the file
    # still holds step 100
    assert hb["step"] == 100
    assert out.count("[adam] step") == 3
