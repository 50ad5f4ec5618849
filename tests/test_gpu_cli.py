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


def test_resume_reference_norm_formula(tmp_path):
    """--rmsnorm-bwd-ref: a checkpoint with trained (non-unit) gains, one step; the first Adam
    moment (the clipped gradient) follows the oracle's reference-formula backward and not the
    exact one."""
    cfg = tiny_cfg()
    P = om.init_params(cfg, seed=0, std=0.02)
    rng = np.random.default_rng(3)
    for n in P:
        if om.is_gain(n):
            P[n] = (1 + 0.5 * rng.standard_normal(P[n].shape)).astype(np.float32)
    Z = {k: np.zeros_like(v) for k, v in P.items()}
    ck = str(tmp_path / "ck.bin")
    ock.write(ck, cfg, P, Z, Z, step=99, total_steps=100, lr=3e-4, loss=0.0)
    data = write_data(tmp_path / "data.bin", cfg, n_ids=300)
    ids = om.vocab_map_build(data, cfg.vocab)
    run_cli(["--resume", "--ckpt", ck, "--data", str(tmp_path / "data.bin"), "--accum", "1", "--warmup", "1",
             "--lr", "3e-4", "--rmsnorm-bwd-ref"], tmp_path)
    (pos,) = od.window_positions(len(data), cfg.seq, 99, 1)
    tok = data[pos:pos + cfg.seq + 1].astype(np.int32)[None]
    _, cache = om.forward(cfg, P, tok, loss_scale=256.0, vocab_ids=ids)
    lr = om.lr_at(99, 3e-4, 1, 100)
    Mo = {}
    for ref in (True, False):
        M = {k: np.zeros_like(v) for k, v in P.items()}
        V = {k: np.zeros_like(v) for k, v in P.items()}
        om.optimizer_step({k: v.copy() for k, v in P.items()}, om.backward(cfg, P, cache, norm_bwd_ref=ref), M, V,
                          1, lr, grad_scale=1 / 256, clip=1.0)
        Mo[ref] = M
    _, _, Mg, _ = ock.read(ck)
    for n in P:
        assert rel_l2(Mg[n], Mo[True][n]) <= 1e-2, n
    assert max(rel_l2(Mg[n], Mo[False][n]) for n in P) > 5e-2


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
    # the step line's ranges and the grad-norm line's groups (TD/train.m:776, 828)
    full = re.findall(r"step (\d+)\s+loss=\S+\s+lr=\S+\s+\S+ms/step\s+x\[(\S+),(\S+)\] dy\[(\S+),(\S+)\]", out)
    assert [int(f[0]) for f in full] == steps
    for f in full:
        xmn, xmx, dmn, dmx = map(float, f[1:])
        assert xmn < 0 < xmx and dmn < 0 < dmx
    # TD/train.m:302 (TR/dashboard.py RE_COMPILED) and the per-phase timing line of
    # TD/train.m:766, printed with each step line: phases in ms, non-negative, within the step
    assert re.search(r"Compiled (\d+) kernels in (\d+)ms", out)
    tl = re.findall(r"timing: ane_fwd=(\S+) io_fwd=(\S+) rms=(\S+) ane_bwd=(\S+) io_bwd=(\S+) rms_bwd=(\S+) "
                    r"cls=(\S+) dw=(\S+) dwait=(\S+) resid=(\S+) gqa=(\S+) rope=(\S+) \[gap=(\S+)\]", out)
    assert len(tl) == len(steps)
    for t in tl:
        v = list(map(float, t))
        assert min(v[:12]) >= 0 and v[0] > 0 and v[3] > 0, t   # %.1f ms: the tiny classifier can read 0.0
    gl = re.findall(r"grad_norm=(\S+)\s+attn=(\S+) ffn=(\S+) embed=(\S+)", out)
    assert len(gl) == 1
    tot, att, ffn, emb = map(float, gl[0])
    assert att > 0 and ffn > 0 and emb > 0 and att ** 2 + ffn ** 2 + emb ** 2 <= tot ** 2 * (1 + 1e-3)
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


@pytest.mark.timeout(300)
def test_seq512_model_header(tmp_path):
    """The SEQ=512 build of Qwen3-0.6B (TD/models/qwen3_06b_seq512.h): the banner carries the
    reference's model name, which TR/dashboard.py's RE_MODEL_NAME reads, and seq=512; two
    steps from --scratch with the classifier over the data's ids run at the loss of an
    untrained model (about ln of the compact vocabulary)."""
    exe = os.path.join(ROOT, "neural-engine_amd", "train_qwen3_06b_seq512")
    data = np.random.default_rng(7).integers(0, 60000, 20000).astype(np.uint16)
    data.tofile(tmp_path / "d.bin")
    cv = len(np.unique(data))
    r = subprocess.run([exe, "--scratch", "--steps", "2", "--accum", "1", "--data", str(tmp_path / "d.bin"),
                        "--ckpt", str(tmp_path / "c.bin")], cwd=tmp_path, capture_output=True, text=True,
                       timeout=280)
    print(r.stdout[-2000:], flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    m = re.search(r"ANE Dynamic Training: (.+?) \((\d+) layers", r.stdout)  # TR/dashboard.py RE_MODEL_NAME
    assert m and m.group(1) == "Qwen3-0.6B-seq512" and m.group(2) == "28"
    assert re.search(r"hd=128 hidden=3072 seq=512 vocab=151936", r.stdout)
    assert f"{cv} active tokens" in r.stdout
    loss = [float(x.group(2)) for x in RE_STEP.finditer(r.stdout)]
    assert len(loss) == 1 and abs(loss[0] - np.log(cv)) < 1.0, loss
