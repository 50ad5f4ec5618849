"""The decode command line (neural-engine_amd/generate.py, the counterpart of the reference's
TD/tools/generate.py): checkpoint header parsing and numpy's sampling draw on the CPU; the
token streams it prints against the oracle's decode on the same checkpoint on the GPU."""
import os
import re
import subprocess
import sys

import numpy as np
import pytest

from oracle import ckpt as ock
from oracle import model as om

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GEN = os.path.join(ROOT, "neural-engine_amd", "generate.py")
sys.path.insert(0, os.path.join(ROOT, "neural-engine_amd"))

import generate  # noqa: E402
import ne  # noqa: E402


def _ckpt(tmp_path, qk_norm, seed=0):
    cfg = om.tiny(qk_norm=qk_norm, rope_theta=1e6 if qk_norm else 1e4, res_alpha=1.0)
    P = om.init_params(cfg, seed=seed, std=0.05)
    P = {k: v.astype(np.float16).astype(np.float32) for k, v in P.items()}   # fp16-exact weights
    Z = {k: np.zeros_like(v) for k, v in P.items()}
    path = str(tmp_path / f"ck_{int(qk_norm)}.bin")
    ock.write(path, cfg, P, Z, Z, step=7, total_steps=9, adam_t=3)
    return cfg, P, path


@pytest.mark.parametrize("qk_norm", [False, True])
def test_checkpoint_header(tmp_path, qk_norm):
    cfg, _, path = _ckpt(tmp_path, qk_norm)
    h = ne.read_ckpt_header(path)
    assert (h["dim"], h["hidden"], h["n_heads"], h["kv_heads"], h["head_dim"], h["n_layers"], h["vocab"]) == \
        (cfg.dim, cfg.hidden, cfg.n_heads, cfg.kv_heads, cfg.head_dim, cfg.n_layers, cfg.vocab)
    assert h["qk_norm"] == qk_norm and h["step"] == 7 and h["adam_t"] == 3
    with open(path, "ab") as f:
        f.write(b"\0\0\0\0")
    with pytest.raises(ne.NEError):
        ne.read_ckpt_header(path)


def test_sampling_draws_are_numpys_choice():
    """np.random.seed(s) then np.random.choice(V, p=probs) per token (generate.py:215, 249)
    consumes one random_sample per token and inverts the CDF in vocabulary order."""
    rng = np.random.default_rng(0)
    probs = [rng.dirichlet(np.ones(50) * 0.3) for _ in range(20)]
    np.random.seed(11)
    want = [int(np.random.choice(50, p=p)) for p in probs]
    u = generate.sampling_uniforms(20, 11)
    got = [int(np.searchsorted(np.cumsum(p), x, side="right")) for p, x in zip(probs, u)]
    assert got == want


def test_cli_arguments_follow_generate_py():
    a = generate.parse_args(["ck.bin"])
    assert (a.tokens, a.temp, a.top_p, a.seed, a.prompt) == (100, 0.8, 0.9, None, "Once upon a time")
    a = generate.parse_args(["ck.bin", "-n", "5", "-t", "0", "--top-p", "1", "--seed", "3", "-p", "hi"])
    assert (a.tokens, a.temp, a.top_p, a.seed, a.prompt) == (5, 0.0, 1.0, 3, "hi")


def _run(args):
    r = subprocess.run([sys.executable, GEN] + args, capture_output=True, text=True, timeout=300)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0
    body = r.stdout.split("---\n")[1]
    m = re.search(r"Generated (\d+) tokens", r.stdout)
    return [int(x) for x in body.split()], int(m.group(1)), r.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("qk_norm", [False, True])
def test_cli_streams_match_oracle(tmp_path, qk_norm):
    if not __import__("torch").cuda.is_available():
        pytest.skip("no GPU")
    cfg, P, path = _ckpt(tmp_path, qk_norm)
    theta = ["--rope-theta", "1e6"] if qk_norm else []
    prompt = [5, 17, 99, 3, 200]
    p = np.array([prompt], np.int32)
    # greedy
    got, n, out = _run([path, "--prompt-ids", "5,17,99,3,200", "-n", "40", "-t", "0"] + theta)
    want = om.decode(cfg, P, p, 40)[0].tolist()
    assert got == want and n == 40
    assert "Prompt (5 tokens): 5 17 99 3 200" in out and "Generating 40 tokens (temp=0.0, top_p=0.9)" in out
    # temperature + top-p with a seed: the same draws as generate.py's numpy sampler
    got, n, _ = _run([path, "--prompt-ids", "5,17,99,3,200", "-n", "40", "-t", "0.8", "--top-p", "0.9",
                      "--seed", "11"] + theta)
    want_s = om.decode(cfg, P, p, 40, temperature=0.8, top_p=0.9,
                       uniforms=generate.sampling_uniforms(40, 11)[None])[0].tolist()
    assert got == want_s
    # EOS stop: the stream ends with the first occurrence of the stop id
    eos = want[6]
    got, n, _ = _run([path, "--prompt-ids", "5,17,99,3,200", "-n", "40", "-t", "0", "--eos", str(eos)] + theta)
    k = want.index(eos) + 1
    assert got == want[:k] and n == k


@pytest.mark.gpu
def test_hf_directory_to_tokens(tmp_path):
    """A local HF-format model directory -> convert_hf.py -> generate.py on the GPU: the
    greedy stream of the oracle on the same (QK-norm, fp16-exact) weights."""
    if not __import__("torch").cuda.is_available():
        pytest.skip("no GPU")
    import json
    from safetensors.numpy import save_file
    import convert_hf
    cfg, P, _ = _ckpt(tmp_path, True)
    hf = {"Wq": "self_attn.q_proj", "Wk": "self_attn.k_proj", "Wv": "self_attn.v_proj", "Wo": "self_attn.o_proj",
          "W1": "mlp.gate_proj", "W2": "mlp.down_proj", "W3": "mlp.up_proj", "rms_att": "input_layernorm",
          "rms_ffn": "post_attention_layernorm", "q_norm": "self_attn.q_norm", "k_norm": "self_attn.k_norm"}
    t = {"model.embed_tokens.weight": P["embed"], "model.norm.weight": P["rms_final"]}
    for n, a in P.items():
        if n.startswith("layers."):
            _, l, name = n.split(".")
            t[f"model.layers.{l}.{hf[name]}.weight"] = a
    d = tmp_path / "hf"
    d.mkdir()
    save_file(t, str(d / "model.safetensors"))
    (d / "config.json").write_text(json.dumps(dict(
        model_type="qwen3", hidden_size=cfg.dim, intermediate_size=cfg.hidden, num_attention_heads=cfg.n_heads,
        num_key_value_heads=cfg.kv_heads, head_dim=cfg.head_dim, num_hidden_layers=cfg.n_layers,
        vocab_size=cfg.vocab)))
    ck = str(tmp_path / "converted.bin")
    assert convert_hf.main([str(d), "-o", ck]) == 0
    got, n, _ = _run([ck, "--prompt-ids", "9,8,7", "-n", "32", "-t", "0", "--rope-theta", "1e6"])
    assert got == om.decode(cfg, P, np.array([[9, 8, 7]], np.int32), 32)[0].tolist()
