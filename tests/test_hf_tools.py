"""Offline HF convert/export (neural-engine_amd/convert_hf.py, export_hf.py; the counterparts
of TD/tools/convert_hf.py and export_hf.py): a synthetic local HF model directory ->
v4 checkpoint, checked with the oracle's independent checkpoint reader, and back."""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

from oracle import ckpt as ock
from oracle import model as om

safetensors = pytest.importorskip("safetensors.numpy")
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "neural-engine_amd")
sys.path.insert(0, PKG)

import convert_hf  # noqa: E402
import export_hf  # noqa: E402

CFG = dict(model_type="qwen3", hidden_size=64, intermediate_size=128, num_attention_heads=4,
           num_key_value_heads=2, head_dim=16, num_hidden_layers=2, vocab_size=97)
HF = {"Wq": "self_attn.q_proj.weight", "Wk": "self_attn.k_proj.weight", "Wv": "self_attn.v_proj.weight",
      "Wo": "self_attn.o_proj.weight", "W1": "mlp.gate_proj.weight", "W2": "mlp.down_proj.weight",
      "W3": "mlp.up_proj.weight", "rms_att": "input_layernorm.weight",
      "rms_ffn": "post_attention_layernorm.weight"}


def _hf_dir(tmp_path, lm_head=False, qk_norm=True):
    D, H, hd, L, V = 64, 128, 16, 2, 97
    shapes = {"Wq": (64, D), "Wk": (32, D), "Wv": (32, D), "Wo": (D, 64), "W1": (H, D), "W2": (D, H),
              "W3": (H, D), "rms_att": (D,), "rms_ffn": (D,)}
    rng = np.random.default_rng(0)
    t = {}
    for l in range(L):
        for ours, hf in HF.items():
            t[f"model.layers.{l}.{hf}"] = rng.standard_normal(shapes[ours]).astype(np.float32)
        if qk_norm:
            t[f"model.layers.{l}.self_attn.q_norm.weight"] = rng.standard_normal(hd).astype(np.float32)
            t[f"model.layers.{l}.self_attn.k_norm.weight"] = rng.standard_normal(hd).astype(np.float32)
    t["model.norm.weight"] = rng.standard_normal(D).astype(np.float32)
    t["model.embed_tokens.weight"] = rng.standard_normal((V, D)).astype(np.float32)
    if lm_head:
        t["lm_head.weight"] = rng.standard_normal((V, D)).astype(np.float32)
    d = tmp_path / "hf"
    d.mkdir()
    # two shards, as larger models ship
    keys = sorted(t)
    safetensors.save_file({k: t[k] for k in keys[::2]}, str(d / "model-00001-of-00002.safetensors"))
    safetensors.save_file({k: t[k] for k in keys[1::2]}, str(d / "model-00002-of-00002.safetensors"))
    (d / "config.json").write_text(json.dumps(CFG))
    (d / "tokenizer.json").write_text("{}")
    return str(d), t


@pytest.mark.parametrize("qk_norm", [True, False])
def test_convert_matches_source_tensors(tmp_path, qk_norm):
    d, t = _hf_dir(tmp_path)
    out = str(tmp_path / "ck.bin")
    args = [d, "-o", out, "--steps", "1234"] + ([] if qk_norm else ["--no-qk-norm"])
    assert convert_hf.main(args) == 0
    h, P, M, V = ock.read(out)
    assert (h["step"], h["total_steps"], h["seq"], h["n_layers"], h["vocab"], h["dim"], h["hidden"], h["n_heads"],
            h["kv_heads"], h["head_dim"], h["q_dim"]) == (0, 1234, 256, 2, 97, 64, 128, 4, 2, 16, 64)
    assert abs(h["lr"] - 3e-4) < 1e-9
    for l in range(2):
        for ours, hf in HF.items():
            np.testing.assert_array_equal(P[f"layers.{l}.{ours}"], t[f"model.layers.{l}.{hf}"])
    np.testing.assert_array_equal(P["rms_final"], t["model.norm.weight"])
    np.testing.assert_array_equal(P["embed"], t["model.embed_tokens.weight"])
    assert all(np.abs(M[n]).max() == 0 and np.abs(V[n]).max() == 0 for n in P)
    cfg = om.Config(dim=64, hidden=128, n_heads=4, kv_heads=2, head_dim=16, n_layers=2, vocab=97, seq=256,
                    qk_norm=qk_norm)
    assert os.path.getsize(out) == ock.expected_size(cfg)
    if qk_norm:
        for l in range(2):
            np.testing.assert_array_equal(P[f"layers.{l}.q_norm"], t[f"model.layers.{l}.self_attn.q_norm.weight"])
            np.testing.assert_array_equal(P[f"layers.{l}.k_norm"], t[f"model.layers.{l}.self_attn.k_norm.weight"])
    else:
        assert "layers.0.q_norm" not in P


def test_convert_prefers_lm_head_as_the_reference(tmp_path):
    d, t = _hf_dir(tmp_path, lm_head=True)
    out = str(tmp_path / "ck.bin")
    convert_hf.main([d, "-o", out])
    _, P, _, _ = ock.read(out)
    np.testing.assert_array_equal(P["embed"], t["lm_head.weight"])


def test_export_round_trip(tmp_path):
    d, t = _hf_dir(tmp_path)
    ck = str(tmp_path / "ck.bin")
    convert_hf.main([d, "-o", ck])
    out = str(tmp_path / "exported")
    assert export_hf.main([ck, "-o", out, "-m", d]) == 0
    got = safetensors.load_file(os.path.join(out, "model.safetensors"))
    assert set(got) == set(t)
    for k in t:
        np.testing.assert_array_equal(got[k], t[k], err_msg=k)
    assert json.load(open(os.path.join(out, "config.json"))) == CFG     # copied from the source model
    assert os.path.exists(os.path.join(out, "tokenizer.json"))
    # without the source model: the minimal config of export_hf.py:140-158
    out2 = str(tmp_path / "exported2")
    export_hf.main([ck, "-o", out2])
    c = json.load(open(os.path.join(out2, "config.json")))
    assert (c["hidden_size"], c["num_key_value_heads"], c["head_dim"], c["vocab_size"], c["tie_word_embeddings"]) == \
        (64, 2, 16, 97, True)
    # export -> convert reproduces the checkpoint bytes
    ck2 = str(tmp_path / "ck2.bin")
    convert_hf.main([out, "-o", ck2, "--steps", "10000"])
    assert open(ck, "rb").read() == open(ck2, "rb").read()


def test_command_lines_run(tmp_path):
    d, _ = _hf_dir(tmp_path, qk_norm=False)
    r = subprocess.run([sys.executable, os.path.join(PKG, "convert_hf.py"), d], cwd=tmp_path, capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert os.path.exists(tmp_path / "ane_qwen3_dyn_ckpt.bin")          # the reference's default name
    r = subprocess.run([sys.executable, os.path.join(PKG, "export_hf.py"), "ane_qwen3_dyn_ckpt.bin", "-o", "x"],
                       cwd=tmp_path, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert os.path.exists(tmp_path / "x" / "model.safetensors")
