"""Pins the oracle's token loop and checkpoint layout against vectors written by the
reference's own numpy decoder (tests/golden/make_generate_vectors.py)."""
import json
import os

import numpy as np
import pytest

from oracle import model as om

GOLD = os.path.join(os.path.dirname(__file__), "golden", "generate_tiny.json")


@pytest.fixture(scope="module")
def gold():
    with open(GOLD) as f:
        g = json.load(f)
    cfg = om.Config(**g["config"], qk_norm=False, res_alpha=1.0)
    P = om.init_params(cfg, seed=g["weight_seed"], std=g["weight_std"])
    return g, cfg, P


def test_checkpoint_probes_match_reference_reader(gold):
    g, cfg, P = gold
    for name, ix, val in g["probes"]:
        assert float(P[name][tuple(ix)]) == val, name


@pytest.mark.parametrize("stream", ["greedy", "t08_p09_s11", "t06_p10_s3"])
def test_token_stream_matches_reference_generate(gold, stream):
    g, cfg, P = gold
    s = g["streams"][stream]
    prompt = np.array([g["prompt"]], np.int32)
    u = None
    if s["seed"] is not None:
        u = np.random.RandomState(s["seed"]).random_sample((1, g["n_new"]))
    toks = om.decode(cfg, P, prompt, g["n_new"], temperature=s["temp"], top_p=s["top_p"], uniforms=u)
    assert toks[0].tolist() == s["tokens"]
