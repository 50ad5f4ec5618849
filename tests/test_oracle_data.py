"""The oracle's restatement of the train CLI's data sampling and --scratch init, pinned
against the C library's own srand48/drand48 (the generator TD/train.m:246-252, 389-398
calls)."""
import ctypes
import ctypes.util

import numpy as np
import pytest

from oracle import data as od
from oracle import model as om


@pytest.fixture(scope="module")
def libc():
    c = ctypes.CDLL(ctypes.util.find_library("c"))
    c.drand48.restype = ctypes.c_double
    c.srand48.argtypes = [ctypes.c_long]
    return c


@pytest.mark.parametrize("seed", [42, 42 + 99, 0, 123456789])
def test_drand48_matches_libc(libc, seed):
    libc.srand48(seed)
    r = od.Drand48(seed)
    for _ in range(2000):
        assert libc.drand48() == r()


def test_window_positions_match_libc(libc):
    n, seq = 100_000, 256
    libc.srand48(42 + 7)
    want = [int(libc.drand48() * (n - seq - 1)) for _ in range(50)]
    assert od.window_positions(n, seq, 7, 50) == want
    assert all(0 <= p <= n - seq - 1 for p in want)


def test_scratch_init_scales_and_order():
    cfg = om.tiny()
    P = od.scratch_init(cfg)
    for name, shp in om.tensor_list(cfg):
        assert P[name].shape == tuple(shp) and P[name].dtype == np.float32
    # uniform +-scale: the extreme values approach the scale, the mean is near 0
    L = cfg.n_layers
    res = 1 / np.sqrt(2 * L)
    for t, sc in (("Wq", 1 / np.sqrt(cfg.dim)), ("Wo", res / np.sqrt(cfg.q_dim)), ("W1", 1 / np.sqrt(cfg.hidden))):
        a = P[f"layers.0.{t}"]
        assert np.abs(a).max() <= sc * (1 + 1e-6) and np.abs(a).max() > 0.99 * sc
        assert abs(float(a.mean())) < 0.02 * sc
    assert np.abs(P["embed"]).max() <= 0.02 * (1 + 1e-6)
    # the first draw belongs to layer 0's Wq[0, 0]
    r = od.Drand48(42)
    assert P["layers.0.Wq"][0, 0] == np.float32(1 / np.sqrt(np.float32(cfg.dim))) * np.float32(2 * r() - 1)
    assert (P["layers.1.rms_att"] == 1).all() and (P["rms_final"] == 1).all()
