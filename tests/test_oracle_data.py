"""The oracle's restatement of the train CLI's data sampling and --scratch init, pinned
against the C library's own srand48/drand48 (the generator TD/train.m:246-252, 389-398
calls)."""
import ctypes
import ctypes.util
import math
import struct

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
    assert (P["layers.1.rms_att"] == 1).all() and (P["rms_final"] == 1).all()


def _f32(x: float) -> float:
    return struct.unpack("f", struct.pack("f", x))[0]


def test_scratch_init_bit_exact_against_libc(libc):
    """Every element of the --scratch init against an independent restatement of
    TD/train.m:240-251: the C library's own srand48(42)/drand48 stream, the float scales
    1.0f/sqrtf(n) (a double sqrt and division rounded to float are the correctly rounded
    float results), and `scale*(2*drand48()-1)` formed in IEEE double by Python and rounded
    once to float.  Three layers make res_scale = 1/sqrt(6) a non-power of two, so the Wo and
    W2 products are exercised too.  A draw rounded to float before a float multiply (the
    plausible mistake) differs in a quarter of the elements of a non-power-of-two scale."""
    cfg = om.tiny(n_layers=3)
    P = od.scratch_init(cfg)
    D, H, Q, KV, L = cfg.dim, cfg.hidden, cfg.q_dim, cfg.kv_dim, cfg.n_layers
    inv_sqrt = lambda n: _f32(1.0 / _f32(math.sqrt(float(n))))
    s_d, s_qd, s_h = inv_sqrt(D), inv_sqrt(Q), inv_sqrt(H)
    res = _f32(1.0 / _f32(math.sqrt(_f32(2.0 * L))))
    scales = {"Wq": s_d, "Wk": s_d, "Wv": s_d, "Wo": _f32(s_qd * res), "W1": s_h,
              "W2": _f32(s_d * res), "W3": s_h}
    libc.srand48(42)
    shapes = om.layer_shapes(cfg)
    differs = {}

    def expect(n, sc):
        u = np.array([2.0 * libc.drand48() - 1.0 for _ in range(n)])
        want = np.array([_f32(sc * x) for x in u], np.float32)
        wrong = (np.float32(sc) * u.astype(np.float32)).astype(np.float32)
        return want, float(np.mean(wrong != want))

    for l in range(L):
        for t in om.LAYER_TENSORS[:7]:
            want, differs[t] = expect(int(np.prod(shapes[t])), scales[t])
            np.testing.assert_array_equal(P[f"layers.{l}.{t}"].ravel(), want, err_msg=f"layer {l} {t}")
    want, differs["embed"] = expect(cfg.vocab * D, _f32(0.02))
    np.testing.assert_array_equal(P["embed"].ravel(), want)
    # the scales that are not powers of two tell the two roundings apart
    assert differs["Wq"] > 0.05 and differs["Wo"] > 0.05 and differs["embed"] > 0.05, differs
