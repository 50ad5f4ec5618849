"""CPU-side checks of the C-ABI library: it loads, exports every symbol ne.h declares,
rejects bad configurations without a GPU, and the tensor naming matches the oracle."""
import ctypes
import os
import re

import pytest

import ne
from oracle import model as om

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    src = open(os.path.join(ROOT, "include", "ne.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(ne_[a-z0-9_]+)\s*\(", src)))


def test_header_symbols_listed_in_binding():
    assert header_symbols() == sorted(ne.EXPORTS)


def test_library_exports_every_header_symbol():
    h = ctypes.CDLL(ne.LIB_PATH)
    for name in header_symbols():
        assert hasattr(h, name), name
    ne.lib()  # signatures bind


def test_invalid_config_rejected_without_device():
    cfg = ne.Config(dim=100, hidden=256, n_heads=4, kv_heads=2, head_dim=64, n_layers=1, vocab=512,
                    seq=64, batch=1, qk_norm=0, rope_theta=1e4, res_alpha=1.0, norm_eps=1e-5,
                    decode_batch=0, decode_ctx=0, dtype=ne.NE_FP16)
    assert not ne.lib().ne_create(ctypes.byref(cfg))
    assert b"multiples of 64" in ne.lib().ne_last_error()
    cfg.dim, cfg.head_dim = 128, 96
    assert not ne.lib().ne_create(ctypes.byref(cfg))
    assert b"head_dim" in ne.lib().ne_last_error()
    cfg.head_dim, cfg.dtype = 64, 7
    assert not ne.lib().ne_create(ctypes.byref(cfg))
    assert b"dtype" in ne.lib().ne_last_error()


def test_kernel_entry_points_validate_shapes_before_launch():
    # a GEMM with M not a multiple of 64 must be refused on the host
    rc = ne.lib().ne_k_gemm(1, 0, 0, 65, 64, 64, None, 64, None, 64, None, 64, None, 0, 1.0, None)
    assert rc == -1 and b"multiples of 64" in ne.lib().ne_last_error()
    rc = ne.lib().ne_k_gemm(5, 0, 0, 64, 64, 64, None, 64, None, 64, None, 64, None, 0, 1.0, None)
    assert rc == -1 and b"16-bit format" in ne.lib().ne_last_error()
    rc = ne.lib().ne_k_attn_fwd(1, None, 64, None, 64, None, 64, None, 64, None, 1, 100, 4, 2, 64, 0.125, None)
    assert rc == -1 and b"multiple of 64" in ne.lib().ne_last_error()
    rc = ne.lib().ne_k_adam(1, None, None, None, None, None, 8, 8, 1e-3, 0.9, 0.95, 1e-8, 0.1, 0, None, 1, None)
    assert rc == -1


def test_swiglu_forward_epilogue_arguments_checked_on_host():
    """The W1|W3 GEMM's SwiGLU-forward epilogue (epi 7) needs both outputs and layout 0; the
    checks run before any launch."""
    L = ne.lib()
    rc = L.ne_k_gemm(ne.NE_FP16, 0, 7, 64, 128, 64, None, 64, None, 64, None, 128, None, 64, 1.0, None)
    assert rc == -1 and b"SwiGLU forward" in L.ne_last_error()
    fake = ctypes.c_void_p(256)  # never dereferenced: the layout is refused before a launch
    rc = L.ne_k_gemm(ne.NE_FP16, 2, 7, 64, 128, 64, fake, 64, fake, 128, fake, 128, fake, 64, 1.0, None)
    assert rc == -1 and b"layout 0" in L.ne_last_error()


def test_wgrad_group_refuses_shapes_off_its_path():
    """The grouped weight-gradient GEMM takes only the long-step shapes (M, N multiples of 256,
    K >= 8192, at least 192 tiles); anything else is refused on the host, before a launch."""
    L = ne.lib()
    n = 2
    arr = lambda ct, xs: (ct * n)(*xs)
    nul = arr(ctypes.c_void_p, [None, None])
    lds = arr(ctypes.c_int64, [1024, 1024])
    for M, N, K in [((4096, 6144), (1024, 1024), 4096), ((4096, 1024), (1024, 1024), 8192),
                    ((4096, 6144), (1000, 1024), 8192)]:
        rc = L.ne_k_gemm_wgrad_group(ne.NE_FP16, n, arr(ctypes.c_int, M), arr(ctypes.c_int, N), K, nul, lds, nul,
                                     lds, nul, 0, 1.0, None)
        assert rc == -1 and b"grouped path" in L.ne_last_error(), (M, N, K)
    rc = L.ne_k_gemm_wgrad_group(ne.NE_FP16, 5, None, None, 8192, None, None, None, None, None, 0, 1.0, None)
    assert rc == -1


@pytest.mark.parametrize("qk", [False, True])
def test_tensor_names_match_oracle_order(qk):
    cfg = om.tiny(qk_norm=qk)
    assert ne.tensor_names(cfg.n_layers, qk) == [n for n, _ in om.tensor_list(cfg)]


def test_attn_bwd_noalloc_rejects_oversized_inputs_without_device():
    """The allocation-free attention backward checks its fixed scratch bound (B*S*NH <= 2^20)
    before touching a device."""
    L = ne.lib()
    rc = L.ne_k_attn_bwd_noalloc(ne.NE_FP16, None, 0, None, 0, None, 0, None, 0, None, None, 0, None, 0, None, 0,
                                 None, 0, 64, 2048, 16, 8, 128, 1.0, None)
    assert rc == -1 and b"exceeds the fixed scratch" in L.ne_last_error()
    rc = L.ne_k_attn_bwd_noalloc(ne.NE_FP16, None, 0, None, 0, None, 0, None, 0, None, None, 0, None, 0, None, 0,
                                 None, 0, 0, 2048, 16, 8, 128, 1.0, None)
    assert rc == -1 and b"must be positive" in L.ne_last_error()


def test_mt19937_uniforms_match_numpy_random_state():
    """ne_mt19937_uniforms (the draws of ne_decode_seeded) against numpy's legacy
    RandomState(seed).random_sample, bit for bit, across the 624-word regeneration; seeds of
    2^32 and above are rejected as numpy rejects them."""
    import numpy as np
    for seed in (0, 1, 42, 1234, 2**32 - 1):
        want = np.random.RandomState(seed).random_sample(1500)
        got = ne.mt19937_uniforms(seed, 1500)
        np.testing.assert_array_equal(got, want, err_msg=str(seed))
    with pytest.raises(ne.NEError):
        ne.mt19937_uniforms(2**32, 4)
    # generate.py draws through np.random.choice: one random_sample per call
    rs = np.random.RandomState(7)
    p = np.full(10, 0.1)
    picks = [rs.choice(10, p=p) for _ in range(5)]
    u = ne.mt19937_uniforms(7, 5)
    cdf = np.cumsum(p)
    cdf /= cdf[-1]
    assert picks == [int(np.searchsorted(cdf, x, side="right")) for x in u]
