"""ne_k_attn_bwd_noalloc (no allocation on any call: its delta scratch is a fixed device array)
against ne_k_attn_bwd with a caller-provided delta: bit-identical gradients on two calls in a
row, the second smaller, so the second call runs over the scratch the first one left."""
import math

import numpy as np
import pytest

from gpu_util import FMT, _release_device_tensors, call, dev, host, need_gpu, ptr, zeros  # noqa: F401
import ne

pytestmark = pytest.mark.gpu


def _inputs(rng, B, S, NH, NKV, HD, rnd, tdt):
    T = B * S
    q = rnd(rng.standard_normal((T, NH * HD)).astype(np.float32))
    k = rnd(rng.standard_normal((T, NKV * HD)).astype(np.float32))
    v = rnd(rng.standard_normal((T, NKV * HD)).astype(np.float32))
    do = rnd(rng.standard_normal((T, NH * HD)).astype(np.float32))
    return dev(q, tdt), dev(k, tdt), dev(v, tdt), dev(do, tdt)


@pytest.mark.parametrize("fmt", ["fp16", "bf16"])
def test_attn_bwd_noalloc_matches_attn_bwd(fmt):
    need_gpu()
    L = ne.lib()
    dt, tdt, rnd, _ = FMT[fmt]
    rng = np.random.default_rng(7)
    for B, S, NH, NKV, HD in [(2, 512, 16, 8, 128), (1, 128, 4, 2, 64)]:
        print(f"\n[noalloc {fmt}] B={B} S={S} NH={NH} NKV={NKV} HD={HD}", flush=True)
        T, scale = B * S, 1.0 / math.sqrt(HD)
        qd, kd, vd, dod = _inputs(rng, B, S, NH, NKV, HD, rnd, tdt)
        o, lse = zeros((T, NH * HD), tdt), zeros((T, NH))
        call(L.ne_k_attn_fwd, dt, ptr(qd), NH * HD, ptr(kd), NKV * HD, ptr(vd), NKV * HD, ptr(o), NH * HD,
             ptr(lse), B, S, NH, NKV, HD, scale, None)
        outs = []
        for noalloc in (False, True):
            dq, dk, dv = zeros((T, NH * HD)), zeros((T, NKV * HD)), zeros((T, NKV * HD), tdt)
            head = (dt, ptr(qd), NH * HD, ptr(kd), NKV * HD, ptr(vd), NKV * HD, ptr(o), NH * HD, ptr(lse),
                    ptr(dod), NH * HD)
            tail = (ptr(dq), NH * HD, ptr(dk), NKV * HD, ptr(dv), NKV * HD, B, S, NH, NKV, HD, scale, None)
            if noalloc:
                call(L.ne_k_attn_bwd_noalloc, *head, *tail)
            else:
                call(L.ne_k_attn_bwd, *head, ptr(zeros((T, NH))), *tail)
            outs.append((host(dq), host(dk), host(dv)))
        for a, b, name in zip(outs[0], outs[1], ("dq", "dk", "dv")):
            assert np.isfinite(a).all() and np.abs(a).max() > 0, name
            np.testing.assert_array_equal(b, a, err_msg=name)
    # beyond the fixed scratch: rejected on the host, nothing launched
    rc = L.ne_k_attn_bwd_noalloc(dt, None, 0, None, 0, None, 0, None, 0, None, None, 0, None, 0, None, 0, None, 0,
                                 64, 2048, 16, 8, 128, 1.0, None)
    assert rc == -1 and b"exceeds the fixed scratch" in L.ne_last_error()
