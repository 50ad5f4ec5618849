"""Kernel-level parity of the HIP kernels through the C-ABI (device pointers) against the
numpy oracle (oracle/model.py) and float64 numpy restatements of the same op, in both
16-bit formats.  Tolerances scale with the format's unit roundoff u (fp16 2^-11, bf16 2^-8):
a single rounding of the output gives rel-L2 ~ u/sqrt(3)."""
import ctypes
import math

import numpy as np
import pytest

from gpu_util import FMT, _release_device_tensors, call, dev, host, need_gpu, ptr, rel_l2, torch, zeros  # noqa: F401
import ne
from oracle import model as om

pytestmark = pytest.mark.gpu
L = None
FMTS = ["fp16", "bf16"]


@pytest.fixture(autouse=True)
def _gpu():
    need_gpu()
    global L
    L = ne.lib()


# ------------------------------------------------------------------------- GEMM

def _operands(rng, M, N, K, layout, fmt):
    dt, tdt, rnd, _ = FMT[fmt]
    A = rnd(rng.standard_normal((M, K)).astype(np.float32))   # logical [M,K]
    B = rnd(rng.standard_normal((K, N)).astype(np.float32))   # logical [K,N]
    a_store = A if layout in (0, 2) else A.T                  # bit0: A stored [K,M]
    b_store = B.T if layout in (0, 1) else B                  # bit1: B stored [K,N]
    return A, B, dev(a_store, tdt), a_store.shape[1], dev(b_store, tdt), b_store.shape[1]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("layout", [0, 2, 3, 1])
@pytest.mark.parametrize("shape", [(64, 64, 64), (128, 192, 320), (256, 4096, 1024), (1024, 1024, 256),
                                   (2048, 1024, 4096), (4096, 4096, 128), (256, 1024, 16384), (512, 12800, 256)])
def test_gemm_f32_layouts(fmt, layout, shape):
    M, N, K = shape
    rng = np.random.default_rng(M + N + K + layout)
    A, B, a, lda, b, ldb = _operands(rng, M, N, K, layout, fmt)
    c = zeros((M, N))
    call(L.ne_k_gemm, FMT[fmt][0], layout, 1, M, N, K, ptr(a), lda, ptr(b), ldb, ptr(c), N, None, 0, 0.5, None)
    ref = 0.5 * (A.astype(np.float64) @ B.astype(np.float64))
    err = np.abs(host(c) - ref).max() / np.abs(ref).max()
    assert err < 1e-5, err


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("accumulate", [0, 1])
def test_gemm_wgrad_group(fmt, accumulate):
    """A layer's weight-gradient GEMMs of a 16k-token step as one launch (whole-K 256x256 tiles,
    the problems' tiles in one grid): each C_p = alpha * A_p^T B_p (+ C_p) against a float64
    product of the same 16-bit operands, and bit-identical to the same GEMM run alone through
    ne_k_gemm (no split-K there either: the same K order for every output element)."""
    dt, tdt, rnd, _ = FMT[fmt]
    K = 8192
    shapes = [(4096, 1024), (1024, 2048), (6144, 1024)]  # 64 + 32 + 96 tiles of 256x256
    n = len(shapes)
    rng = np.random.default_rng(7 + accumulate)
    As = [dev(rnd(rng.standard_normal((K, M)).astype(np.float32)), tdt) for M, _ in shapes]
    Bs = [dev(rnd(rng.standard_normal((K, N)).astype(np.float32)), tdt) for _, N in shapes]
    C0 = [rng.standard_normal((M, N)).astype(np.float32) for M, N in shapes]
    Cs = [dev(c) if accumulate else zeros(c.shape) for c in C0]
    arr = lambda ct, xs: (ct * n)(*xs)
    call(L.ne_k_gemm_wgrad_group, dt, n, arr(ctypes.c_int, [M for M, _ in shapes]),
         arr(ctypes.c_int, [N for _, N in shapes]), K, arr(ctypes.c_void_p, [a.data_ptr() for a in As]),
         arr(ctypes.c_int64, [M for M, _ in shapes]), arr(ctypes.c_void_p, [b.data_ptr() for b in Bs]),
         arr(ctypes.c_int64, [N for _, N in shapes]), arr(ctypes.c_void_p, [c.data_ptr() for c in Cs]),
         accumulate, 0.5, None)
    for p, (M, N) in enumerate(shapes):
        ref = 0.5 * (As[p].double().T @ Bs[p].double())
        if accumulate:
            ref += torch.as_tensor(C0[p], dtype=torch.float64, device="cuda")
        ref = ref.cpu().numpy()
        got = host(Cs[p])
        err = np.abs(got - ref).max() / np.abs(ref).max()
        assert err < 1e-5, (p, err)
        alone = dev(C0[p]) if accumulate else zeros((M, N))
        call(L.ne_k_gemm, dt, 3, 2 if accumulate else 1, M, N, K, ptr(As[p]), M, ptr(Bs[p]), N, ptr(alone), N,
             None, 0, 0.5, None)
        np.testing.assert_array_equal(host(alone), got, err_msg=f"problem {p}")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("epi", [0, 2, 3])
def test_gemm_epilogues(fmt, epi):
    M, N, K = 256, 512, 256
    dt, tdt, _, u = FMT[fmt]
    rng = np.random.default_rng(epi)
    A, B, a, lda, b, ldb = _operands(rng, M, N, K, 0, fmt)
    ref = A.astype(np.float64) @ B.astype(np.float64)
    R = rng.standard_normal((M, N)).astype(np.float32)
    if epi == 0:
        c = zeros((M, N), tdt)
        call(L.ne_k_gemm, dt, 0, 0, M, N, K, ptr(a), lda, ptr(b), ldb, ptr(c), N, None, 0, 1.0, None)
        assert rel_l2(host(c), ref) < u
    elif epi == 2:
        c = dev(R)
        call(L.ne_k_gemm, dt, 0, 2, M, N, K, ptr(a), lda, ptr(b), ldb, ptr(c), N, None, 0, 2.0, None)
        assert rel_l2(host(c), R + 2 * ref) < 1e-6
    else:
        c = zeros((M, N))
        r = dev(R)
        call(L.ne_k_gemm, dt, 0, 3, M, N, K, ptr(a), lda, ptr(b), ldb, ptr(c), N, ptr(r), N, 0.25, None)
        assert rel_l2(host(c), R + 0.25 * ref) < 1e-6


@pytest.mark.parametrize("layout,epi,M,N", [(0, 0, 2048, 32896), (0, 1, 2048, 32896), (0, 3, 2048, 32896),
                                            (3, 1, 65664, 1024)])
def test_gemm_ragged_split(layout, epi, M, N):
    """A large output whose N (or M) is not a multiple of 256 (128.5 or 256.5 tiles of 256,
    1024-deep) runs as a part of whole 256-wide tiles and the remaining columns (rows): the
    seam and the last columns (rows) match the float64 product, and the guard row past the
    output stays zero."""
    K = 1024
    dt, tdt, _, u = FMT["fp16"]
    rng = np.random.default_rng(M + N + epi)
    A, B, a, lda, b, ldb = _operands(rng, M, N, K, layout, "fp16")
    ref = A.astype(np.float64) @ B.astype(np.float64)
    if epi == 0:
        c = zeros((M + 1, N), tdt)
        call(L.ne_k_gemm, dt, layout, 0, M, N, K, ptr(a), lda, ptr(b), ldb, ptr(c), N, None, 0, 1.0, None)
        got = host(c)
        assert rel_l2(got[:M], ref) < u
        assert rel_l2(got[:, -128:][:M], ref[:, -128:]) < u  # the remainder part
    elif epi == 1:
        c = zeros((M + 1, N))
        call(L.ne_k_gemm, dt, layout, 1, M, N, K, ptr(a), lda, ptr(b), ldb, ptr(c), N, None, 0, 0.5, None)
        got = host(c)
        err = np.abs(got[:M] - 0.5 * ref).max() / np.abs(ref).max()
        assert err < 1e-5, err
        tail = got[M - 128:M] if layout == 3 else got[:M, -128:]
        tref = 0.5 * (ref[M - 128:] if layout == 3 else ref[:, -128:])
        assert np.abs(tail - tref).max() / np.abs(ref).max() < 1e-5
    else:
        R = rng.standard_normal((M, N)).astype(np.float32)
        c = zeros((M + 1, N))
        call(L.ne_k_gemm, dt, layout, 3, M, N, K, ptr(a), lda, ptr(b), ldb, ptr(c), N, ptr(dev(R)), N, 0.25, None)
        got = host(c)
        assert rel_l2(got[:M], R + 0.25 * ref) < 1e-6
    assert np.abs(got[M]).max() == 0


@pytest.mark.parametrize("fmt", FMTS)
def test_gemm_swiglu_backward_epilogue(fmt):
    T, D, H = 128, 256, 320
    dt, tdt, rnd, u = FMT[fmt]
    rng = np.random.default_rng(7)
    dy = rnd(rng.standard_normal((T, D)).astype(np.float32))
    W2 = rnd(rng.standard_normal((D, H)).astype(np.float32) * 0.05)
    h13 = rnd(rng.standard_normal((T, 2 * H)).astype(np.float32))
    dh = zeros((T, 2 * H), tdt)
    call(L.ne_k_gemm, dt, 2, 4, T, H, D, ptr(dev(dy, tdt)), D, ptr(dev(W2, tdt)), H, ptr(dh), 2 * H,
         ptr(dev(h13, tdt)), 2 * H, 1.0, None)
    dgate = dy.astype(np.float64) @ W2
    h1, h3 = h13[:, :H].astype(np.float64), h13[:, H:].astype(np.float64)
    sg = 1 / (1 + np.exp(-h1))
    ref = np.concatenate([dgate * h3 * sg * (1 + h1 * (1 - sg)), dgate * h1 * sg], axis=1)
    assert rel_l2(host(dh), ref) < u


# --------------------------------------------------------------------- norms, embed

@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T,D", [(64, 128), (256, 768), (512, 1024)])
def test_rmsnorm_fwd_bwd(fmt, T, D):
    dt, tdt, _, u = FMT[fmt]
    rng = np.random.default_rng(T)
    x = rng.standard_normal((T, D)).astype(np.float32) * 3
    g = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    dy = rng.standard_normal((T, D)).astype(np.float32)
    res = rng.standard_normal((T, D)).astype(np.float32)
    xd, gd = dev(x), dev(g)
    y = zeros((T, D), tdt)
    r = zeros((T,))
    call(L.ne_k_rmsnorm_fwd, dt, ptr(xd), ptr(gd), ptr(y), ptr(r), T, D, 1e-5, None)
    yr, rr = om.rmsnorm(x, g, 1e-5)
    assert rel_l2(host(y), yr) < u
    np.testing.assert_allclose(host(r), rr[:, 0], rtol=1e-6)
    dx = zeros((T, D))
    dxb = zeros((T, D), tdt)
    dg = dev(np.full(D, 0.5, np.float32))
    call(L.ne_k_rmsnorm_bwd, dt, ptr(dev(dy)), ptr(xd), ptr(gd), ptr(r), ptr(dev(res)), ptr(dx), ptr(dxb), 0.5,
         ptr(dg), 0.25, T, D, None)
    dxr, dgr = om.rmsnorm_bwd(dy, x, g, rr)
    assert rel_l2(host(dx), dxr + res) < 1e-5
    assert rel_l2(host(dxb), 0.5 * (dxr + res)) < u
    assert rel_l2(host(dg), 0.25 * dgr + 0.5) < 1e-5


def test_embed_fwd_bwd_with_repeated_ids():
    V, D, T = 512, 256, 192
    rng = np.random.default_rng(3)
    E = rng.standard_normal((V, D)).astype(np.float32)
    tok = rng.integers(0, 16, T).astype(np.int32)      # many collisions
    x = zeros((T, D))
    call(L.ne_k_embed_fwd, ptr(dev(E)), ptr(dev(tok)), ptr(x), T, D, None)
    np.testing.assert_array_equal(host(x), E[tok])
    dx = rng.standard_normal((T, D)).astype(np.float32)
    gE = zeros((V, D))
    call(L.ne_k_embed_bwd, ptr(gE), ptr(dev(tok)), ptr(dev(dx)), 0.5, T, D, None)
    ref = np.zeros((V, D))
    np.add.at(ref, tok, 0.5 * dx.astype(np.float64))
    np.testing.assert_allclose(host(gE), ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("fmt", FMTS)
def test_swiglu_fwd(fmt):
    T, H = 64, 192
    dt, tdt, rnd, u = FMT[fmt]
    rng = np.random.default_rng(4)
    h13 = rnd(rng.standard_normal((T, 2 * H)).astype(np.float32) * 2)
    gate = zeros((T, H), tdt)
    call(L.ne_k_swiglu_fwd, dt, ptr(dev(h13, tdt)), ptr(gate), T, H, None)
    ref = om.silu(h13[:, :H]) * h13[:, H:]
    assert rel_l2(host(gate), ref) < u


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T,H,D", [(256, 3072, 1024), (256, 2048, 768), (2048, 3072, 1024), (4096, 3072, 1024),
                                   (1024, 3072, 1024), (128, 192, 256), (128, 256, 192)])
def test_gemm_swiglu_fwd_epilogue(fmt, T, H, D):
    """The W1|W3 GEMM with the SwiGLU forward in its epilogue (B rows gathered so that h1 and h3
    of a column share a work-group) writes the same h13 and gate, bit for bit, as the plain
    16-bit GEMM followed by the SwiGLU kernel; the gate against silu(h1) * h3 of float64 sums."""
    dt, tdt, rnd, u = FMT[fmt]
    rng = np.random.default_rng(T + H)
    x = rnd(rng.standard_normal((T, D)).astype(np.float32))
    w13 = rnd((rng.standard_normal((2 * H, D)) / np.sqrt(D)).astype(np.float32))
    xd, wd = dev(x, tdt), dev(w13, tdt)
    h13, gate = zeros((T, 2 * H), tdt), zeros((T, H), tdt)
    call(L.ne_k_gemm, dt, 0, 7, T, 2 * H, D, ptr(xd), D, ptr(wd), D, ptr(h13), 2 * H, ptr(gate), H, 1.0, None)
    h13_ref, gate_ref = zeros((T, 2 * H), tdt), zeros((T, H), tdt)
    call(L.ne_k_gemm, dt, 0, 0, T, 2 * H, D, ptr(xd), D, ptr(wd), D, ptr(h13_ref), 2 * H, None, 0, 1.0, None)
    call(L.ne_k_swiglu_fwd, dt, ptr(h13_ref), ptr(gate_ref), T, H, None)
    np.testing.assert_array_equal(host(h13), host(h13_ref))
    np.testing.assert_array_equal(host(gate), host(gate_ref))
    h = x.astype(np.float64) @ w13.astype(np.float64).T
    ref = om.silu(h[:, :H]) * h[:, H:]
    assert rel_l2(host(gate), ref) < 3 * u


# -------------------------------------------------------------------- RoPE / QK-norm

@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("HD,qk", [(64, False), (128, True), (64, True)])
def test_qk_prep_fwd_bwd(fmt, HD, qk):
    dt, tdt, rnd, u = FMT[fmt]
    B, S, NH, NKV = 2, 64, 4, 2
    T, Q, KV = B * S, NH * HD, NKV * HD
    QKV = Q + 2 * KV
    theta = 1e6 if qk else 1e4
    rng = np.random.default_rng(HD + qk)
    qkv = rnd(rng.standard_normal((T, QKV)).astype(np.float32))
    gq = (1 + 0.3 * rng.standard_normal(HD)).astype(np.float32)
    gk = (1 + 0.3 * rng.standard_normal(HD)).astype(np.float32)
    cos, sin = om.rope_tables(S, HD, theta)
    cosd, sind = dev(cos.astype(np.float32)), dev(sin.astype(np.float32))
    qkvd = dev(qkv, tdt)
    qr, kr = zeros((T, Q), tdt), zeros((T, KV), tdt)
    rq, rk = zeros((T, NH)), zeros((T, NKV))
    gqd, gkd = (dev(gq), dev(gk)) if qk else (None, None)
    call(L.ne_k_qk_prep_fwd, dt, ptr(qkvd), QKV, ptr(cosd), ptr(sind), ptr(gqd), ptr(gkd), ptr(qr), ptr(kr),
         ptr(rq), ptr(rk), T, S, NH, NKV, HD, 1e-5, None)
    q = qkv[:, :Q].reshape(B, S, NH, HD)
    k = qkv[:, Q:Q + KV].reshape(B, S, NKV, HD)
    if qk:
        q, rqr = om.rmsnorm(q, gq, 1e-5)
        k, rkr = om.rmsnorm(k, gk, 1e-5)
        np.testing.assert_allclose(host(rq), rqr.reshape(T, NH), rtol=1e-5)
    qe = om.rope_apply(q, cos, sin).reshape(T, Q)
    ke = om.rope_apply(k, cos, sin).reshape(T, KV)
    assert rel_l2(host(qr), qe) < u and rel_l2(host(kr), ke) < u
    # backward
    dq = rng.standard_normal((T, Q)).astype(np.float32)
    dk = rng.standard_normal((T, KV)).astype(np.float32)
    dqkv = zeros((T, QKV), tdt)
    dgq, dgk = (zeros((HD,)), zeros((HD,))) if qk else (None, None)
    call(L.ne_k_qk_prep_bwd, dt, ptr(dev(dq)), ptr(dev(dk)), ptr(qkvd), QKV, ptr(cosd), ptr(sind), ptr(gqd),
         ptr(gkd), ptr(rq), ptr(rk), ptr(dqkv), ptr(dgq), ptr(dgk), 2.0, T, S, NH, NKV, HD, None)
    dqn = om.rope_bwd(dq.reshape(B, S, NH, HD), cos, sin)
    dkn = om.rope_bwd(dk.reshape(B, S, NKV, HD), cos, sin)
    if qk:
        dqn, dgqr = om.rmsnorm_bwd(dqn, qkv[:, :Q].reshape(B, S, NH, HD), gq, rqr)
        dkn, dgkr = om.rmsnorm_bwd(dkn, qkv[:, Q:Q + KV].reshape(B, S, NKV, HD), gk, rkr)
        assert rel_l2(host(dgq), 2 * dgqr) < 1e-4 and rel_l2(host(dgk), 2 * dgkr) < 1e-4
    got = host(dqkv)
    assert rel_l2(got[:, :Q], dqn.reshape(T, Q)) < u
    assert rel_l2(got[:, Q:Q + KV], dkn.reshape(T, KV)) < u


# ------------------------------------------------------------------------ attention

def _attn_ref(q, k, v, do, NH, NKV, scale):
    """float64 causal GQA attention fwd/bwd; q [B,S,NH,HD], k/v [B,S,NKV,HD]."""
    B, S, _, HD = q.shape
    r = NH // NKV
    o = np.zeros_like(q, dtype=np.float64)
    lse = np.zeros((B, S, NH))
    dq = np.zeros_like(o)
    dk = np.zeros((B, S, NKV, HD))
    dv = np.zeros((B, S, NKV, HD))
    mask = np.triu(np.ones((S, S), bool), 1)
    for b in range(B):
        for h in range(NH):
            kh = h // r
            s = scale * (q[b, :, h].astype(np.float64) @ k[b, :, kh].T.astype(np.float64))
            s[mask] = -np.inf
            m = s.max(1, keepdims=True)
            e = np.exp(s - m)
            l = e.sum(1, keepdims=True)
            p = e / l
            lse[b, :, h] = (m + np.log(l))[:, 0]
            o[b, :, h] = p @ v[b, :, kh]
            dp = do[b, :, h] @ v[b, :, kh].T
            ds = p * (dp - (dp * p).sum(1, keepdims=True))
            dq[b, :, h] = scale * ds @ k[b, :, kh]
            dk[b, :, kh] += scale * ds.T @ q[b, :, h]
            dv[b, :, kh] += p.T @ do[b, :, h]
    return o, lse, dq, dk, dv


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("B,S,NH,NKV,HD", [(1, 64, 2, 2, 64), (2, 128, 4, 2, 64), (1, 256, 4, 2, 128),
                                           (2, 192, 2, 1, 128), (2, 512, 16, 4, 128),
                                           (1, 1024, 64, 16, 128)])
def test_flash_attention_fwd_bwd(fmt, B, S, NH, NKV, HD):
    dt, tdt, rnd, u = FMT[fmt]
    T = B * S
    rng = np.random.default_rng(S + HD)
    q = rnd(rng.standard_normal((B, S, NH, HD)).astype(np.float32))
    k = rnd(rng.standard_normal((B, S, NKV, HD)).astype(np.float32))
    v = rnd(rng.standard_normal((B, S, NKV, HD)).astype(np.float32))
    do = rnd(rng.standard_normal((B, S, NH, HD)).astype(np.float32))
    scale = 1.0 / math.sqrt(HD)
    # q/k/v as column blocks of one wide row (strided like the model's qkv buffer)
    ld = NH * HD + 2 * NKV * HD
    qkv = np.concatenate([q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1)], axis=1)
    qkvd = dev(qkv, tdt)
    qd = qkvd[:, :NH * HD]
    kd = qkvd[:, NH * HD:NH * HD + NKV * HD]
    vd = qkvd[:, NH * HD + NKV * HD:]
    o = zeros((T, NH * HD), tdt)
    lse = zeros((T, NH))
    call(L.ne_k_attn_fwd, dt, ptr(qd), ld, ptr(kd), ld, ptr(vd), ld, ptr(o), NH * HD, ptr(lse), B, S, NH, NKV, HD,
         scale, None)
    o_r, lse_r, dq_r, dk_r, dv_r = _attn_ref(q, k, v, do, NH, NKV, scale)
    np.testing.assert_allclose(host(lse), lse_r.reshape(T, NH), rtol=1e-4, atol=1e-4)
    delta = zeros((T, NH))
    dq, dk = zeros((T, NH * HD)), zeros((T, NKV * HD))
    dqkv = zeros((T, ld), tdt)
    dv = dqkv[:, NH * HD + NKV * HD:]
    call(L.ne_k_attn_bwd, dt, ptr(qd), ld, ptr(kd), ld, ptr(vd), ld, ptr(o), NH * HD, ptr(lse),
         ptr(dev(do, tdt)), NH * HD, ptr(delta), ptr(dq), NH * HD, ptr(dk), NKV * HD, ptr(dv), ld, B, S, NH, NKV, HD,
         scale, None)
    e = (rel_l2(host(o), o_r.reshape(T, -1)), rel_l2(host(dq), dq_r.reshape(T, -1)),
         rel_l2(host(dk), dk_r.reshape(T, -1)), rel_l2(host(dqkv)[:, NH * HD + NKV * HD:], dv_r.reshape(T, -1)))
    print(f"\n  {fmt} rel-L2 o={e[0]:.2e} dq={e[1]:.2e} dk={e[2]:.2e} dv={e[3]:.2e}")
    # P and dS are rounded to the 16-bit format for the MFMAs: a few roundings deep
    assert max(e) < 4 * u
    # q and k columns of dqkv untouched
    assert np.abs(host(dqkv)[:, :NH * HD + NKV * HD]).max() == 0


@pytest.mark.timeout(300)
@pytest.mark.parametrize("fmt", FMTS)
def test_flash_attention_at_scale(fmt):
    """The at-scale shape, B=8 x S=2048 with Qwen3-0.6B's 16 query / 8 KV heads of 128: the
    whole batch runs (the XCD block order covers the full grid); the float64 reference is
    computed for sequences 0 and 7 and KV heads 0 and 7 with their query heads."""
    dt, tdt, rnd, u = FMT[fmt]
    B, S, NH, NKV, HD = 8, 2048, 16, 8, 128
    T = B * S
    rng = np.random.default_rng(2048)
    q = rnd(rng.standard_normal((B, S, NH, HD)).astype(np.float32))
    k = rnd(rng.standard_normal((B, S, NKV, HD)).astype(np.float32))
    v = rnd(rng.standard_normal((B, S, NKV, HD)).astype(np.float32))
    do = rnd(rng.standard_normal((B, S, NH, HD)).astype(np.float32))
    scale = 1.0 / math.sqrt(HD)
    qd, kd, vd = dev(q.reshape(T, -1), tdt), dev(k.reshape(T, -1), tdt), dev(v.reshape(T, -1), tdt)
    o, lse = zeros((T, NH * HD), tdt), zeros((T, NH))
    call(L.ne_k_attn_fwd, dt, ptr(qd), NH * HD, ptr(kd), NKV * HD, ptr(vd), NKV * HD, ptr(o), NH * HD, ptr(lse), B, S,
         NH, NKV, HD, scale, None)
    delta, dq, dk = zeros((T, NH)), zeros((T, NH * HD)), zeros((T, NKV * HD))
    dv = zeros((T, NKV * HD), tdt)
    call(L.ne_k_attn_bwd, dt, ptr(qd), NH * HD, ptr(kd), NKV * HD, ptr(vd), NKV * HD, ptr(o), NH * HD, ptr(lse),
         ptr(dev(do.reshape(T, -1), tdt)), NH * HD, ptr(delta), ptr(dq), NH * HD, ptr(dk), NKV * HD, ptr(dv),
         NKV * HD, B, S, NH, NKV, HD, scale, None)
    o_g = host(o).reshape(B, S, NH, HD)
    lse_g = host(lse).reshape(B, S, NH)
    dq_g = host(dq).reshape(B, S, NH, HD)
    dk_g = host(dk).reshape(B, S, NKV, HD)
    dv_g = host(dv).reshape(B, S, NKV, HD)
    worst = 0.0
    for b in (0, 7):
        for kvh in (0, 7):
            hs = slice(2 * kvh, 2 * kvh + 2)
            o_r, lse_r, dq_r, dk_r, dv_r = _attn_ref(q[b:b + 1, :, hs], k[b:b + 1, :, kvh:kvh + 1],
                                                     v[b:b + 1, :, kvh:kvh + 1], do[b:b + 1, :, hs], 2, 1, scale)
            np.testing.assert_allclose(lse_g[b, :, hs], lse_r[0], rtol=1e-4, atol=1e-4)
            e = (rel_l2(o_g[b, :, hs], o_r[0]), rel_l2(dq_g[b, :, hs], dq_r[0]),
                 rel_l2(dk_g[b, :, kvh], dk_r[0, :, 0]), rel_l2(dv_g[b, :, kvh], dv_r[0, :, 0]))
            worst = max(worst, max(e))
            assert max(e) < 4 * u, (b, kvh, e)
    print(f"\n  {fmt} B=8 S=2048 worst rel-L2 {worst:.2e}")


# --------------------------------------------------------------- cross-entropy (LM head)

@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T,D,V", [(64, 128, 512), (256, 768, 32000), (2048, 128, 32768), (256, 128, 65664),
                                   (2048, 1024, 32896), (64, 192, 512), (64, 320, 512)])
def test_fused_ce_fwd_bwd(fmt, T, D, V):
    """(256, 128, 65664): a vocabulary 256.5 tiles of 256 wide.  (2048, 1024, 32896): 128.5
    tiles, large enough that the classifier GEMMs run as whole 256-wide tiles plus the last 128
    columns (partial slots and target columns offset in the second launch).  D = 192 and 320
    on the 64-row tile: 3 and 5 K steps of 64, an odd count, which the cross-entropy epilogues
    run as one more step over a zeroed A stage (the padded K loop).  The guard row after
    dlogits must stay zero (no store past the last column)."""
    dt, tdt, rnd, u = FMT[fmt]
    rng = np.random.default_rng(V)
    x = rnd(rng.standard_normal((T, D)).astype(np.float32))
    E = rnd(rng.standard_normal((V, D)).astype(np.float32) * 0.05)
    tgt = rng.integers(0, V, T).astype(np.int32)
    xd, Ed, td = dev(x, tdt), dev(E, tdt), dev(tgt)
    part = zeros((T * (V // 64) * 2,))
    tl, lse, rows, loss = zeros((T,)), zeros((T,)), zeros((T,)), zeros((4,))
    call(L.ne_k_ce_fwd, dt, ptr(xd), ptr(Ed), ptr(td), T, D, V, ptr(part), ptr(tl), ptr(lse), ptr(rows), ptr(loss),
         None)
    logits = x.astype(np.float64) @ E.T.astype(np.float64)
    m = logits.max(1, keepdims=True)
    lse_r = (m + np.log(np.exp(logits - m).sum(1, keepdims=True)))[:, 0]
    p_t = np.exp(logits[np.arange(T), tgt] - lse_r)
    loss_r = np.mean(-np.log(p_t + 1e-10))
    np.testing.assert_allclose(host(lse), lse_r, rtol=1e-5)
    assert abs(host(loss)[0] - loss_r) < 1e-4 * abs(loss_r)
    dlg = zeros((T + 1, V), tdt)  # + a guard row
    scale = 1024.0
    call(L.ne_k_ce_bwd, dt, ptr(xd), ptr(Ed), ptr(td), ptr(lse), T, D, V, scale, ptr(dlg), None)
    ref = np.exp(logits - lse_r[:, None])
    ref[np.arange(T), tgt] -= 1
    ref *= scale
    got = host(dlg)
    assert rel_l2(got[:T], ref) < u
    assert np.abs(got[T]).max() == 0


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("T,D,V,estd", [(64, 128, 512, 0.05), (256, 768, 32000, 0.05), (2048, 1024, 32896, 0.05),
                                        (256, 128, 65664, 0.05), (256, 1024, 4096, 0.5), (64, 320, 512, 0.05)])
def test_fused_ce_fwd_grad(fmt, T, D, V, estd):
    """The forward with its gradient in one call (ne_k_ce_fwd_grad): loss and log-sum-exp as
    ne_k_ce_fwd's, and dlogits against float64 within two roundings of the format (the stored
    exp(logit - tile max), then the gradient), whichever tiling the vocabulary takes (ragged
    256.5 and 128.5 tiles as in test_fused_ce_fwd_bwd).  estd 0.5 makes logits of std ~16, a
    peaked softmax like a trained model's, where the target's gradient p - 1 is small.  The
    guard row after dlogits stays zero."""
    dt, tdt, rnd, u = FMT[fmt]
    rng = np.random.default_rng(V + 1)
    x = rnd(rng.standard_normal((T, D)).astype(np.float32))
    E = rnd(rng.standard_normal((V, D)).astype(np.float32) * estd)
    tgt = rng.integers(0, V, T).astype(np.int32)
    logits = x.astype(np.float64) @ E.T.astype(np.float64)
    if estd > 0.1:  # targets at each row's most likely token: p_tgt near 1
        tgt = logits.argmax(1).astype(np.int32)
    xd, Ed, td = dev(x, tdt), dev(E, tdt), dev(tgt)
    part = zeros((T * (V // 64) * 2,))
    tl, lse, rows, loss = zeros((T,)), zeros((T,)), zeros((T,)), zeros((4,))
    dlg = zeros((T + 1, V), tdt)  # + a guard row
    scale = 1024.0
    call(L.ne_k_ce_fwd_grad, dt, ptr(xd), ptr(Ed), ptr(td), T, D, V, ptr(part), ptr(tl), ptr(lse), ptr(rows),
         ptr(loss), scale, ptr(dlg), None)
    m = logits.max(1, keepdims=True)
    lse_r = (m + np.log(np.exp(logits - m).sum(1, keepdims=True)))[:, 0]
    p_t = np.exp(logits[np.arange(T), tgt] - lse_r)
    loss_r = np.mean(-np.log(p_t + 1e-10))
    np.testing.assert_allclose(host(lse), lse_r, rtol=1e-5)
    assert abs(host(loss)[0] - loss_r) < 1e-4 * abs(loss_r) + 1e-6
    ref = np.exp(logits - lse_r[:, None])
    ref[np.arange(T), tgt] -= 1
    ref *= scale
    got = host(dlg)
    err = rel_l2(got[:T], ref)
    print(f"\n  {fmt} T={T} V={V} estd={estd}: dlogits rel-L2 {err:.2e} (u {u:.1e})", flush=True)
    assert err < 2 * u
    assert np.abs(got[T]).max() == 0
    # the loss outputs equal the forward alone
    lse2, loss2 = zeros((T,)), zeros((4,))
    call(L.ne_k_ce_fwd, dt, ptr(xd), ptr(Ed), ptr(td), T, D, V, ptr(part), ptr(tl), ptr(lse2), ptr(rows),
         ptr(loss2), None)
    np.testing.assert_array_equal(host(lse2), host(lse))
    assert host(loss2)[0] == host(loss)[0]


# ------------------------------------------------------------------------ optimizer

@pytest.mark.parametrize("fmt", FMTS)
def test_adam_matches_oracle_and_grad_norm(fmt):
    dt, tdt, rnd, _ = FMT[fmt]
    n, n_decay = 4096 * 3, 4096 * 2
    rng = np.random.default_rng(11)
    p = rng.standard_normal(n).astype(np.float32) * 0.02
    g = rng.standard_normal(n).astype(np.float32) * 1e-2
    m = rng.standard_normal(n).astype(np.float32) * 1e-3
    v = np.abs(rng.standard_normal(n).astype(np.float32)) * 1e-5
    pd, gd, md, vd = dev(p), dev(g), dev(m), dev(v)
    pb = zeros((n,), tdt)
    part = zeros((1024,), torch.float64)
    gs, gn = zeros((1,)), zeros((1,))
    call(L.ne_k_grad_norm, ptr(gd), n, 0.5, 1.0, ptr(part), ptr(gs), ptr(gn), None)
    norm = 0.5 * np.linalg.norm(g.astype(np.float64))
    assert abs(host(gn)[0] - norm) < 1e-5 * norm
    scale = 0.5 * min(1.0, 1.0 / norm)
    assert abs(host(gs)[0] - scale) < 1e-6 * scale
    t = 7
    call(L.ne_k_adam, dt, ptr(pd), ptr(gd), ptr(md), ptr(vd), ptr(pb), n, n_decay, 3e-4, 0.9, 0.95, 1e-8, 0.1, t,
         ptr(gs), 1, None)
    pr, mr, vr = p.copy(), m.copy(), v.copy()
    ge = g * np.float32(host(gs)[0])
    om.adam_update(pr[:n_decay], ge[:n_decay], mr[:n_decay], vr[:n_decay], t, 3e-4, 0.9, 0.95, 1e-8, 0.1)
    om.adam_update(pr[n_decay:], ge[n_decay:], mr[n_decay:], vr[n_decay:], t, 3e-4, 0.9, 0.95, 1e-8, 0.0)
    # per element within 1e-5 relative, with an absolute floor of ~one fp32 ulp of the
    # tensor's scale (terms that cancel in m = b1*m + (1-b1)*g leave ulp-level residue)
    np.testing.assert_allclose(host(pd), pr, rtol=1e-5, atol=1e-7 * np.abs(pr).max())
    np.testing.assert_allclose(host(md), mr, rtol=1e-5, atol=1e-7 * np.abs(mr).max())
    np.testing.assert_allclose(host(vd), vr, rtol=1e-5, atol=1e-7 * np.abs(vr).max())
    assert np.abs(host(gd)).max() == 0
    np.testing.assert_array_equal(host(pb), rnd(host(pd)))
