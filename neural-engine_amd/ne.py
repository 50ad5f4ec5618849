"""ctypes binding of libne.so (include/ne.h): the Python harness over the C-ABI.

The library is loaded from this directory; a missing or stale build raises instead of
falling back to anything else.  Tensor names follow the checkpoint order of the
reference (TD/train.m:111-129): "layers.{l}.{Wq,Wk,Wv,Wo,W1,W2,W3,rms_att,rms_ffn}",
"rms_final", "embed", and with QK-norm "layers.{l}.{q_norm,k_norm}".
"""
from __future__ import annotations

import ctypes as C
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libne.so")

NE_PARAM, NE_GRAD, NE_ADAM_M, NE_ADAM_V = 0, 1, 2, 3
NE_BF16, NE_FP16 = 0, 1
PROF_FAMILIES = ("gemm_fwd", "gemm_bwd", "attn_fwd", "attn_bwd", "norm", "ce", "adam", "gnorm",
                 "embed", "decode")
LAYER_TENSORS = ("Wq", "Wk", "Wv", "Wo", "W1", "W2", "W3", "rms_att", "rms_ffn")
TIMELINE_PHASES = ("wait", "fwd", "cls", "bwd", "dwait", "tail", "step", "opt", "update")
OVF_SITES = ("norm_fwd", "qkv", "h13", "swiglu", "dlogits", "norm_bwd", "dh13", "dattn", "dv", "dqkv")

# every symbol include/ne.h declares
EXPORTS = (
    "ne_create", "ne_destroy", "ne_last_error", "ne_sync", "ne_num_tensors", "ne_tensor_numel",
    "ne_set_tensor", "ne_get_tensor", "ne_train_step", "ne_use_graphs", "ne_overlap_weight_grads", "ne_optimizer_step",
    "ne_rmsnorm_bwd_formula", "ne_zero_grads",
    "ne_grad_scale_info", "ne_grad_norm_parts", "ne_step_stats", "ne_get_state", "ne_set_state", "ne_load_ckpt_v4", "ne_save_ckpt_v4",
    "ne_decode", "ne_decode_seeded", "ne_mt19937_uniforms", "ne_set_vocab_map",
    "ne_prof_enable", "ne_prof_reset", "ne_prof_get", "ne_timeline", "ne_step_timeline", "ne_update_launches", "ne_k_rmsnorm_fwd", "ne_k_rmsnorm_bwd",
    "ne_k_gemm", "ne_k_gemm_wgrad_group", "ne_k_qk_prep_fwd", "ne_k_qk_prep_bwd", "ne_k_attn_fwd", "ne_k_attn_bwd", "ne_k_attn_bwd_noalloc",
    "ne_k_ce_fwd", "ne_k_ce_bwd", "ne_k_ce_fwd_grad", "ne_k_adam", "ne_k_grad_norm", "ne_k_embed_fwd",
    "ne_k_embed_bwd", "ne_k_swiglu_fwd", "ne_k_mfma_ceiling",
)


class NEError(RuntimeError):
    pass


CKPT_MAGIC = 0x424C5A54
_CKPT_HDR = struct.Struct("<10i2f3d6i")   # 96 bytes, TD/config.h:82-91


def read_ckpt_header(path):
    """Model dims and counters of a v4 checkpoint (TD/config.h:82-91), plus whether the
    QK-norm gain trailer follows the body (detected from the file size)."""
    with open(path, "rb") as f:
        raw = f.read(_CKPT_HDR.size)
    if len(raw) != _CKPT_HDR.size:
        raise NEError(f"{path}: short header")
    (magic, version, step, total_steps, n_layers, vocab, dim, hidden, n_heads, seq, lr, loss,
     cum_compile, cum_train, cum_wall, cum_steps, cum_batches, adam_t, kv_heads, head_dim, q_dim) = _CKPT_HDR.unpack(raw)
    if magic != CKPT_MAGIC or version != 4:
        raise NEError(f"{path}: not a v4 checkpoint")
    if kv_heads <= 0:                           # files of the MHA trainer leave the GQA slots empty
        kv_heads, head_dim, q_dim = n_heads, dim // n_heads, dim
    kv_dim = kv_heads * head_dim
    n = n_layers * (q_dim * dim + 2 * kv_dim * dim + dim * q_dim + 3 * hidden * dim + 2 * dim) + dim + vocab * dim
    base = _CKPT_HDR.size + 3 * 4 * n
    size = os.path.getsize(path)
    qkn = size == base + 12 + n_layers * 6 * head_dim * 4
    if size != base and not qkn:
        raise NEError(f"{path}: size {size}, expected {base}")
    return dict(step=step, total_steps=total_steps, n_layers=n_layers, vocab=vocab, dim=dim, hidden=hidden,
                n_heads=n_heads, kv_heads=kv_heads, head_dim=head_dim, q_dim=q_dim, seq=seq, lr=lr, loss=loss,
                adam_t=adam_t, qk_norm=qkn)


class Config(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("dim", "hidden", "n_heads", "kv_heads", "head_dim",
                                          "n_layers", "vocab", "seq", "batch", "qk_norm")] + \
               [(n, C.c_float) for n in ("rope_theta", "res_alpha", "norm_eps")] + \
               [(n, C.c_int32) for n in ("decode_batch", "decode_ctx", "dtype")]


class TrainState(C.Structure):
    _fields_ = [("step", C.c_int32), ("total_steps", C.c_int32), ("lr", C.c_float),
                ("loss", C.c_float), ("cum_compile", C.c_double), ("cum_train", C.c_double),
                ("cum_wall", C.c_double), ("cum_steps", C.c_int32), ("cum_batches", C.c_int32),
                ("adam_t", C.c_int32)]


_lib = None

P, I, F, D, L = C.c_void_p, C.c_int, C.c_float, C.c_double, C.c_int64


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise NEError(f"{LIB_PATH} is not built (run __graft_entry__.build() or make -C neural-engine_amd)")
    h = C.CDLL(LIB_PATH)
    sig = {
        "ne_create": (P, [C.POINTER(Config)]),
        "ne_destroy": (None, [P]),
        "ne_last_error": (C.c_char_p, []),
        "ne_sync": (I, [P]),
        "ne_num_tensors": (I, [P]),
        "ne_tensor_numel": (L, [P, I]),
        "ne_set_tensor": (I, [P, I, I, P, C.c_size_t]),
        "ne_get_tensor": (I, [P, I, I, P, C.c_size_t]),
        "ne_train_step": (I, [P, P, F, P]),
        "ne_use_graphs": (I, [P, I]),
        "ne_overlap_weight_grads": (I, [P, I]),
        "ne_rmsnorm_bwd_formula": (I, [P, I]),
        "ne_optimizer_step": (I, [P, F, F, F, F, F, F, F, P]),
        "ne_zero_grads": (I, [P]),
        "ne_grad_scale_info": (I, [P, C.POINTER(C.c_float), C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
        "ne_grad_norm_parts": (I, [P, P]),
        "ne_step_stats": (I, [P, P]),
        "ne_get_state": (I, [P, C.POINTER(TrainState)]),
        "ne_set_state": (I, [P, C.POINTER(TrainState)]),
        "ne_load_ckpt_v4": (I, [P, C.c_char_p, C.POINTER(TrainState)]),
        "ne_save_ckpt_v4": (I, [P, C.c_char_p, C.POINTER(TrainState)]),
        "ne_decode": (I, [P, P, I, I, I, F, F, P, P]),
        "ne_decode_seeded": (I, [P, P, I, I, I, F, F, C.c_uint64, P]),
        "ne_mt19937_uniforms": (I, [C.c_uint64, L, P]),
        "ne_set_vocab_map": (I, [P, P, I]),
        "ne_prof_enable": (I, [P, I]),
        "ne_prof_reset": (I, [P]),
        "ne_prof_get": (I, [P, I, C.POINTER(C.c_double), C.POINTER(C.c_int64)]),
        "ne_timeline": (I, [P, I]),
        "ne_step_timeline": (I, [P, P, P, P]),
        "ne_update_launches": (I, [P]),
        "ne_k_rmsnorm_fwd": (I, [I, P, P, P, P, I, I, F, P]),
        "ne_k_rmsnorm_bwd": (I, [I, P, P, P, P, P, P, P, F, P, F, I, I, P]),
        "ne_k_gemm": (I, [I, I, I, I, I, I, P, L, P, L, P, L, P, L, F, P]),
        "ne_k_gemm_wgrad_group": (I, [I, I, P, P, I, P, P, P, P, P, I, F, P]),
        "ne_k_qk_prep_fwd": (I, [I, P, L, P, P, P, P, P, P, P, P, I, I, I, I, I, F, P]),
        "ne_k_qk_prep_bwd": (I, [I, P, P, P, L, P, P, P, P, P, P, P, P, P, F, I, I, I, I, I, P]),
        "ne_k_attn_fwd": (I, [I, P, L, P, L, P, L, P, L, P, I, I, I, I, I, F, P]),
        "ne_k_attn_bwd": (I, [I, P, L, P, L, P, L, P, L, P, P, L, P, P, L, P, L, P, L, I, I, I, I, I, F, P]),
        "ne_k_attn_bwd_noalloc": (I, [I, P, L, P, L, P, L, P, L, P, P, L, P, L, P, L, P, L, I, I, I, I, I, F, P]),
        "ne_k_ce_fwd": (I, [I, P, P, P, I, I, I, P, P, P, P, P, P]),
        "ne_k_ce_bwd": (I, [I, P, P, P, P, I, I, I, F, P, P]),
        "ne_k_ce_fwd_grad": (I, [I, P, P, P, I, I, I, P, P, P, P, P, F, P, P]),
        "ne_k_adam": (I, [I, P, P, P, P, P, L, L, F, F, F, F, F, I, P, I, P]),
        "ne_k_grad_norm": (I, [P, L, F, F, P, P, P, P]),
        "ne_k_embed_fwd": (I, [P, P, P, I, I, P]),
        "ne_k_embed_bwd": (I, [P, P, P, F, I, I, P]),
        "ne_k_swiglu_fwd": (I, [I, P, P, I, I, P]),
        "ne_k_mfma_ceiling": (I, [I, I, I, I, P, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(h, name)
        fn.restype = res
        fn.argtypes = args
    _lib = h
    return h


def check(rc: int, what: str = ""):
    if rc != 0:
        msg = lib().ne_last_error().decode(errors="replace")
        raise NEError(f"{what} failed ({rc}): {msg}")


def mt19937_uniforms(seed: int, n: int) -> np.ndarray:
    """ne_mt19937_uniforms: the draws numpy's RandomState(seed).random_sample(n) gives."""
    out = np.zeros(n, np.float64)
    check(lib().ne_mt19937_uniforms(seed, n, _ptr(out)), "mt19937_uniforms")
    return out


def tensor_names(n_layers: int, qk_norm: bool):
    names = [f"layers.{l}.{t}" for l in range(n_layers) for t in LAYER_TENSORS]
    names += ["rms_final", "embed"]
    if qk_norm:
        for l in range(n_layers):
            names += [f"layers.{l}.q_norm", f"layers.{l}.k_norm"]
    return names


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


class Model:
    """One device-resident model + optimizer state + activation workspace (ne_ctx)."""

    def __init__(self, dim, hidden, n_heads, kv_heads, head_dim, n_layers, vocab, seq, batch=1,
                 qk_norm=False, rope_theta=10000.0, res_alpha=1.0, norm_eps=1e-5,
                 decode_batch=0, decode_ctx=0, dtype=NE_FP16):
        self.cfg = Config(dim, hidden, n_heads, kv_heads, head_dim, n_layers, vocab, seq, batch,
                          int(bool(qk_norm)), rope_theta, res_alpha, norm_eps, decode_batch, decode_ctx,
                          dtype)
        self._h = lib().ne_create(C.byref(self.cfg))
        if not self._h:
            raise NEError("ne_create failed: " + lib().ne_last_error().decode(errors="replace"))
        self.names = tensor_names(n_layers, qk_norm)
        self.ids = {n: i for i, n in enumerate(self.names)}
        assert lib().ne_num_tensors(self._h) == len(self.names)

    @classmethod
    def from_oracle(cls, ocfg, batch=1, decode_batch=0, decode_ctx=0, dtype=NE_FP16):
        return cls(ocfg.dim, ocfg.hidden, ocfg.n_heads, ocfg.kv_heads, ocfg.head_dim, ocfg.n_layers,
                   ocfg.vocab, ocfg.seq, batch, ocfg.qk_norm, ocfg.rope_theta, ocfg.res_alpha,
                   ocfg.eps, decode_batch, decode_ctx, dtype)

    def close(self):
        if self._h:
            lib().ne_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._h

    def numel(self, name):
        return int(lib().ne_tensor_numel(self._h, self.ids[name]))

    def set(self, name, arr, kind=NE_PARAM):
        a = np.ascontiguousarray(arr, np.float32).reshape(-1)
        check(lib().ne_set_tensor(self._h, kind, self.ids[name], _ptr(a), a.size), f"set {name}")

    def get(self, name, kind=NE_PARAM):
        out = np.empty(self.numel(name), np.float32)
        check(lib().ne_get_tensor(self._h, kind, self.ids[name], _ptr(out), out.size), f"get {name}")
        return out

    def set_params(self, P: dict, kind=NE_PARAM):
        for n in self.names:
            if n in P:
                self.set(n, P[n], kind)

    def get_all(self, shapes: dict, kind=NE_PARAM):
        return {n: self.get(n, kind).reshape(shapes[n]) for n in self.names}

    def train_step(self, tokens: np.ndarray, loss_scale=1.0, want_loss=True):
        t = np.ascontiguousarray(tokens, np.int32)
        loss = C.c_float(0.0)
        check(lib().ne_train_step(self._h, _ptr(t), loss_scale, C.byref(loss) if want_loss else None),
              "train_step")
        return float(loss.value) if want_loss else None

    def optimizer_step(self, lr, b1=0.9, b2=0.95, eps=1e-8, wd=0.1, grad_scale=1.0, clip=1.0,
                       want_norm=True):
        """Returns the pre-clip grad norm (NaN when the step was skipped after an overflow)."""
        gn = C.c_float(0.0)
        rc = lib().ne_optimizer_step(self._h, lr, b1, b2, eps, wd, grad_scale, clip,
                                     C.byref(gn) if want_norm else None)
        if rc not in (0, 1):
            check(rc, "optimizer_step")
        return float(gn.value) if want_norm else None

    def grad_scale_info(self):
        """(internal gradient scale, skipped steps, overflow-site names of the last skip)"""
        sc, sk, st = C.c_float(0), C.c_int32(0), C.c_int32(0)
        check(lib().ne_grad_scale_info(self._h, C.byref(sc), C.byref(sk), C.byref(st)), "grad_scale_info")
        names = [n for i, n in enumerate(OVF_SITES) if st.value >> i & 1]
        return float(sc.value), int(sk.value), names

    def grad_norm_parts(self):
        """(global, attention, FFN, embedding) gradient norms of the last optimizer step."""
        out = np.zeros(4, np.float32)
        check(lib().ne_grad_norm_parts(self._h, _ptr(out)), "grad_norm_parts")
        return tuple(float(v) for v in out)

    def step_stats(self):
        """(x_min, x_max, dy_min, dy_max) of the last training step (reference scale)."""
        out = np.zeros(4, np.float32)
        check(lib().ne_step_stats(self._h, _ptr(out)), "step_stats")
        return tuple(float(v) for v in out)

    def use_graphs(self, on=True):
        check(lib().ne_use_graphs(self._h, int(on)), "use_graphs")

    def overlap_weight_grads(self, on=True):
        check(lib().ne_overlap_weight_grads(self._h, int(on)), "overlap_weight_grads")

    def rmsnorm_bwd_formula(self, ref=True):
        """ref=True: the reference's RMSNorm backward (extra gain factor on the projection
        term, TD/cpu_ops.h:108-261); False: the exact gradient (default)."""
        check(lib().ne_rmsnorm_bwd_formula(self._h, int(ref)), "rmsnorm_bwd_formula")

    def set_vocab_map(self, ids):
        """Vocabulary compaction: classifier + softmax over these embedding rows (None: all)."""
        if ids is None:
            check(lib().ne_set_vocab_map(self._h, None, 0), "set_vocab_map")
            return
        a = np.ascontiguousarray(ids, dtype=np.int32)
        check(lib().ne_set_vocab_map(self._h, a.ctypes.data_as(C.c_void_p), len(a)), "set_vocab_map")

    def zero_grads(self):
        check(lib().ne_zero_grads(self._h), "zero_grads")

    def sync(self):
        check(lib().ne_sync(self._h), "sync")

    def state(self):
        st = TrainState()
        check(lib().ne_get_state(self._h, C.byref(st)), "get_state")
        return st

    def set_state(self, st: TrainState):
        check(lib().ne_set_state(self._h, C.byref(st)), "set_state")

    def save(self, path, st: TrainState | None = None):
        check(lib().ne_save_ckpt_v4(self._h, str(path).encode(), C.byref(st) if st else None), "save")

    def load(self, path):
        st = TrainState()
        check(lib().ne_load_ckpt_v4(self._h, str(path).encode(), C.byref(st)), "load")
        return st

    def decode(self, prompt: np.ndarray, n_new: int, temperature=0.0, top_p=1.0, uniforms=None):
        p = np.ascontiguousarray(prompt, np.int32)
        B, P0 = p.shape
        out = np.zeros((B, n_new), np.int32)
        u = None
        if uniforms is not None:
            u = np.ascontiguousarray(uniforms, np.float64).reshape(B, n_new)
        check(lib().ne_decode(self._h, _ptr(p), B, P0, n_new, temperature, top_p,
                              _ptr(u) if u is not None else None, _ptr(out)), "decode")
        return out

    def decode_seeded(self, prompt: np.ndarray, n_new: int, temperature: float, top_p: float, seed: int):
        """ne_decode_seeded: sampling draws from MT19937(seed), as generate.py --seed."""
        p = np.ascontiguousarray(prompt, np.int32)
        B, P0 = p.shape
        out = np.zeros((B, n_new), np.int32)
        check(lib().ne_decode_seeded(self._h, _ptr(p), B, P0, n_new, temperature, top_p, seed, _ptr(out)),
              "decode_seeded")
        return out

    def prof_enable(self, families=PROF_FAMILIES):
        """Time the given families (names from PROF_FAMILIES) with HIP events; () disables."""
        mask = 0
        for f in families:
            mask |= 1 << PROF_FAMILIES.index(f)
        check(lib().ne_prof_enable(self._h, mask), "prof_enable")

    def prof_reset(self):
        check(lib().ne_prof_reset(self._h), "prof_reset")

    def timeline(self, on=True):
        """Record the step's phase boundaries with HIP events (ne_timeline)."""
        check(lib().ne_timeline(self._h, int(bool(on))), "timeline")

    def update_launches(self):
        """Launches of the AdamW pass a two-stream step runs beside its forward."""
        n = lib().ne_update_launches(self._h)
        if n < 0:
            raise NEError(lib().ne_last_error().decode())
        return n

    def step_timeline(self, layers=False):
        """Phases of the last step in ms (TIMELINE_PHASES), and with layers=True the per-layer
        forward and backward times."""
        out = np.zeros(len(TIMELINE_PHASES), np.float32)
        lf = np.zeros(self.cfg.n_layers, np.float32)
        lb = np.zeros(self.cfg.n_layers, np.float32)
        check(lib().ne_step_timeline(self._h, _ptr(out), _ptr(lf), _ptr(lb)), "step_timeline")
        ph = {k: float(v) for k, v in zip(TIMELINE_PHASES, out)}
        return (ph, lf, lb) if layers else ph

    def prof(self):
        out = {}
        for i, name in enumerate(PROF_FAMILIES):
            ms, cnt = C.c_double(0), C.c_int64(0)
            check(lib().ne_prof_get(self._h, i, C.byref(ms), C.byref(cnt)), "prof_get")
            out[name] = (ms.value, cnt.value)
        return out
