"""Device-memory plumbing for the GPU tests (torch allocates, the C-ABI computes)."""
import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import ne  # noqa: E402


def need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def dev(a, dtype=None):
    t = torch.as_tensor(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda().contiguous()


def zeros(shape, dtype=torch.float32):
    return torch.zeros(shape, dtype=dtype, device="cuda")


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def host(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def call(fn, *args):
    rc = fn(*args)
    if rc != 0:
        raise ne.NEError(f"{fn.__name__}: {rc}: {ne.lib().ne_last_error().decode()}")
    torch.cuda.synchronize()


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def bf16_round(a):
    return torch.as_tensor(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).float().numpy()
