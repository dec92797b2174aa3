"""CPU oracle for mtorch's SD-UNet hot path -- TEST INFRASTRUCTURE ONLY.

ctypes wrapper over liboracle.so (oracle.c), a plain-C restatement of the reference's x86-64
Linux CPU path; see oracle.h for the per-function citations.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may use it, and only as the checker:
the product (mtorch_amd + libmthip) never imports it.

Arrays: fp32 as numpy float32; fp16 as numpy uint16 bit patterns (use h2f/f2h to convert).

Parity pins (what fixes each function besides this restatement): see tests/test_oracle_*.py.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_DIR, "liboracle.so")
F16, F32 = 0, 1

_lib = None


def build() -> None:
    subprocess.run(["make", "-C", _DIR, "-s"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, i32, dbl = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double
        L.orc_f2h.restype = ctypes.c_uint16
        L.orc_f2h.argtypes = [ctypes.c_float]
        L.orc_h2f.restype = ctypes.c_float
        L.orc_h2f.argtypes = [ctypes.c_uint16]
        L.orc_f2h_array.argtypes = [vp, vp, i64]
        L.orc_h2f_array.argtypes = [vp, vp, i64]
        L.orc_rng_seed.argtypes = [vp, ctypes.c_uint64]
        L.orc_rng_next_u64.restype = ctypes.c_uint64
        L.orc_rng_next_u64.argtypes = [vp]
        L.orc_rng_uniform_open.restype = dbl
        L.orc_rng_uniform_open.argtypes = [vp]
        L.orc_rng_normal_pair.argtypes = [vp, ctypes.POINTER(dbl), ctypes.POINTER(dbl)]
        L.orc_rng_next_normal.restype = dbl
        L.orc_rng_next_normal.argtypes = [vp]
        for name in ("orc_fill_normal_f32", "orc_fill_normal_f16", "orc_fill_uniform_f32", "orc_fill_uniform_f16"):
            getattr(L, name).argtypes = [vp, vp, i64, dbl, dbl]
        L.orc_linear.argtypes = [i32, vp, vp, vp, vp, i64, i64, i64]
        L.orc_matmul.argtypes = [i32, vp, vp, vp, i64, i64, i64, i64, i64, i64]
        L.orc_addmm.argtypes = [i32, vp, vp, vp, vp, i64, i64, i64, dbl, dbl]
        L.orc_conv2d.argtypes = [i32, vp, vp, vp, vp] + [i64] * 14
        L.orc_conv2d_out_size.restype = i64
        L.orc_conv2d_out_size.argtypes = [i64] * 5
        L.orc_sdpa.argtypes = [i32, vp, vp, vp, vp, i64, i64, i64, i64, i64, i32, vp, i32, i32, dbl]
        L.orc_group_norm.argtypes = [i32, vp, vp, vp, vp, i64, i64, i64, i64, dbl]
        L.orc_layer_norm.argtypes = [i32, vp, vp, vp, vp, i64, i64, dbl]
        L.orc_softmax_lastdim.argtypes = [i32, vp, vp, i64, i64, i32]
        L.orc_softmax_generic.argtypes = [i32, vp, i32, vp, i64, i64]
        L.orc_gelu.argtypes = [i32, vp, vp, i64, i32]
        L.orc_fast_erf_float.restype = ctypes.c_float
        L.orc_fast_erf_float.argtypes = [ctypes.c_float]
        L.orc_gelu_unit_polynomial_float.restype = ctypes.c_float
        L.orc_gelu_unit_polynomial_float.argtypes = [ctypes.c_float]
        L.orc_silu.argtypes = [i32, vp, vp, i64]
        L.orc_binary.argtypes = [i32, i32, vp, vp, vp, i64]
        for fn in ("orc_linear", "orc_matmul", "orc_addmm", "orc_conv2d", "orc_sdpa", "orc_group_norm",
                   "orc_layer_norm", "orc_softmax_lastdim", "orc_softmax_generic", "orc_gelu", "orc_silu", "orc_binary"):
            getattr(L, fn).restype = i32
        _lib = L
    return _lib


# ------------------------------------------------------------------------------ helpers


def _dt(a: np.ndarray) -> int:
    if a.dtype == np.uint16:
        return F16
    if a.dtype == np.float32:
        return F32
    raise TypeError(f"oracle arrays must be float32 or uint16 (fp16 bits), got {a.dtype}")


def _c(a):
    return None if a is None else np.ascontiguousarray(a)


def _p(a):
    return None if a is None else a.ctypes.data


def f2h(x) -> np.ndarray:
    shape = np.shape(x)  # ascontiguousarray lifts 0-dim inputs to 1-dim
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(shape, np.uint16)
    lib().orc_f2h_array(x.ctypes.data, out.ctypes.data, x.size)
    return out


def h2f(h) -> np.ndarray:
    shape = np.shape(h)
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(shape, np.float32)
    lib().orc_h2f_array(h.ctypes.data, out.ctypes.data, h.size)
    return out


class Rng:
    """mtorch's generator state (module.cpp:47-51) driven by the oracle."""

    class _State(ctypes.Structure):
        _fields_ = [("state", ctypes.c_uint64), ("has_spare_normal", ctypes.c_int), ("spare_normal", ctypes.c_double)]

    def __init__(self, seed=0):
        self.s = Rng._State()
        lib().orc_rng_seed(ctypes.byref(self.s), seed)

    def seed(self, seed):
        lib().orc_rng_seed(ctypes.byref(self.s), seed)

    def next_u64(self):
        return lib().orc_rng_next_u64(ctypes.byref(self.s))

    def uniform_open(self):
        return lib().orc_rng_uniform_open(ctypes.byref(self.s))

    def normal_pair(self):
        a, b = ctypes.c_double(), ctypes.c_double()
        lib().orc_rng_normal_pair(ctypes.byref(self.s), ctypes.byref(a), ctypes.byref(b))
        return a.value, b.value

    def next_normal(self):
        return lib().orc_rng_next_normal(ctypes.byref(self.s))

    def randn(self, shape, dtype="float32", mean=0.0, std=1.0):
        n = int(np.prod(shape))
        if dtype == "float16":
            out = np.empty(n, np.uint16)
            lib().orc_fill_normal_f16(ctypes.byref(self.s), out.ctypes.data, n, mean, std)
        else:
            out = np.empty(n, np.float32)
            lib().orc_fill_normal_f32(ctypes.byref(self.s), out.ctypes.data, n, mean, std)
        return out.reshape(shape)

    def uniform(self, shape, a, b, dtype="float32"):
        n = int(np.prod(shape))
        if dtype == "float16":
            out = np.empty(n, np.uint16)
            lib().orc_fill_uniform_f16(ctypes.byref(self.s), out.ctypes.data, n, a, b)
        else:
            out = np.empty(n, np.float32)
            lib().orc_fill_uniform_f32(ctypes.byref(self.s), out.ctypes.data, n, a, b)
        return out.reshape(shape)


# ------------------------------------------------------------------------------ ops


def linear(x, w, b=None):
    x, w, b = _c(x), _c(w), _c(b)
    K = x.shape[-1]
    N = w.shape[0]
    M = x.size // K if K else 0
    y = np.empty(x.shape[:-1] + (N,), x.dtype)
    lib().orc_linear(_dt(x), _p(x), _p(w), _p(b), _p(y), M, N, K)
    return y


def matmul(a, b):
    """[batch?, M, K] @ [batch?, K, N] (same batch or batch of 1)."""
    a, b = _c(a), _c(b)
    a3 = a.reshape((-1,) + a.shape[-2:])
    b3 = b.reshape((-1,) + b.shape[-2:])
    batch = max(a3.shape[0], b3.shape[0])
    M, K = a3.shape[1:]
    N = b3.shape[2]
    c = np.empty((batch, M, N), a.dtype)
    lib().orc_matmul(_dt(a), _p(a3), _p(b3), _p(c), batch, M, N, K, 0 if a3.shape[0] == 1 else M * K,
                     0 if b3.shape[0] == 1 else K * N)
    lead = a.shape[:-2] if a3.shape[0] == batch else b.shape[:-2]
    return c.reshape(lead + (M, N))


def addmm(inp, m1, m2, beta=1.0, alpha=1.0):
    m1, m2 = _c(m1), _c(m2)
    M, K = m1.shape
    N = m2.shape[1]
    full = np.ascontiguousarray(np.broadcast_to(inp, (M, N)))
    out = np.empty((M, N), m1.dtype)
    lib().orc_addmm(_dt(m1), _p(full), _p(m1), _p(m2), _p(out), M, N, K, beta, alpha)
    return out


def conv2d(x, w, b=None, stride=1, padding=0, dilation=1, groups=1):
    x, w, b = _c(x), _c(w), _c(b)
    pair = lambda v: (v, v) if isinstance(v, int) else tuple(v)  # noqa: E731
    sh, sw = pair(stride)
    ph, pw = pair(padding)
    dh, dw = pair(dilation)
    B, C, H, W = x.shape
    O, _, KH, KW = w.shape
    OH = lib().orc_conv2d_out_size(H, KH, sh, ph, dh)
    OW = lib().orc_conv2d_out_size(W, KW, sw, pw, dw)
    y = np.empty((B, O, OH, OW), x.dtype)
    rc = lib().orc_conv2d(_dt(x), _p(x), _p(w), _p(b), _p(y), B, C, H, W, O, KH, KW, sh, sw, ph, pw, dh, dw, groups)
    assert rc == 0
    return y


def sdpa(q, k, v, mask=None, is_causal=False, scale=None):
    """q[..., Lq, E], k[..., Lk, E], v[..., Lk, Ev]; mask broadcastable to [..., Lq, Lk]
    (bool -> keep where True; float32 -> added).  scale=None is 1/sqrt(E); any other value,
    zero and negative ones included, multiplies the scores as given (tensor.cpp:31019)."""
    q, k, v = _c(q), _c(k), _c(v)
    lead = q.shape[:-2]
    P = int(np.prod(lead)) if lead else 1
    Lq, E = q.shape[-2:]
    Lk, Ev = v.shape[-2:]
    o = np.empty(lead + (Lq, Ev), q.dtype)
    kind, mp = 0, None
    if mask is not None:
        m = np.ascontiguousarray(np.broadcast_to(mask, lead + (Lq, Lk)))
        if m.dtype == np.bool_:
            m = m.astype(np.uint8)
            kind = 1
        else:
            m = m.astype(np.float32)
            kind = 2
        mp = m
    lib().orc_sdpa(_dt(q), _p(q), _p(k), _p(v), _p(o), P, Lq, Lk, E, Ev, kind, _p(mp), 1 if is_causal else 0,
                   0 if scale is None else 1, 0.0 if scale is None else float(scale))
    return o


def group_norm(x, groups, weight=None, bias=None, eps=1e-5):
    x, weight, bias = _c(x), _c(weight), _c(bias)
    B, C = x.shape[:2]
    inner = int(np.prod(x.shape[2:])) if x.ndim > 2 else 1
    y = np.empty_like(x)
    lib().orc_group_norm(_dt(x), _p(x), _p(weight), _p(bias), _p(y), B, C, inner, groups, eps)
    return y


def layer_norm(x, n, weight=None, bias=None, eps=1e-5):
    x, weight, bias = _c(x), _c(weight), _c(bias)
    y = np.empty_like(x)
    lib().orc_layer_norm(_dt(x), _p(x), _p(weight), _p(bias), _p(y), x.size // n, n, eps)
    return y


def softmax_lastdim(x):
    x = _c(x)
    cols = x.shape[-1]
    y = np.empty_like(x)
    lib().orc_softmax_lastdim(_dt(x), _p(x), _p(y), x.size // cols, cols, x.ndim)
    return y


def softmax_generic(x, out_dtype):
    """softmax over the last dim with the output dtype ("float16"/"float32") differing from the
    input's: the reference's generic double path."""
    x = _c(x)
    cols = x.shape[-1]
    y = np.empty(x.shape, np.uint16 if out_dtype == "float16" else np.float32)
    lib().orc_softmax_generic(_dt(x), _p(x), 0 if out_dtype == "float16" else 1, _p(y), x.size // cols, cols)
    return y


def gelu(x, approximate="none"):
    x = _c(x)
    y = np.empty_like(x)
    lib().orc_gelu(_dt(x), _p(x), _p(y), x.size, 0 if approximate == "none" else 1)
    return y


def silu(x):
    x = _c(x)
    y = np.empty_like(x)
    lib().orc_silu(_dt(x), _p(x), _p(y), x.size)
    return y


def binary(a, b, op):
    a, b = np.broadcast_arrays(a, b)
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    y = np.empty_like(a)
    lib().orc_binary(_dt(a), {"add": 0, "mul": 1, "sub": 2}[op], _p(a), _p(b), _p(y), a.size)
    return y
