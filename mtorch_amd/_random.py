"""Seeded generation with mtorch's generator and host-side fp16 narrowing.

The generator lives in libmthip (host code): splitmix64 + Marsaglia polar normals with a
spare-normal cache, module.cpp:47-183, 245-274, 335-365.  Values are produced on the host in
the tensor's dtype, in logical element order, and then copied to the tensor's device, so a
seeded tensor is bit-identical to the one mtorch builds on the CPU.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from . import _tensor as T


class Generator:
    def __init__(self, device="cpu"):
        self._handle = _lib.lib().mthip_generator_create(0)
        if not self._handle:
            raise RuntimeError("could not create a generator")
        self._initial_seed = 0
        self.device = T.device(device)

    def __del__(self):
        try:
            h = getattr(self, "_handle", None)
            if h and _lib._lib is not None:
                _lib._lib.mthip_generator_destroy(h)
                self._handle = None
        except Exception:  # interpreter shutdown: module globals may already be gone
            pass

    def manual_seed(self, seed):
        seed = int(seed) & 0xFFFFFFFFFFFFFFFF
        _lib.check(_lib.lib().mthip_generator_seed(self._handle, seed))
        self._initial_seed = seed
        return self

    def initial_seed(self):
        return self._initial_seed

    def get_state(self):
        st, sp, sv = ctypes.c_uint64(), ctypes.c_int(), ctypes.c_double()
        _lib.check(_lib.lib().mthip_generator_get_state(self._handle, ctypes.byref(st), ctypes.byref(sp), ctypes.byref(sv)))
        return (st.value, sp.value, sv.value)

    def set_state(self, state):
        st, sp, sv = state
        _lib.check(_lib.lib().mthip_generator_set_state(self._handle, int(st), int(sp), float(sv)))
        return self


_default = None


def default_generator() -> Generator:
    global _default
    if _default is None:
        _default = Generator()
    return _default


def manual_seed(seed):
    """mtorch.manual_seed (module.cpp:2626): reseeds the global generator, clearing the spare."""
    return default_generator().manual_seed(seed)


def initial_seed():
    return default_generator().initial_seed()


def _fill_host(kind, dt, n, a, b, generator):
    gen = generator or default_generator()
    if dt not in (T.float16, T.float32, T.float64):
        raise ValueError(f"{kind} is only implemented for floating point tensors")
    host = np.empty(n, dtype=dt.np)
    fn = _lib.lib().mthip_rng_normal if kind == "normal_" else _lib.lib().mthip_rng_uniform
    _lib.check(fn(gen._handle, dt.code, host.ctypes.data if n else None, n, float(a), float(b)))
    return host


def _write_logical(t: "T.Tensor", host: np.ndarray):
    """Writes values given in logical (row-major) order into t, which may be a view."""
    sizes = list(t.shape)
    src = T.Tensor(T.Storage(t.dtype, host.size, T.device("cpu"), host=host), sizes, T.contiguous_strides(sizes))
    from . import _ops

    _ops.copy_into(t, src)


def normal_(t, mean=0.0, std=1.0, generator=None):
    n = t.numel()
    if n == 0:
        return t
    _write_logical(t, _fill_host("normal_", t.dtype, n, mean, std, generator))
    return t


def uniform_(t, a=0.0, b=1.0, generator=None):
    n = t.numel()
    if n == 0:
        return t
    _write_logical(t, _fill_host("uniform_", t.dtype, n, a, b, generator))
    return t


def _factory(kind, sizes, dtype, device, generator, requires_grad, a, b):
    if len(sizes) == 1 and isinstance(sizes[0], (list, tuple)):
        sizes = tuple(sizes[0])
    sizes = [int(s) for s in sizes]
    dt = T._as_dtype(dtype, T.float32)
    if not dt.is_floating_point:
        # py_randn / py_rand (module.cpp:2501-2530) raise NotImplementedError here.
        raise NotImplementedError(f"{'randn' if kind == 'normal_' else 'rand'} is only implemented for floating point dtypes")
    n = T._numel(sizes)
    host = _fill_host(kind, dt, n, a, b, generator) if n else np.empty(0, dtype=dt.np)
    t = T.Tensor(T.Storage(dt, n, T.device("cpu"), host=host), sizes, T.contiguous_strides(sizes))
    if device is not None and T.device(device).type != "cpu":
        t = t.to(device)
    t.requires_grad = requires_grad
    return t


def randn(*sizes, dtype=None, device=None, generator=None, requires_grad=False):
    """fill_randn_result (module.cpp:159-183)."""
    return _factory("normal_", sizes, dtype, device, generator, requires_grad, 0.0, 1.0)


def rand(*sizes, dtype=None, device=None, generator=None, requires_grad=False):
    return _factory("uniform_", sizes, dtype, device, generator, requires_grad, 0.0, 1.0)


# ------------------------------------------------------------------------------ host casts


def float_to_half_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> binary16 bits with mtorch's rounding (tensor.cpp:276-315), vectorised."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = x.view(np.uint32).astype(np.int64)
    sign = (bits >> 16) & 0x8000
    raw = (bits >> 23) & 0xFF
    man = bits & 0x7FFFFF
    e = raw - 112
    normal = (e << 10) + ((man + 0x1000) >> 13)
    normal = np.minimum(normal, 0x7C00)
    shift = np.clip(1 - e, 0, 63)
    sub = (((man | 0x800000) >> shift) + 0x1000) >> 13
    out = np.where(e > 0, normal, np.where(e < -10, 0, sub))
    payload = man >> 13
    nan_bits = 0x7C00 | np.where(man == 0, 0, np.where(payload == 0, 0x200, payload))
    out = np.where(raw == 0xFF, nan_bits, out)
    return (sign | out).astype(np.uint16)


def half_bits_to_float(h: np.ndarray) -> np.ndarray:
    """binary16 bits -> float32, exact (tensor.cpp:317-344) including NaN payloads."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    f = h.view(np.float16).astype(np.float32)
    exp_all_ones = (h & 0x7C00) == 0x7C00
    if exp_all_ones.any():
        special = ((h.astype(np.uint32) & 0x8000) << 16) | 0x7F800000 | ((h.astype(np.uint32) & 0x3FF) << 13)
        f = np.where(exp_all_ones, special.view(np.float32), f)
    return f


def host_cast(values: np.ndarray, src: "T.dtype", dst: "T.dtype") -> np.ndarray:
    """Element-wise dtype conversion of a CPU buffer, as mtorch's try_dense_cast
    (tensor.cpp:2764-2796): widen to double, narrow per storage_set_unchecked (:593-614)."""
    if src is dst:
        return values.copy()
    if src is T.float16:
        wide = half_bits_to_float(values).astype(np.float64)
    elif src is T.bool_:
        wide = (values != 0).astype(np.float64)
    else:
        wide = values.astype(np.float64)
    if dst is T.float16:
        return float_to_half_bits(wide.astype(np.float32))
    if dst is T.bool_:
        return (wide != 0).astype(np.uint8)
    if dst in (T.int32, T.int64):
        with np.errstate(invalid="ignore"):
            return np.trunc(wide).astype(dst.np)
    return wide.astype(dst.np)
