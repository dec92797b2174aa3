"""Tensor, dtype and device for the mtorch_amd surface.

A Tensor is (storage, sizes, strides, offset, dtype) exactly as mtorch's core models it
(tensor.h:60-126).  Storage is either a host numpy buffer (device "cpu") or a block of device
memory from libmthip's caching allocator (device "cuda").  Views share storage; shape/stride
arithmetic follows the reference so metadata matches bit for bit:

- contiguous strides and is_contiguous: tensor.cpp:8368-8376, 8133-8135
- reshape view-stride solver:           tensor.cpp:8533-8612
- transpose / permute:                  tensor.cpp:8653, 8680
- unsqueeze / squeeze / narrow / select: tensor.cpp:12043-12107
- split / chunk:                        tensor.cpp:12519-12584
- expand:                               tensor.cpp:8820

Compute on device tensors is implemented in _ops; the host side only creates, converts and
moves data (factories, the seeded generator, dtype casts, .to()).
"""

from __future__ import annotations

import builtins as _builtins
import ctypes
import math
import threading

import numpy as np

from . import _lib

# ------------------------------------------------------------------------------ dtypes


class dtype:
    __slots__ = ("name", "code", "itemsize", "np", "is_floating_point")

    def __init__(self, name, code, itemsize, np_dtype, is_float):
        self.name = name
        self.code = code
        self.itemsize = itemsize
        self.np = np.dtype(np_dtype)
        self.is_floating_point = is_float

    def __repr__(self):
        return f"mtorch_amd.{self.name}"

    __str__ = __repr__

    def __reduce__(self):
        return (_dtype_by_name, (self.name,))


float16 = dtype("float16", _lib.F16, 2, np.uint16, True)  # stored as IEEE binary16 bit patterns
float32 = dtype("float32", _lib.F32, 4, np.float32, True)
float64 = dtype("float64", _lib.F64, 8, np.float64, True)
int32 = dtype("int32", _lib.I32, 4, np.int32, False)
int64 = dtype("int64", _lib.I64, 8, np.int64, False)
bool_ = dtype("bool", _lib.BOOL, 1, np.uint8, False)
half = float16
float = float32  # noqa: A001 - mirrors the reference's aliases
double = float64
long = int64
int = int32  # noqa: A001

_DTYPES = {d.name: d for d in (float16, float32, float64, int32, int64, bool_)}
_BY_CODE = {d.code: d for d in _DTYPES.values()}


def _dtype_by_name(name):
    return _DTYPES[name]


def _as_dtype(value, default=None):
    """Parses a dtype argument the way the reference binding does (module.cpp:820-868)."""
    if value is None:
        return default
    if isinstance(value, dtype):
        return value
    text = value if isinstance(value, str) else getattr(value, "name", str(value))
    text = str(text)
    if "float16" in text or text == "half":
        return float16
    if "float64" in text or "double" in text:
        return float64
    if "int32" in text:
        return int32
    if "int64" in text or "long" in text:
        return int64
    if "bool" in text:
        return bool_
    return float32


def promote_types(a: dtype, b: dtype) -> dtype:
    """promote_dtype (tensor.cpp): bool < int32 < int64 < float16 < float32 < float64."""
    order = [bool_, int32, int64, float16, float32, float64]
    return a if order.index(a) >= order.index(b) else b


# ------------------------------------------------------------------------------ devices


class device(str):
    """Device spec: "cpu", "cuda[:i]" (the MI355X backend; "hip" is an alias).

    The reference accepts only cpu/mps and rejects "cuda" (mtorch/__init__.py:33-45); this
    backend adds the GPU type.  "metal" parses to "mps" as in the reference, and, as there,
    only creating storage on it raises NotImplementedError (no Apple GPU on this platform).
    """

    def __new__(cls, spec="cpu", index=None):
        if isinstance(spec, device) and index is None:
            return spec
        if isinstance(spec, _builtins.int):
            spec = f"cuda:{spec}"
        text = str(spec)
        kind, _, idx = text.partition(":")
        if kind == "hip":
            kind = "cuda"
        if kind == "metal":
            kind = "mps"
        if kind not in {"cpu", "cuda", "mps"}:
            raise NotImplementedError(f"{kind!r} device is not implemented")
        if index is not None:
            idx = str(index)
        if kind == "cuda" and not idx:
            idx_val = None
        else:
            idx_val = _builtins.int(idx) if idx else None
        normalized = kind if idx_val is None else f"{kind}:{idx_val}"
        obj = str.__new__(cls, normalized)
        obj.type = kind
        obj.index = idx_val
        return obj

    def __repr__(self):
        if self.index is None:
            return f"device(type='{self.type}')"
        return f"device(type='{self.type}', index={self.index})"

    def __str__(self):
        return self.type if self.index is None else f"{self.type}:{self.index}"

    def __eq__(self, other):
        if isinstance(other, str):
            try:
                other = device(other)
            except NotImplementedError:
                return False
            return self.type == other.type and _device_index(self) == _device_index(other)
        return NotImplemented

    def __hash__(self):
        return hash((self.type, _device_index(self)))


def _device_index(d: device):
    if d.type == "cpu":
        return None
    return 0 if d.index is None else d.index


# ------------------------------------------------------------------------------ grad mode

_grad_state = threading.local()


def is_grad_enabled() -> bool:
    return getattr(_grad_state, "enabled", True)


def set_grad_enabled(mode) -> bool:
    previous = is_grad_enabled()
    _grad_state.enabled = _builtins.bool(mode)
    return previous


class _GradMode:
    """Context manager / decorator, as the reference's _GradModeContext (mtorch/__init__.py:1959-1998)."""

    def __init__(self, mode):
        self.mode = _builtins.bool(mode)
        self.previous = None

    def __enter__(self):
        self.previous = set_grad_enabled(self.mode)
        return self

    def __exit__(self, *exc):
        set_grad_enabled(self.previous)
        return False

    def __call__(self, func):
        import functools

        @functools.wraps(func)
        def wrapped(*args, **kwargs):
            with _GradMode(self.mode):
                return func(*args, **kwargs)

        return wrapped


def no_grad():
    return _GradMode(False)


def enable_grad():
    return _GradMode(True)


# ------------------------------------------------------------------------------ storage


class _DeviceBuffer:
    """A device allocation owned by the library's caching allocator; freed on collection."""

    __slots__ = ("ptr", "nbytes", "device")

    def __init__(self, nbytes: _builtins.int, dev: _builtins.int):
        lib = _lib.lib()
        out = ctypes.c_void_p()
        _lib.check(lib.mthip_malloc(dev, _builtins.max(nbytes, 1), ctypes.byref(out)))
        self.ptr = out.value
        self.nbytes = nbytes
        self.device = dev

    def __del__(self):
        try:
            if self.ptr and _lib._lib is not None:
                _lib._lib.mthip_free(self.device, self.ptr)
                self.ptr = None
        except Exception:  # interpreter shutdown: module globals may already be gone
            pass


class Storage:
    """Bytes shared by views (tensor.h:60-85).  `version` counts in-place writes; `packs` holds
    derived device layouts of this storage (the packed conv weight), each tagged with the
    version it was built from -- the device counterpart of the reference's per-Storage weight
    caches (tensor.h:65-78)."""

    __slots__ = ("dtype", "device", "numel", "host", "buf", "version", "packs")

    def __init__(self, dt: dtype, numel: _builtins.int, dev: device, host=None, zero=False):
        self.dtype = dt
        self.device = dev
        self.numel = numel
        self.version = 0
        self.packs = None
        if dev.type == "mps":
            raise NotImplementedError("'mps' device storage is not implemented")
        if dev.type == "cpu":
            self.host = host if host is not None else (np.zeros(numel, dtype=dt.np) if zero else np.empty(numel, dtype=dt.np))
            self.buf = None
        else:
            self.host = None
            self.buf = _DeviceBuffer(numel * dt.itemsize, _device_index(dev))
            if zero and numel:
                _lib.check(_lib.lib().mthip_fill(self.buf.device, dt.code, self.buf.ptr, numel, 0.0))

    @property
    def ptr(self):
        return self.buf.ptr if self.buf is not None else self.host.ctypes.data


def contiguous_strides(sizes):
    strides = [1] * len(sizes)
    running = 1
    for i in range(len(sizes) - 1, -1, -1):
        strides[i] = running
        running *= _builtins.max(sizes[i], 1)
    return strides


def _numel(sizes):
    n = 1
    for s in sizes:
        n *= s
    return n


def _positive_dim(dim, rank):
    if rank == 0:
        rank = 1
    if dim < -rank or dim >= rank:
        raise IndexError("dimension out of range")
    return dim + rank if dim < 0 else dim


def _broadcast_shape(a, b):
    out = []
    for i in range(_builtins.max(len(a), len(b))):
        x = a[len(a) - 1 - i] if i < len(a) else 1
        y = b[len(b) - 1 - i] if i < len(b) else 1
        if x != y and x != 1 and y != 1:
            raise ValueError("shapes are not broadcastable")
        out.append(y if x == 1 else x)
    return out[::-1]


# ------------------------------------------------------------------------------ Tensor


class Tensor:
    __slots__ = ("_storage", "_sizes", "_strides", "_offset", "_dtype", "_requires_grad", "__weakref__", "__dict__")

    def __init__(self, storage: Storage, sizes, strides, offset=0, requires_grad=False):
        self._storage = storage
        self._sizes = list(sizes)
        self._strides = list(strides)
        self._offset = offset
        self._dtype = storage.dtype
        self._requires_grad = _builtins.bool(requires_grad)

    # ---- metadata -----------------------------------------------------------------------
    @property
    def shape(self):
        return Size(self._sizes)

    def size(self, dim=None):
        if dim is None:
            return Size(self._sizes)
        return self._sizes[_positive_dim(dim, len(self._sizes))]

    def stride(self, dim=None):
        if dim is None:
            return tuple(self._strides)
        return self._strides[_positive_dim(dim, len(self._sizes))]

    def storage_offset(self):
        return self._offset

    @property
    def dtype(self):
        return self._dtype

    @property
    def device(self):
        return self._storage.device

    @property
    def is_cuda(self):
        return self._storage.device.type == "cuda"

    @property
    def ndim(self):
        return len(self._sizes)

    def dim(self):
        return len(self._sizes)

    def numel(self):
        return _numel(self._sizes)

    def element_size(self):
        return self._dtype.itemsize

    def is_contiguous(self, memory_format=None):
        return self._strides == contiguous_strides(self._sizes)

    def is_floating_point(self):
        return self._dtype.is_floating_point

    @property
    def requires_grad(self):
        return self._requires_grad

    @requires_grad.setter
    def requires_grad(self, value):
        self._requires_grad = _builtins.bool(value)

    def requires_grad_(self, value=True):
        self._requires_grad = _builtins.bool(value)
        return self

    def detach(self):
        return Tensor(self._storage, self._sizes, self._strides, self._offset, False)

    def data_ptr(self):
        return self._storage.ptr + self._offset * self._dtype.itemsize

    def _dev(self):
        return _device_index(self._storage.device)

    def __len__(self):
        if not self._sizes:
            raise TypeError("len() of a 0-d tensor")
        return self._sizes[0]

    # ---- host access --------------------------------------------------------------------
    def _host_view(self):
        """numpy view (CPU tensors) with this tensor's sizes/strides, in storage dtype."""
        host = self._storage.host
        itemsize = self._dtype.itemsize
        return np.lib.stride_tricks.as_strided(
            host[self._offset:],
            shape=tuple(self._sizes),
            strides=tuple(s * itemsize for s in self._strides),
            writeable=False,
        )

    def numpy(self):
        """Values as a numpy array (fp16 as numpy float16 by value)."""
        t = self if self.device.type == "cpu" else self.cpu()
        arr = np.ascontiguousarray(t._host_view()).reshape(tuple(t._sizes))  # keeps 0-dim shapes
        if t._dtype is float16:
            return arr.view(np.float16).copy()
        if t._dtype is bool_:
            return arr.astype(np.bool_)
        return arr.copy()

    def half_bits(self):
        """fp16 tensors: raw IEEE binary16 bit patterns as a contiguous uint16 numpy array."""
        if self._dtype is not float16:
            raise TypeError("half_bits() expects a float16 tensor")
        t = self if self.device.type == "cpu" else self.cpu()
        return np.ascontiguousarray(t._host_view()).reshape(tuple(t._sizes)).copy()

    def tolist(self):
        arr = self.numpy()
        return arr.tolist()

    def item(self):
        if self.numel() != 1:
            raise ValueError("only one element tensors can be converted to Python scalars")
        return self.numpy().reshape(-1)[0].item()

    def __float__(self):
        return _builtins.float(self.item())

    def __int__(self):
        return _builtins.int(self.item())

    def __repr__(self):
        dev = "" if self.device.type == "cpu" else f", device='{self.device}'"
        try:
            body = np.array2string(self.numpy(), precision=4, threshold=64)
        except Exception:  # pragma: no cover - repr must not raise
            body = "<unavailable>"
        return f"tensor({body}, dtype={self._dtype}{dev})"

    # ---- conversion ---------------------------------------------------------------------
    def to(self, *args, **kwargs):
        """Tensor.to(device), .to(dtype), .to(device, dtype), .to(other) (module.cpp:9262-9275)."""
        dev = kwargs.pop("device", None)
        dt = kwargs.pop("dtype", None)
        copy = kwargs.pop("copy", False)
        kwargs.pop("non_blocking", None)
        kwargs.pop("memory_format", None)
        if kwargs:
            raise TypeError(f"to() got unexpected keyword arguments {sorted(kwargs)}")
        for a in args:
            if isinstance(a, Tensor):
                dev, dt = a.device, a.dtype
            elif isinstance(a, dtype):
                dt = a
            elif isinstance(a, (str, device, _builtins.int)) and not (isinstance(a, str) and a in _DTYPES):
                dev = a
            elif isinstance(a, str):
                dt = _DTYPES[a]
            elif a is not None:
                raise TypeError(f"to() received an invalid argument {a!r}")
        target_dev = self.device if dev is None else device(dev)
        target_dt = self._dtype if dt is None else _as_dtype(dt)
        from . import _ops

        return _ops.to(self, target_dt, target_dev, copy)

    def cuda(self, device_index=None):
        return self.to(device("cuda" if device_index is None else f"cuda:{device_index}"))

    def cpu(self):
        return self.to(device("cpu"))

    def half(self):
        return self.to(float16)

    def float(self):
        return self.to(float32)

    def double(self):
        return self.to(float64)

    def type(self, dt=None):
        if dt is None:
            return f"mtorch_amd.{self._dtype.name}"
        return self.to(_as_dtype(dt))

    def contiguous(self, memory_format=None):
        if self.is_contiguous():
            return self
        from . import _ops

        return _ops.contiguous_copy(self)

    def clone(self, memory_format=None):
        from . import _ops

        return _ops.contiguous_copy(self)

    # ---- views --------------------------------------------------------------------------
    def _view(self, sizes, strides, offset=None):
        return Tensor(self._storage, sizes, strides, self._offset if offset is None else offset, self._requires_grad)

    def _resolve_sizes(self, sizes):
        if len(sizes) == 1 and isinstance(sizes[0], (list, tuple, Size)):
            sizes = tuple(sizes[0])
        sizes = [_builtins.int(s) for s in sizes]
        n = self.numel()
        if sizes.count(-1) > 1:
            raise ValueError("only one dimension can be inferred")
        if -1 in sizes:
            known = 1
            for s in sizes:
                if s != -1:
                    known *= s
            if known == 0 or n % known != 0:
                raise ValueError(f"shape '{sizes}' is invalid for input of size {n}")
            sizes[sizes.index(-1)] = n // known
        if _numel(sizes) != n:
            raise ValueError(f"shape '{sizes}' is invalid for input of size {n}")
        return sizes

    def _reshape_view_strides(self, resolved):
        """compute_reshape_view_strides (tensor.cpp:8533-8582): strides of a view, or None."""
        if self.numel() == 0:
            return None
        if not self._sizes:
            return contiguous_strides(resolved)
        new_strides = [0] * len(resolved)
        view_dim = len(resolved) - 1
        chunk_base = self._strides[-1]
        tensor_numel = 1
        view_numel = 1
        for tdim in range(len(self._sizes) - 1, -1, -1):
            tensor_numel *= self._sizes[tdim]
            boundary = tdim == 0 or (
                self._sizes[tdim - 1] != 1 and self._strides[tdim - 1] != tensor_numel * chunk_base
            )
            if not boundary:
                continue
            while view_dim >= 0 and (view_numel < tensor_numel or resolved[view_dim] == 1):
                new_strides[view_dim] = view_numel * chunk_base
                view_numel *= resolved[view_dim]
                view_dim -= 1
            if view_numel != tensor_numel:
                return None
            if tdim > 0:
                chunk_base = self._strides[tdim - 1]
                tensor_numel = 1
                view_numel = 1
        while view_dim >= 0:
            if resolved[view_dim] != 1:
                return None
            new_strides[view_dim] = 1
            view_dim -= 1
        return new_strides

    def reshape(self, *sizes):
        resolved = self._resolve_sizes(sizes)
        if self.is_contiguous():
            return self._view(resolved, contiguous_strides(resolved))
        strides = self._reshape_view_strides(resolved)
        if strides is not None:
            return self._view(resolved, strides)
        c = self.contiguous()
        return c._view(resolved, contiguous_strides(resolved))

    def view(self, *sizes):
        if len(sizes) == 1 and isinstance(sizes[0], dtype):
            raise NotImplementedError("view(dtype) is not supported")
        resolved = self._resolve_sizes(sizes)
        if self.is_contiguous():
            return self._view(resolved, contiguous_strides(resolved))
        strides = self._reshape_view_strides(resolved)
        if strides is None:
            raise RuntimeError("view size is not compatible with input tensor's size and stride")
        return self._view(resolved, strides)

    def flatten(self, start_dim=0, end_dim=-1):
        if not self._sizes:
            return self.reshape(1)
        s = _positive_dim(start_dim, self.dim())
        e = _positive_dim(end_dim, self.dim())
        if s > e:
            raise ValueError("flatten() has invalid args: start_dim cannot come after end_dim")
        sizes = self._sizes[:s] + [_numel(self._sizes[s:e + 1])] + self._sizes[e + 1:]
        return self.reshape(sizes)

    def unflatten(self, dim, sizes):
        d = _positive_dim(dim, self.dim())
        sizes = list(sizes)
        if -1 in sizes:
            known = _numel([x for x in sizes if x != -1])
            sizes[sizes.index(-1)] = self._sizes[d] // known
        return self.reshape(self._sizes[:d] + sizes + self._sizes[d + 1:])

    def transpose(self, dim0, dim1):
        rank = self.dim()
        d0, d1 = _positive_dim(dim0, rank), _positive_dim(dim1, rank)
        sizes, strides = list(self._sizes), list(self._strides)
        if rank:
            sizes[d0], sizes[d1] = sizes[d1], sizes[d0]
            strides[d0], strides[d1] = strides[d1], strides[d0]
        return self._view(sizes, strides)

    def t(self):
        if self.dim() > 2:
            raise ValueError("t() expects a tensor with <= 2 dimensions")
        return self.transpose(0, 1) if self.dim() == 2 else self

    @property
    def T(self):
        return self.permute(*reversed(range(self.dim())))

    def permute(self, *dims):
        if len(dims) == 1 and isinstance(dims[0], (list, tuple)):
            dims = tuple(dims[0])
        rank = self.dim()
        dims = [_positive_dim(d, rank) for d in dims]
        if sorted(dims) != list(range(rank)):
            raise ValueError("permute dims must be a permutation of the tensor dimensions")
        return self._view([self._sizes[d] for d in dims], [self._strides[d] for d in dims])

    def unsqueeze(self, dim):
        rank = self.dim() + 1
        if dim < 0:
            dim += rank
        if dim < 0 or dim > self.dim():
            raise IndexError("dimension out of range")
        stride = 1 if dim >= self.dim() else self._strides[dim] * self._sizes[dim]
        sizes = self._sizes[:dim] + [1] + self._sizes[dim:]
        strides = self._strides[:dim] + [stride] + self._strides[dim:]
        return self._view(sizes, strides)

    def squeeze(self, dim=None):
        if dim is None:
            keep = [i for i, s in enumerate(self._sizes) if s != 1]
            return self._view([self._sizes[i] for i in keep], [self._strides[i] for i in keep])
        d = _positive_dim(dim, self.dim())
        if self._sizes[d] != 1:
            return self._view(self._sizes, self._strides)
        return self._view(self._sizes[:d] + self._sizes[d + 1:], self._strides[:d] + self._strides[d + 1:])

    def narrow(self, dim, start, length):
        d = _positive_dim(dim, self.dim())
        if start < 0 or length < 0 or start + length > self._sizes[d]:
            raise IndexError("narrow range out of bounds")
        sizes = list(self._sizes)
        sizes[d] = length
        return self._view(sizes, self._strides, self._offset + start * self._strides[d])

    def select(self, dim, index):
        d = _positive_dim(dim, self.dim())
        size = self._sizes[d]
        if index < 0:
            index += size
        if index < 0 or index >= size:
            raise IndexError("select index out of bounds")
        return self._view(
            self._sizes[:d] + self._sizes[d + 1:],
            self._strides[:d] + self._strides[d + 1:],
            self._offset + index * self._strides[d],
        )

    def split(self, split_size, dim=0):
        d = _positive_dim(dim, self.dim())
        size = self._sizes[d]
        if isinstance(split_size, (list, tuple)):
            if any(s < 0 for s in split_size):
                raise ValueError("split sizes must be non-negative")
            if sum(split_size) != size:
                raise ValueError("split sizes must sum exactly to the selected dimension size")
            out, start = [], 0
            for s in split_size:
                out.append(self.narrow(d, start, s))
                start += s
            return tuple(out)
        if split_size <= 0:
            raise ValueError("split_size must be greater than zero")
        if size == 0:
            return (self.narrow(d, 0, 0),)
        return tuple(self.narrow(d, s, _builtins.min(split_size, size - s)) for s in range(0, size, split_size))

    def chunk(self, chunks, dim=0):
        if chunks <= 0:
            raise ValueError("chunks must be greater than zero")
        d = _positive_dim(dim, self.dim())
        size = self._sizes[d]
        if size == 0:
            return tuple(self.narrow(d, 0, 0) for _ in range(chunks))
        cs = (size + chunks - 1) // chunks
        return tuple(self.narrow(d, s, _builtins.min(cs, size - s)) for s in range(0, size, cs))

    def expand(self, *sizes):
        if len(sizes) == 1 and isinstance(sizes[0], (list, tuple, Size)):
            sizes = tuple(sizes[0])
        sizes = list(sizes)
        rank, trank = self.dim(), len(sizes)
        if trank < rank:
            raise ValueError("expand target rank must be greater than or equal to input rank")
        out_s, out_st = [0] * trank, [0] * trank
        delta = trank - rank
        for td in range(trank - 1, -1, -1):
            idim = td - delta
            ts = sizes[td]
            if idim < 0:
                if ts < 0:
                    raise ValueError("expanded sizes must be non-negative")
                out_s[td], out_st[td] = ts, 0
                continue
            isz, ist = self._sizes[idim], self._strides[idim]
            if ts == -1:
                ts = isz
            if isz == ts:
                out_s[td], out_st[td] = ts, ist
            elif isz == 1:
                out_s[td], out_st[td] = ts, 0
            else:
                raise ValueError("expanded size must match the existing size at non-singleton dimensions")
        return self._view(out_s, out_st)

    def expand_as(self, other):
        return self.expand(other.shape)

    def __getitem__(self, key):
        if not isinstance(key, tuple):
            key = (key,)
        if any(isinstance(k, Tensor) for k in key):
            raise NotImplementedError("tensor indexing is not supported by mtorch_amd")
        n_real = sum(1 for k in key if k is not None and k is not Ellipsis)
        if n_real > self.dim():
            raise IndexError("too many indices for tensor")
        expanded = []
        for k in key:
            if k is Ellipsis:
                expanded.extend([slice(None)] * (self.dim() - n_real))
            else:
                expanded.append(k)
        sizes, strides, offset = [], [], self._offset
        d = 0
        for k in expanded:
            if k is None:
                # New axis: the stride unsqueeze would give at this position (tensor.cpp:12068-12082).
                sizes.append(1)
                strides.append(self._strides[d] * self._sizes[d] if d < self.dim() else 1)
                continue
            if isinstance(k, slice):
                start, stop, step = k.indices(self._sizes[d])
                if step <= 0:
                    raise ValueError("slice step must be positive")
                length = _builtins.max(0, (stop - start + step - 1) // step)
                offset += start * self._strides[d] if length else 0
                sizes.append(length)
                strides.append(self._strides[d] * step)
                d += 1
                continue
            idx = _builtins.int(k)
            size = self._sizes[d]
            if idx < 0:
                idx += size
            if idx < 0 or idx >= size:
                raise IndexError(f"index {k} is out of bounds for dimension {d} with size {size}")
            offset += idx * self._strides[d]
            d += 1
        sizes.extend(self._sizes[d:])
        strides.extend(self._strides[d:])
        return self._view(sizes, strides, offset)

    def __setitem__(self, key, value):
        """Item assignment into the view self[key] (a scalar fills it, a tensor is copied in with
        broadcasting), as the reference's Tensor.__setitem__ does for basic indices."""
        from . import _ops

        _ops.copy_into(self[key], value)

    # ---- arithmetic ---------------------------------------------------------------------
    def __add__(self, other):
        from . import _ops

        return _ops.binary(self, other, "add")

    def __radd__(self, other):
        from . import _ops

        return _ops.binary(other, self, "add")

    def __sub__(self, other):
        from . import _ops

        return _ops.binary(self, other, "sub")

    def __rsub__(self, other):
        from . import _ops

        return _ops.binary(other, self, "sub")

    def __mul__(self, other):
        from . import _ops

        return _ops.binary(self, other, "mul")

    def __rmul__(self, other):
        from . import _ops

        return _ops.binary(other, self, "mul")

    def __truediv__(self, other):
        from . import _ops

        return _ops.binary(self, other, "div")

    def __rtruediv__(self, other):
        from . import _ops

        return _ops.binary(other, self, "div")

    def __neg__(self):
        from . import _ops

        return _ops.unary(self, "neg")

    def __invert__(self):
        from . import _ops

        return _ops.logical_not(self)

    def logical_not(self):
        from . import _ops

        return _ops.logical_not(self)

    def masked_fill(self, mask, value):
        from . import _ops

        return _ops.masked_fill(self, mask, value)

    def __matmul__(self, other):
        from . import _ops

        return _ops.matmul(self, other)

    def add(self, other, alpha=1):
        from . import _ops

        if alpha != 1:
            other = _ops.binary(other, alpha, "mul")
        return _ops.binary(self, other, "add")

    def sub(self, other, alpha=1):
        from . import _ops

        if alpha != 1:
            other = _ops.binary(other, alpha, "mul")
        return _ops.binary(self, other, "sub")

    def mul(self, other):
        from . import _ops

        return _ops.binary(self, other, "mul")

    def div(self, other):
        from . import _ops

        return _ops.binary(self, other, "div")

    def matmul(self, other):
        from . import _ops

        return _ops.matmul(self, other)

    def softmax(self, dim, dtype=None):
        from . import _ops

        return _ops.softmax(self, dim, dtype)

    def exp(self):
        from . import _ops

        return _ops.unary(self, "exp")

    def sin(self):
        from . import _ops

        return _ops.unary(self, "sin")

    def cos(self):
        from . import _ops

        return _ops.unary(self, "cos")

    def sigmoid(self):
        from . import _ops

        return _ops.unary(self, "sigmoid")

    def relu(self):
        from . import _ops

        return _ops.unary(self, "relu")

    # ---- in-place (data initialisation) -------------------------------------------------
    def copy_(self, src):
        from . import _ops

        _ops.copy_into(self, src)
        return self

    def fill_(self, value):
        from . import _ops

        _ops.fill_(self, value)
        return self

    def zero_(self):
        return self.fill_(0.0)

    def normal_(self, mean=0.0, std=1.0, generator=None):
        from . import _random

        _random.normal_(self, mean, std, generator)
        return self

    def uniform_(self, a=0.0, b=1.0, generator=None):
        from . import _random

        _random.uniform_(self, a, b, generator)
        return self


class Size(tuple):
    def __new__(cls, sizes):
        return tuple.__new__(cls, (_builtins.int(s) for s in sizes))

    def numel(self):
        return _numel(self)

    def __repr__(self):
        return f"mtorch_amd.Size({list(self)})"


# ------------------------------------------------------------------------------ construction


def empty(*sizes, dtype=None, device=None, requires_grad=False):
    if len(sizes) == 1 and isinstance(sizes[0], (list, tuple, Size)):
        sizes = tuple(sizes[0])
    sizes = [_builtins.int(s) for s in sizes]
    dt = _as_dtype(dtype, float32)
    dev = _resolve_device(device)
    st = Storage(dt, _numel(sizes), dev)
    return Tensor(st, sizes, contiguous_strides(sizes), 0, requires_grad)


def _resolve_device(dev):
    return globals()["device"]("cpu") if dev is None else globals()["device"](dev)


def zeros(*sizes, dtype=None, device=None, requires_grad=False):
    return full(_size_args(sizes), 0.0, dtype=dtype, device=device, requires_grad=requires_grad)


def ones(*sizes, dtype=None, device=None, requires_grad=False):
    return full(_size_args(sizes), 1.0, dtype=dtype, device=device, requires_grad=requires_grad)


def _size_args(sizes):
    if len(sizes) == 1 and isinstance(sizes[0], (list, tuple, Size)):
        return tuple(sizes[0])
    return tuple(sizes)


def full(size, fill_value, dtype=None, device=None, requires_grad=False):
    t = empty(size, dtype=dtype, device=device, requires_grad=requires_grad)
    t.fill_(fill_value)
    return t


def from_numpy(array, dtype=None, device=None):
    """Tensor from a numpy array; float16 arrays (by value) map to float16 storage."""
    arr = np.asarray(array)
    if dtype is None:
        dtype = {
            np.dtype(np.float16): float16,
            np.dtype(np.float32): float32,
            np.dtype(np.float64): float64,
            np.dtype(np.int32): int32,
            np.dtype(np.int64): int64,
            np.dtype(np.bool_): bool_,
        }.get(arr.dtype, float32)
    dt = _as_dtype(dtype)
    sizes = list(arr.shape)
    if dt is float16:
        if arr.dtype == np.float16:
            host = np.ascontiguousarray(arr).view(np.uint16).reshape(-1).copy()
        elif arr.dtype == np.uint16:
            host = np.ascontiguousarray(arr).reshape(-1).copy()
        else:
            # Narrow through fp32 with mtorch's rounding rule (float_to_half_bits).
            from . import _random

            host = _random.float_to_half_bits(np.ascontiguousarray(arr, dtype=np.float32).reshape(-1))
    elif dt is bool_:
        host = np.ascontiguousarray(arr).astype(np.uint8).reshape(-1)
    else:
        host = np.ascontiguousarray(arr, dtype=dt.np).reshape(-1).copy()
    cpu = Tensor(Storage(dt, host.size, globals()["device"]("cpu"), host=host), sizes, contiguous_strides(sizes))
    if device is not None and globals()["device"](device).type != "cpu":
        return cpu.to(device)
    return cpu


def tensor(data, dtype=None, device=None, requires_grad=False):
    if isinstance(data, Tensor):
        out = data.to(dtype=dtype or data.dtype).clone() if device is None else data.to(device=device, dtype=dtype or data.dtype, copy=True)
        out.requires_grad = requires_grad
        return out
    arr = np.asarray(data)
    if dtype is None:
        if arr.dtype == np.bool_:
            dtype = bool_
        elif np.issubdtype(arr.dtype, np.integer):
            dtype = int64
        else:
            dtype = float32
    dt = _as_dtype(dtype)
    if dt is float16 and arr.dtype != np.float16:
        arr = arr.astype(np.float64)
        from . import _random

        host = _random.float_to_half_bits(arr.astype(np.float32).reshape(-1))
        sizes = list(arr.shape)
        t = Tensor(Storage(dt, host.size, globals()["device"]("cpu"), host=host), sizes, contiguous_strides(sizes))
    else:
        t = from_numpy(arr.astype(dt.np) if dt not in (float16, bool_) else arr, dtype=dt)
    if device is not None and globals()["device"](device).type != "cpu":
        t = t.to(device)
    t.requires_grad = requires_grad
    return t
