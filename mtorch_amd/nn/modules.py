"""nn modules of the hot path: Module, Parameter, Linear, Conv2d, GroupNorm, LayerNorm, SiLU,
GELU and containers.  Default initialisation reproduces the reference's deterministic
formulas (Linear._initial_weight mtorch/__init__.py:3330-3332, Conv2d._initial_weight
:3498-3502, ones/zeros for the norms :5066-5070, :5196-5197) but is computed natively instead
of through nested Python lists.
"""

from __future__ import annotations

from collections import OrderedDict

import numpy as np

from .. import _ops
from .. import _random
from .. import _tensor as T
from . import functional


class Parameter(T.Tensor):
    """A Tensor registered on a Module; shares storage with `data`."""

    def __init__(self, data=None, requires_grad=True):
        if data is None:
            data = T.empty(0)
        super().__init__(data._storage, data._sizes, data._strides, data._offset, requires_grad)

    def __repr__(self):
        return "Parameter containing:\n" + super().__repr__()


def _make(values_f64: np.ndarray, sizes, dtype, device):
    dt = T._as_dtype(dtype, T.float32)
    host = _random.host_cast(values_f64.reshape(-1), T.float64, dt)
    t = T.Tensor(T.Storage(dt, host.size, T.device("cpu"), host=host), list(sizes), T.contiguous_strides(list(sizes)))
    if device is not None and T.device(device).type != "cpu":
        t = t.to(device)
    return t


class Module:
    training = True

    def __init__(self):
        object.__setattr__(self, "training", True)

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)

    def forward(self, *args, **kwargs):  # pragma: no cover - abstract
        raise NotImplementedError

    # ---- traversal ---------------------------------------------------------------------
    def named_children(self):
        for name, value in self.__dict__.items():
            if isinstance(value, Module):
                yield name, value

    def children(self):
        for _, m in self.named_children():
            yield m

    def named_modules(self, prefix=""):
        yield prefix, self
        for name, child in self.named_children():
            yield from child.named_modules(f"{prefix}.{name}" if prefix else name)

    def modules(self):
        for _, m in self.named_modules():
            yield m

    def named_parameters(self, prefix=""):
        seen = set()
        for mname, m in self.named_modules(prefix):
            for name, value in m.__dict__.items():
                if isinstance(value, Parameter) and id(value) not in seen:
                    seen.add(id(value))
                    yield (f"{mname}.{name}" if mname else name), value

    def parameters(self):
        for _, p in self.named_parameters():
            yield p

    def state_dict(self):
        return OrderedDict(self.named_parameters())

    def load_state_dict(self, state, strict=True):
        own = dict(self.named_parameters())
        missing = [k for k in own if k not in state]
        unexpected = [k for k in state if k not in own]
        if strict and (missing or unexpected):
            raise RuntimeError(f"load_state_dict: missing {missing}, unexpected {unexpected}")
        for k, v in state.items():
            if k in own:
                own[k].copy_(v)
        return self

    # ---- conversion --------------------------------------------------------------------
    def to(self, *args, **kwargs):
        """Module.to(device/dtype) (mtorch/__init__.py:2848-2904): converts every parameter
        (floating dtypes only for a dtype change) and recurses into children."""
        dev = kwargs.pop("device", None)
        dt = kwargs.pop("dtype", None)
        for a in args:
            if isinstance(a, T.dtype):
                dt = a
            elif a is not None:
                dev = a
        target_dev = None if dev is None else T.device(dev)
        target_dt = None if dt is None else T._as_dtype(dt)
        for m in self.modules():
            for name, value in list(m.__dict__.items()):
                if isinstance(value, T.Tensor):
                    new_dt = target_dt if (target_dt is not None and value.dtype.is_floating_point) else value.dtype
                    converted = value.to(device=target_dev or value.device, dtype=new_dt)
                    if isinstance(value, Parameter) and not isinstance(converted, Parameter):
                        converted = Parameter(converted, value.requires_grad)
                    object.__setattr__(m, name, converted)
        return self

    def cuda(self, device=None):
        return self.to("cuda" if device is None else f"cuda:{device}")

    def cpu(self):
        return self.to("cpu")

    def half(self):
        return self.to(dtype=T.float16)

    def float(self):
        return self.to(dtype=T.float32)

    def eval(self):
        for m in self.modules():
            object.__setattr__(m, "training", False)
        return self

    def train(self, mode=True):
        for m in self.modules():
            object.__setattr__(m, "training", bool(mode))
        return self

    def requires_grad_(self, requires_grad=True):
        for p in self.parameters():
            p.requires_grad = requires_grad
        return self

    def zero_grad(self, set_to_none=True):
        return None


class Identity(Module):
    def forward(self, x):
        return x


class Sequential(Module):
    def __init__(self, *modules):
        super().__init__()
        for i, m in enumerate(modules):
            setattr(self, str(i), m)
        object.__setattr__(self, "_order", [str(i) for i in range(len(modules))])

    def forward(self, x):
        for name in self._order:
            x = getattr(self, name)(x)
        return x

    def __getitem__(self, i):
        return getattr(self, self._order[i])

    def __len__(self):
        return len(self._order)


class ModuleList(Module):
    def __init__(self, modules=()):
        super().__init__()
        object.__setattr__(self, "_order", [])
        for m in modules:
            self.append(m)

    def append(self, m):
        name = str(len(self._order))
        setattr(self, name, m)
        self._order.append(name)
        return self

    def __getitem__(self, i):
        return getattr(self, self._order[i])

    def __iter__(self):
        return (getattr(self, n) for n in self._order)

    def __len__(self):
        return len(self._order)


class Linear(Module):
    def __init__(self, in_features, out_features, bias=True, device=None, dtype=None):
        super().__init__()
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        span = max(1, self.in_features)
        idx = np.arange(self.out_features * self.in_features, dtype=np.int64)
        vals = ((idx % (2 * span + 1)) - span).astype(np.float64) / float(span * span)
        self.weight = Parameter(_make(vals, [self.out_features, self.in_features], dtype, device))
        self.bias = Parameter(_make(np.zeros(self.out_features), [self.out_features], dtype, device)) if bias else None

    def forward(self, input):
        return functional.linear(input, self.weight, self.bias)


class Conv2d(Module):
    def __init__(self, in_channels, out_channels, kernel_size, stride=1, padding=0, dilation=1, groups=1, bias=True,
                 padding_mode="zeros", device=None, dtype=None):
        super().__init__()
        pair = lambda v: (int(v), int(v)) if isinstance(v, int) else tuple(int(x) for x in v)  # noqa: E731
        self.in_channels = int(in_channels)
        self.out_channels = int(out_channels)
        self.kernel_size = pair(kernel_size)
        self.stride = pair(stride)
        self.padding = padding if isinstance(padding, str) else pair(padding)
        self.dilation = pair(dilation)
        self.groups = int(groups)
        if self.groups <= 0:
            raise ValueError("groups must be a positive integer")
        if self.in_channels % self.groups != 0:
            raise ValueError("in_channels must be divisible by groups")
        if self.out_channels % self.groups != 0:
            raise ValueError("out_channels must be divisible by groups")
        if padding_mode != "zeros":
            raise NotImplementedError("only padding_mode='zeros' is supported on the device")
        self.padding_mode = padding_mode
        cpg = self.in_channels // self.groups
        kh, kw = self.kernel_size
        fan_in = max(1, cpg * kh * kw)
        pos = np.arange(self.out_channels * cpg * kh * kw, dtype=np.int64)
        vals = ((pos % (2 * fan_in + 1)) - fan_in).astype(np.float64) / float(fan_in * fan_in)
        self.weight = Parameter(_make(vals, [self.out_channels, cpg, kh, kw], dtype, device))
        self.bias = Parameter(_make(np.zeros(self.out_channels), [self.out_channels], dtype, device)) if bias else None

    def forward(self, input):
        return functional.conv2d(input, self.weight, self.bias, self.stride, self.padding, self.dilation, self.groups)


class GroupNorm(Module):
    def __init__(self, num_groups, num_channels, eps=1e-5, affine=True, device=None, dtype=None):
        super().__init__()
        self.num_groups = int(num_groups)
        self.num_channels = int(num_channels)
        self.eps = float(eps)
        self.affine = bool(affine)
        if self.affine:
            self.weight = Parameter(_make(np.ones(self.num_channels), [self.num_channels], dtype, device))
            self.bias = Parameter(_make(np.zeros(self.num_channels), [self.num_channels], dtype, device))
        else:
            self.weight = None
            self.bias = None

    def forward(self, input):
        return functional.group_norm(input, self.num_groups, self.weight, self.bias, self.eps)


class LayerNorm(Module):
    def __init__(self, normalized_shape, eps=1e-5, elementwise_affine=True, bias=True, device=None, dtype=None):
        super().__init__()
        if isinstance(normalized_shape, int):
            normalized_shape = (normalized_shape,)
        self.normalized_shape = tuple(normalized_shape)
        self.eps = eps
        self.elementwise_affine = bool(elementwise_affine)
        n = int(np.prod(self.normalized_shape))
        if self.elementwise_affine:
            self.weight = Parameter(_make(np.ones(n), list(self.normalized_shape), dtype, device))
            self.bias = Parameter(_make(np.zeros(n), list(self.normalized_shape), dtype, device)) if bias else None
        else:
            self.weight = None
            self.bias = None

    def forward(self, input):
        return functional.layer_norm(input, self.normalized_shape, self.weight, self.bias, self.eps)


class SiLU(Module):
    def __init__(self, inplace=False):
        super().__init__()

    def forward(self, input):
        return functional.silu(input)


class GELU(Module):
    def __init__(self, approximate="none"):
        super().__init__()
        self.approximate = approximate

    def forward(self, input):
        return functional.gelu(input, approximate=self.approximate)


class Dropout(Module):
    def __init__(self, p=0.5, inplace=False):
        super().__init__()
        self.p = p

    def forward(self, input):
        return functional.dropout(input, self.p, self.training)


class Softmax(Module):
    def __init__(self, dim=None):
        super().__init__()
        self.dim = dim

    def forward(self, input):
        return functional.softmax(input, self.dim)


class Upsample(Module):
    def __init__(self, size=None, scale_factor=None, mode="nearest"):
        super().__init__()
        self.size, self.scale_factor, self.mode = size, scale_factor, mode

    def forward(self, input):
        return functional.interpolate(input, self.size, self.scale_factor, self.mode)
