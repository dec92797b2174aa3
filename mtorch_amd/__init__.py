"""mtorch_amd -- mtorch's SD-UNet hot path on AMD Instinct MI355X (gfx950).

The operator surface is mtorch's (mtorch/__init__.py): tensors are created and seeded on the
host with mtorch's generator, moved with ``.to("cuda")`` and every hot-path operator then
runs as a hand-written HIP kernel in libmthip (include/mthip.h).
"""

from __future__ import annotations

from . import _lib, cuda, nn
from ._einsum import einsum
from ._ops import (
    addmm,
    arange,
    baddbmm,
    bmm,
    cat,
    logical_not,
    masked_fill,
    matmul,
)
from ._ops import add as _add
from ._random import Generator, initial_seed, manual_seed, rand, randn
from ._tensor import (
    Size,
    Tensor,
    bool_,
    device,
    double,
    dtype,
    empty,
    enable_grad,
    float,
    float16,
    float32,
    float64,
    from_numpy,
    full,
    half,
    int32,
    int64,
    is_grad_enabled,
    long,
    no_grad,
    ones,
    set_grad_enabled,
    tensor,
    zeros,
)
from .nn import functional as _F
from .serialization import load, save

bool = bool_  # noqa: A001 - mtorch exposes mtorch.bool

softmax = _F.softmax
sigmoid = _F.sigmoid
relu = _F.relu
silu = _F.silu
gelu = _F.gelu


def add(input, other, alpha=1):
    return _add(input, other, alpha)


def mul(input, other):
    return input * other


def sub(input, other):
    return input - other


def exp(input):
    return input.exp()


def sin(input):
    return input.sin()


def cos(input):
    return input.cos()


def chunk(input, chunks, dim=0):
    return input.chunk(chunks, dim)


def split(input, split_size_or_sections, dim=0):
    return input.split(split_size_or_sections, dim)


def reshape(input, shape):
    return input.reshape(shape)


def transpose(input, dim0, dim1):
    return input.transpose(dim0, dim1)


def permute(input, dims):
    return input.permute(dims)


def flatten(input, start_dim=0, end_dim=-1):
    return input.flatten(start_dim, end_dim)


def unsqueeze(input, dim):
    return input.unsqueeze(dim)


def backend_version() -> str:
    return _lib.lib().mthip_version().decode()


__all__ = [
    "Tensor", "Size", "dtype", "device", "float16", "float32", "float64", "half", "float", "double", "int32",
    "int64", "long", "bool", "tensor", "from_numpy", "empty", "zeros", "ones", "full", "randn", "rand",
    "manual_seed", "initial_seed", "Generator", "no_grad", "enable_grad", "set_grad_enabled", "is_grad_enabled",
    "matmul", "bmm", "addmm", "baddbmm", "cat", "arange", "softmax", "sigmoid", "relu", "silu", "gelu", "add",
    "mul", "sub", "exp", "sin", "cos", "chunk", "split", "reshape", "transpose", "permute", "flatten", "unsqueeze",
    "einsum", "masked_fill", "logical_not", "save", "load", "nn", "cuda",
]
