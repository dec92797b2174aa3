"""mtorch.nn surface for the SD-UNet hot path."""

from . import functional, init
from .modules import (
    GELU,
    Conv2d,
    Dropout,
    GroupNorm,
    Identity,
    LayerNorm,
    Linear,
    Module,
    ModuleList,
    MultiheadAttention,
    Parameter,
    Sequential,
    SiLU,
    Softmax,
    Upsample,
)

__all__ = [
    "functional", "init", "Module", "Parameter", "Linear", "Conv2d", "GroupNorm", "LayerNorm", "SiLU", "GELU",
    "Dropout", "Identity", "Sequential", "ModuleList", "Softmax", "Upsample", "MultiheadAttention",
]
