"""mtorch.nn.init for the hot path (mtorch/__init__.py:5436-5512), drawing from mtorch's generator."""

from __future__ import annotations

import math


def calculate_gain(nonlinearity, param=None):
    """_calculate_gain (mtorch/__init__.py:5463-5478)."""
    name = str(nonlinearity).lower()
    if name in {"linear", "sigmoid", "conv1d", "conv2d", "conv3d", "conv_transpose1d", "conv_transpose2d",
                "conv_transpose3d"}:
        return 1.0
    if name == "tanh":
        return 5.0 / 3.0
    if name == "relu":
        return math.sqrt(2.0)
    if name == "leaky_relu":
        slope = 0.01 if param is None else float(param)
        return math.sqrt(2.0 / (1.0 + slope * slope))
    if name == "selu":
        return 0.75
    raise ValueError(f"unsupported nonlinearity {nonlinearity!r}")


def _calculate_fan_in_and_fan_out(tensor):
    if tensor.ndim < 2:
        raise ValueError("fan in and fan out can not be computed for tensor with fewer than 2 dimensions")
    receptive = 1
    for v in tensor.shape[2:]:
        receptive *= v
    return tensor.shape[1] * receptive, tensor.shape[0] * receptive


def normal_(tensor, mean=0.0, std=1.0, generator=None):
    return tensor.normal_(mean, std, generator=generator)


def uniform_(tensor, a=0.0, b=1.0, generator=None):
    return tensor.uniform_(a, b, generator=generator)


def zeros_(tensor):
    return tensor.fill_(0.0)


def ones_(tensor):
    return tensor.fill_(1.0)


def constant_(tensor, val):
    return tensor.fill_(val)


def xavier_uniform_(tensor, gain=1.0, generator=None):
    fan_in, fan_out = _calculate_fan_in_and_fan_out(tensor)
    bound = float(gain) * math.sqrt(6.0 / float(fan_in + fan_out))
    return tensor.uniform_(-bound, bound, generator=generator)


def xavier_normal_(tensor, gain=1.0, generator=None):
    fan_in, fan_out = _calculate_fan_in_and_fan_out(tensor)
    return tensor.normal_(0.0, float(gain) * math.sqrt(2.0 / float(fan_in + fan_out)), generator=generator)


def kaiming_uniform_(tensor, a=0.0, mode="fan_in", nonlinearity="leaky_relu", generator=None):
    """_init_kaiming_uniform_ (mtorch/__init__.py:5487-5499)."""
    fan_in, fan_out = _calculate_fan_in_and_fan_out(tensor)
    if mode == "fan_in":
        fan = fan_in
    elif mode == "fan_out":
        fan = fan_out
    else:
        raise ValueError("mode must be 'fan_in' or 'fan_out'")
    gain = calculate_gain(nonlinearity, a)
    std = gain / math.sqrt(float(fan))
    bound = math.sqrt(3.0) * std
    return tensor.uniform_(-bound, bound, generator=generator)


def kaiming_normal_(tensor, a=0.0, mode="fan_in", nonlinearity="leaky_relu", generator=None):
    fan_in, fan_out = _calculate_fan_in_and_fan_out(tensor)
    fan = fan_in if mode == "fan_in" else fan_out
    return tensor.normal_(0.0, calculate_gain(nonlinearity, a) / math.sqrt(float(fan)), generator=generator)
