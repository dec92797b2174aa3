"""mtorch.nn.functional surface for the hot path (mtorch/__init__.py:5515-5573)."""

from __future__ import annotations

from .. import _ops

linear = _ops.linear
conv2d = _ops.conv2d
scaled_dot_product_attention = _ops.scaled_dot_product_attention
group_norm = _ops.group_norm
layer_norm = _ops.layer_norm
gelu = _ops.gelu
silu = _ops.silu
interpolate = _ops.interpolate


def softmax(input, dim=None, _stacklevel=3, dtype=None):
    return _ops.softmax(input, -1 if dim is None else dim, dtype)


def relu(input, inplace=False):
    return _ops.unary(input, "relu")


def sigmoid(input):
    return _ops.unary(input, "sigmoid")


def dropout(input, p=0.5, training=True, inplace=False):
    """Inference: identity unless training with p > 0 (no device dropout kernel)."""
    if not training or p == 0.0:
        return input
    if p == 1.0:
        return _ops.binary(input, 0.0, "mul")
    raise _ops.unsupported("dropout(training=True)", input.device)


# Fused forms of op sequences the SD blocks use; each equals the unfused sequence
# (every intermediate narrowed to the storage dtype in the same order).


def linear_gelu(input, weight, bias=None):
    """gelu(linear(input, weight, bias))"""
    return _ops.linear(input, weight, bias, act=_ops.ACT_GELU)


def linear_silu(input, weight, bias=None):
    """silu(linear(input, weight, bias))"""
    return _ops.linear(input, weight, bias, act=_ops.ACT_SILU)


def linear_residual(input, weight, bias, residual):
    """linear(input, weight, bias) + residual"""
    return _ops.linear(input, weight, bias, residual=residual)


def group_norm_silu(input, num_groups, weight=None, bias=None, eps=1e-5):
    """silu(group_norm(input, ...))"""
    return _ops.group_norm(input, num_groups, weight, bias, eps, fuse_silu=True)


def group_norm_silu_conv2d(input, num_groups, gn_weight, gn_bias, eps, weight, bias=None, stride=1, padding=0,
                           dilation=1, residual=None, chan_add=None):
    """conv2d(silu(group_norm(input, num_groups, gn_weight, gn_bias, eps)), weight, bias, ...)
    (+ chan_add[:, :, None, None]) (+ residual), with the normalised activation handed to the
    conv channels-last and both adds in the conv's epilogue"""
    return _ops.group_norm_silu_conv2d(input, num_groups, gn_weight, gn_bias, eps, weight, bias, stride, padding,
                                       dilation, residual, chan_add)


def conv2d_residual(input, weight, bias, residual, stride=1, padding=0, dilation=1, groups=1):
    """conv2d(input, weight, bias, ...) + residual"""
    return _ops.conv2d(input, weight, bias, stride, padding, dilation, groups, residual=residual)


def linear_geglu(input, weight, bias=None):
    """a * gelu(gate) with (a, gate) = linear(input, weight, bias).chunk(2, dim=-1)"""
    return _ops.linear_geglu(input, weight, bias)


def geglu(input):
    """a * gelu(gate) with (a, gate) = input.chunk(2, dim=-1)"""
    return _ops.geglu(input)
