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


def _logical_and(a, b):
    """Bool AND with broadcasting: a (broadcast to the joint shape) with False wherever b is
    false -- one masked_fill launch, no separate kernel."""
    shape = T._broadcast_shape(list(a.shape), list(b.shape))
    return _ops.masked_fill(a.expand(shape), b.logical_not(), False)


def _keep_mask_to_bias(mask):
    """where(mask, 0.0, -inf) in float32 (mtorch/__init__.py:4413-4418)."""
    zeros = T.zeros(list(mask.shape), dtype=T.float32, device=mask.device)
    return _ops.masked_fill(zeros, mask.logical_not(), float("-inf"))


class MultiheadAttention(Module):
    """nn.MultiheadAttention (mtorch/__init__.py:4297-4578) over the device kernels: the fused
    (3E x E) input projection when query, key and value are one tensor, the flash SDPA kernel
    for the heads, and out_proj.  Deterministic default weights as the reference's
    `_initial_weight(row, col, width)` (:4383-4385), input-projection bias zero, and the same
    mask merging: a bool attn_mask / key_padding_mask marks positions to EXCLUDE and is inverted
    into SDPA's keep mask; bool and float masks combine as an additive -inf bias."""

    def __init__(self, embed_dim, num_heads, dropout=0.0, bias=True, add_bias_kv=False, add_zero_attn=False,
                 kdim=None, vdim=None, batch_first=False, device=None, dtype=None):
        super().__init__()
        self.embed_dim = int(embed_dim)
        self.num_heads = int(num_heads)
        self.dropout = float(dropout)
        self.batch_first = batch_first
        self.head_dim = self.embed_dim // self.num_heads
        if self.head_dim * self.num_heads != self.embed_dim:
            raise ValueError("embed_dim must be divisible by num_heads")
        self.kdim = self.embed_dim if kdim is None else int(kdim)
        self.vdim = self.embed_dim if vdim is None else int(vdim)
        self._qkv_same_embed_dim = self.kdim == self.embed_dim and self.vdim == self.embed_dim
        self.add_zero_attn = bool(add_zero_attn)
        E = self.embed_dim
        if self._qkv_same_embed_dim:
            self.in_proj_weight = Parameter(_make(self._initial(3 * E, E, E), [3 * E, E], dtype, device))
            self.q_proj_weight = self.k_proj_weight = self.v_proj_weight = None
        else:
            self.in_proj_weight = None
            self.q_proj_weight = Parameter(_make(self._initial(E, E, E), [E, E], dtype, device))
            self.k_proj_weight = Parameter(_make(self._initial(E, self.kdim, self.kdim), [E, self.kdim], dtype, device))
            self.v_proj_weight = Parameter(_make(self._initial(E, self.vdim, self.vdim), [E, self.vdim], dtype, device))
        self.in_proj_bias = Parameter(_make(np.zeros(3 * E), [3 * E], dtype, device)) if bias else None
        if add_bias_kv:
            self.bias_k = Parameter(_make(self._initial(1, E, E), [1, 1, E], dtype, device))
            self.bias_v = Parameter(_make(self._initial(2, E, E)[E:], [1, 1, E], dtype, device))
        else:
            self.bias_k = self.bias_v = None
        self.out_proj = Linear(E, E, bias=bias, device=device, dtype=dtype)

    @staticmethod
    def _initial(rows, cols, width):
        """_initial_weight(row, col, width) for row < rows, col < cols, in float64."""
        span = max(1, width)
        r = np.arange(rows, dtype=np.int64)[:, None]
        c = np.arange(cols, dtype=np.int64)[None, :]
        return (((r * width + c) % (2 * span + 1)) - span).astype(np.float64).reshape(-1) / float(span * span)

    # ---- layout ------------------------------------------------------------------------
    def _as_batch_first(self, x):
        if x.dim() == 2:
            return x.reshape(1, x.shape[0], x.shape[1]), True
        if x.dim() != 3:
            raise ValueError("MultiheadAttention input must be 2-D or 3-D")
        return (x, False) if self.batch_first else (x.transpose(0, 1), False)

    def _restore_layout(self, x, unbatched):
        if unbatched:
            return x.squeeze(0)
        return x if self.batch_first else x.transpose(0, 1)

    def _split_heads(self, x):
        b, n, _ = x.shape
        return x.reshape(b, n, self.num_heads, self.head_dim).transpose(1, 2)

    def _merge_heads(self, x):
        b, _, n, _ = x.shape
        return x.transpose(1, 2).contiguous().reshape(b, n, self.embed_dim)

    # ---- masks -------------------------------------------------------------------------
    @staticmethod
    def _pad_source_mask(mask):
        if mask is None:
            return None
        pad = T.zeros(list(mask.shape[:-1]) + [1], dtype=mask.dtype, device=mask.device)
        return _ops.cat([mask, pad], dim=mask.dim() - 1)

    def _append_bias_kv(self, k, v, kpm, am):
        if self.bias_k is None:
            return k, v, kpm, am
        b = k.shape[0]
        k = _ops.cat([k, self.bias_k.expand(b, 1, self.embed_dim)], dim=1)
        v = _ops.cat([v, self.bias_v.expand(b, 1, self.embed_dim)], dim=1)
        return k, v, self._pad_source_mask(kpm), self._pad_source_mask(am)

    def _append_zero_kv(self, k, v, kpm, am):
        if not self.add_zero_attn:
            return k, v, kpm, am
        k = _ops.cat([k, T.zeros([k.shape[0], 1, k.shape[2]], dtype=k.dtype, device=k.device)], dim=1)
        v = _ops.cat([v, T.zeros([v.shape[0], 1, v.shape[2]], dtype=v.dtype, device=v.device)], dim=1)
        return k, v, self._pad_source_mask(kpm), self._pad_source_mask(am)

    def _merge_attention_masks(self, attn_mask, key_padding_mask, batch, source_length):
        """mtorch/__init__.py:4439-4470."""
        merged = None
        if attn_mask is not None:
            merged = attn_mask.logical_not() if attn_mask.dtype is T.bool_ else attn_mask
        if key_padding_mask is not None:
            kpm = key_padding_mask
            if kpm.dim() == 1:
                if kpm.shape[0] != source_length:
                    raise ValueError("key_padding_mask source length does not match key")
                kpm = kpm.reshape(1, source_length)
            elif kpm.dim() != 2:
                raise ValueError("key_padding_mask must be 1-D or 2-D")
            if kpm.shape[0] != batch or kpm.shape[1] != source_length:
                raise ValueError("key_padding_mask shape must be (batch, source_length)")
            km = kpm.logical_not() if kpm.dtype is T.bool_ else kpm
            km = km.reshape(batch, 1, 1, source_length)
            if merged is None:
                merged = km
            elif merged.dtype is T.bool_ and km.dtype is T.bool_:
                merged = _logical_and(merged, km)
            else:
                if merged.dtype is T.bool_:
                    merged = _keep_mask_to_bias(merged)
                if km.dtype is T.bool_:
                    km = _keep_mask_to_bias(km)
                merged = merged + km
        return merged

    def _attention_weights(self, q, k, mask, is_causal, average, unbatched):
        """The per-head probabilities SDPA used (the reference runs SDPA against an identity value,
        mtorch/__init__.py:4472-4491): softmax(q k^T / sqrt(head_dim) + mask) computed in float32
        as SDPA does, averaged over heads before the one narrowing to the query dtype."""
        b, h, lq, d = q.shape
        lk = k.shape[2]
        q32 = q if q.dtype is T.float32 else q.float()
        k32 = k if k.dtype is T.float32 else k.float()
        scores = _ops.matmul(q32, k32.transpose(-1, -2).contiguous()) * (1.0 / float(np.sqrt(d)))
        if mask is not None:
            if mask.dtype is T.bool_:
                scores = _ops.masked_fill(scores, _broadcast_to(mask, scores.shape).logical_not(), float("-inf"))
            else:
                scores = scores + (mask if mask.dtype is T.float32 else mask.float())
        if is_causal:
            keep = T.from_numpy(np.tril(np.ones((lq, lk), dtype=bool))).to(q.device)
            scores = _ops.masked_fill(scores, keep.logical_not(), float("-inf"))
        w = _ops.softmax(scores, dim=-1)
        if average:
            ones = T.ones([1, h], dtype=T.float32, device=q.device)
            w = (_ops.matmul(ones, w.reshape(b, h, lq * lk)) * (1.0 / h)).reshape(b, lq, lk)
        if w.dtype is not q.dtype:
            w = w.to(dtype=q.dtype)
        return w.squeeze(0) if unbatched else w

    def forward(self, query, key, value, key_padding_mask=None, need_weights=True, attn_mask=None,
                average_attn_weights=True, is_causal=False):
        q_bf, q_unb = self._as_batch_first(query)
        k_bf, k_unb = self._as_batch_first(key)
        v_bf, v_unb = self._as_batch_first(value)
        if k_unb != q_unb or v_unb != q_unb:
            raise ValueError("query, key, and value must agree on batching")
        if q_bf.shape[2] != self.embed_dim or k_bf.shape[2] != self.kdim or v_bf.shape[2] != self.vdim:
            raise ValueError("query, key, and value embedding dimensions must match configured dimensions")
        E = self.embed_dim
        ib = self.in_proj_bias
        bq = None if ib is None else ib.narrow(0, 0, E)
        bk = None if ib is None else ib.narrow(0, E, E)
        bv = None if ib is None else ib.narrow(0, 2 * E, E)
        if self._qkv_same_embed_dim and query is key and key is value:
            qkv = functional.linear(q_bf, self.in_proj_weight, ib)  # one (3E x E) GEMM
            q_p, k_p, v_p = qkv.narrow(2, 0, E), qkv.narrow(2, E, E), qkv.narrow(2, 2 * E, E)
        elif self._qkv_same_embed_dim:
            w = self.in_proj_weight
            q_p = functional.linear(q_bf, w.narrow(0, 0, E), bq)
            k_p = functional.linear(k_bf, w.narrow(0, E, E), bk)
            v_p = functional.linear(v_bf, w.narrow(0, 2 * E, E), bv)
        else:
            q_p = functional.linear(q_bf, self.q_proj_weight, bq)
            k_p = functional.linear(k_bf, self.k_proj_weight, bk)
            v_p = functional.linear(v_bf, self.v_proj_weight, bv)
        k_p, v_p, key_padding_mask, attn_mask = self._append_bias_kv(k_p, v_p, key_padding_mask, attn_mask)
        k_p, v_p, key_padding_mask, attn_mask = self._append_zero_kv(k_p, v_p, key_padding_mask, attn_mask)
        qh, kh, vh = self._split_heads(q_p), self._split_heads(k_p), self._split_heads(v_p)
        merged = None
        if attn_mask is not None or key_padding_mask is not None:
            merged = self._merge_attention_masks(attn_mask, key_padding_mask, qh.shape[0], kh.shape[2])
        p = self.dropout if self.training else 0.0
        att = functional.scaled_dot_product_attention(qh, kh, vh, merged, p, is_causal)
        m = self._merge_heads(att)
        b, n, _ = m.shape
        out = self.out_proj(m.reshape(b * n, E)).reshape(b, n, E)
        weights = None
        if need_weights:
            weights = self._attention_weights(qh, kh, merged, is_causal, average_attn_weights, q_unb)
        return self._restore_layout(out, q_unb), weights


def _broadcast_to(t, shape):
    shape = list(shape)
    return t if list(t.shape) == shape else t.expand(shape)
