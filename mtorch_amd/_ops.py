"""Device implementations of the hot-path operators.

Each public op validates its arguments the way mtorch does (same exception classes and
messages: the binding's same-dtype rules module.cpp:6000-6033 raise RuntimeError, the core's
std::invalid_argument surfaces as ValueError, module.cpp:792-808), allocates a contiguous
output and makes one call into libmthip on the tensors' GPU.  There is no CPU path here: an
op handed CPU tensors raises, naming the operator and device, as the reference's planned
`unsupported_device` does (docs/design/08-phase5-device-layer.md:700-705).
"""

from __future__ import annotations

import ctypes
import math

import numpy as np

from . import _lib
from . import _random
from . import _tensor as T
from ._tensor import Tensor

_BIN = {"add": 0, "mul": 1, "sub": 2, "div": 3}
_UNARY = {"silu": 0, "gelu": 1, "gelu_tanh": 2, "exp": 3, "sin": 4, "cos": 5, "neg": 6, "sigmoid": 7, "relu": 8}
ACT_NONE, ACT_GELU, ACT_GELU_TANH, ACT_SILU = 0, 1, 2, 3


def unsupported(op: str, dev) -> RuntimeError:
    return RuntimeError(f"mtorch: operator '{op}' is not implemented for device '{getattr(dev, 'type', dev)}'")


def _gpu(op: str, *tensors) -> int:
    """Common guards: every tensor on the same GPU, no autograd (guard G1 of the reference's
    device plan, docs/design/10-phase7-cuda-backend.md:320-340).  Returns the device index."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        d = t.device
        if d.type != "cuda":
            raise unsupported(op, d)
        idx = T._device_index(d)
        if dev is None:
            dev = idx
        elif dev != idx:
            raise RuntimeError(f"{op}: expected all tensors to be on the same device")
    if T.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        raise RuntimeError(
            f"mtorch: operator '{op}' is not implemented for device 'cuda' with autograd; "
            "run inference under mtorch.no_grad()"
        )
    return dev


def _empty(sizes, dt, dev: int) -> Tensor:
    sizes = [int(s) for s in sizes]
    st = T.Storage(dt, T._numel(sizes), T.device(f"cuda:{dev}"))
    return Tensor(st, sizes, T.contiguous_strides(sizes))


def _ptr(t):
    return None if t is None else t.data_ptr()


def _L():
    return _lib.lib()


def _same_dtype(op, tensors, what="operands"):
    tensors = [t for t in tensors if t is not None]
    dt = tensors[0].dtype
    for t in tensors:
        if t.dtype is not dt:
            raise RuntimeError(f"expected {op} {what} to have the same dtype")
    if dt is T.bool_:
        raise RuntimeError(f"{op} is not implemented for bool tensors")
    return dt


def _float_dtype(op, dt):
    if dt not in (T.float16, T.float32):
        raise unsupported(f"{op}[{dt.name}]", "cuda")


# ------------------------------------------------------------------------------ movement


def to(t: Tensor, dt, dev, copy=False) -> Tensor:
    """mtorch::to (tensor.cpp:8479-8508) across host and device."""
    src_dev = t.device
    if dev.type == "mps":
        raise NotImplementedError("'mps' device storage is not implemented")
    same_dev = src_dev.type == dev.type and T._device_index(src_dev) == T._device_index(dev)
    if same_dev and dt is t.dtype:
        return contiguous_copy(t) if copy else t
    if src_dev.type == "cpu" and dev.type == "cpu":
        host = np.ascontiguousarray(t._host_view()).reshape(-1)
        out = _random.host_cast(host, t.dtype, dt)
        sizes = list(t.shape)
        return Tensor(T.Storage(dt, out.size, dev, host=out), sizes, T.contiguous_strides(sizes), 0, t.requires_grad)
    if src_dev.type == "cpu":
        di = T._device_index(dev)
        host = np.ascontiguousarray(t._host_view()).reshape(-1)
        staged = _empty(t.shape, t.dtype, di)
        if host.size:
            _lib.check(_L().mthip_memcpy_h2d(di, staged.data_ptr(), host.ctypes.data, host.nbytes))
        out = staged if dt is t.dtype else cast(staged, dt)
        out.requires_grad = t.requires_grad
        return out
    # device source
    src = t if dt is t.dtype else cast(t, dt)
    src = src.contiguous()
    if dev.type == "cpu":
        n = src.numel()
        host = np.empty(n, dtype=dt.np)
        if n:
            _lib.check(_L().mthip_memcpy_d2h(src._dev(), host.ctypes.data, src.data_ptr(), host.nbytes))
        sizes = list(t.shape)
        return Tensor(T.Storage(dt, n, dev, host=host), sizes, T.contiguous_strides(sizes), 0, t.requires_grad)
    di = T._device_index(dev)
    if di == src._dev():
        out = src if (src is not t or not copy) else contiguous_copy(src)
        return out
    raise NotImplementedError("copies between two GPUs are not part of this single-GPU backend")


def cast(t: Tensor, dt) -> Tensor:
    """Device dtype conversion with mtorch's rounding (mthip_cast)."""
    dev = T._device_index(t.device)
    src = t.contiguous()
    out = _empty(t.shape, dt, dev)
    n = out.numel()
    if n:
        _lib.check(_L().mthip_cast(dev, src.dtype.code, src.data_ptr(), dt.code, out.data_ptr(), n))
    return out


def contiguous_copy(t: Tensor) -> Tensor:
    if t.device.type == "cpu":
        host = np.ascontiguousarray(t._host_view()).reshape(-1).copy()
        sizes = list(t.shape)
        return Tensor(T.Storage(t.dtype, host.size, t.device, host=host), sizes, T.contiguous_strides(sizes), 0, t.requires_grad)
    dev = t._dev()
    out = _empty(t.shape, t.dtype, dev)
    n = out.numel()
    if n:
        rank = t.dim()
        _lib.check(_L().mthip_copy_strided(dev, t.dtype.code, t.data_ptr(), rank, _lib.int64_array(t.shape),
                                           _lib.int64_array(t.stride()), out.data_ptr()))
    out.requires_grad = t.requires_grad
    return out


def _last_writes(dst: Tensor, src: Tensor):
    """The elements of dst that the reference's copy writes last.  Tensor::copy_from
    (tensor.cpp:8335-8338) writes every index in row-major order, so along a zero-stride
    (expanded) dimension of dst the last index wins; only that index of dst and of the
    same-shaped src is kept.  (Expansion is the only way a view here overlaps itself.)"""
    for d in range(dst.dim()):
        if dst.stride(d) == 0 and dst.shape[d] > 1:
            dst = dst.narrow(d, dst.shape[d] - 1, 1)
            src = src.narrow(d, src.shape[d] - 1, 1)
    return dst, src


def copy_into(dst: Tensor, src: Tensor) -> None:
    """dst[...] = src with broadcasting and dtype conversion (Tensor::copy_from)."""
    if not isinstance(src, Tensor):
        fill_(dst, float(src))
        return
    src = src.expand(dst.shape) if list(src.shape) != list(dst.shape) else src
    dst, src = _last_writes(dst, src)
    if dst.device.type == "cpu":
        vals = np.ascontiguousarray((src if src.device.type == "cpu" else src.cpu())._host_view())
        if src.dtype is not dst.dtype:
            vals = _random.host_cast(vals.reshape(-1), src.dtype, dst.dtype).reshape(vals.shape)
        itemsize = dst.dtype.itemsize
        view = np.lib.stride_tricks.as_strided(
            dst._storage.host[dst._offset:], shape=tuple(dst.shape), strides=tuple(s * itemsize for s in dst.stride())
        )
        view[...] = vals
        dst._storage.version += 1
        return
    dev = dst._dev()
    if src.device.type == "cpu" or src.dtype is not dst.dtype:
        src = src.to(device=dst.device, dtype=dst.dtype)
    n = dst.numel()
    if n and dst.is_contiguous():
        _lib.check(_L().mthip_copy_strided(dev, dst.dtype.code, src.data_ptr(), src.dim(), _lib.int64_array(src.shape),
                                           _lib.int64_array(src.stride()), dst.data_ptr()))
    elif n:
        if src._storage is dst._storage:
            src = contiguous_copy(src)  # an overlapping source is staged before the strided write
        _lib.check(_L().mthip_copy_strided_to(dev, dst.dtype.code, src.data_ptr(), _lib.int64_array(src.stride()),
                                              dst.dim(), _lib.int64_array(dst.shape), dst.data_ptr(),
                                              _lib.int64_array(dst.stride())))
    dst._storage.version += 1


def fill_(t: Tensor, value) -> None:
    if t.device.type == "cpu":
        itemsize = t.dtype.itemsize
        view = np.lib.stride_tricks.as_strided(
            t._storage.host[t._offset:], shape=tuple(t.shape), strides=tuple(s * itemsize for s in t.stride())
        )
        if t.dtype is T.float16:
            view[...] = _random.float_to_half_bits(np.array([value], dtype=np.float32))[0]
        else:
            view[...] = value
        t._storage.version += 1
        return
    n = t.numel()
    if n and t.is_contiguous():
        _lib.check(_L().mthip_fill(t._dev(), t.dtype.code, t.data_ptr(), n, float(value)))
    elif n:
        _lib.check(_L().mthip_fill_strided(t._dev(), t.dtype.code, t.data_ptr(), t.dim(), _lib.int64_array(t.shape),
                                           _lib.int64_array(t.stride()), float(value)))
    t._storage.version += 1


def masked_fill(x: Tensor, mask: Tensor, value) -> Tensor:
    """masked_fill (tensor.cpp:13497-13610): a new contiguous tensor of x's dtype holding value
    (narrowed once, fp16 as float_to_half_bits((float)value)) where the bool mask -- broadcast to
    x's shape -- is true, x elsewhere."""
    if isinstance(value, Tensor):
        value = value.item()
    if mask.dtype is not T.bool_:
        raise ValueError("masked_fill mask must be a bool tensor")
    if list(T._broadcast_shape(list(x.shape), list(mask.shape))) != list(x.shape):
        raise ValueError("masked_fill mask is not broadcastable to input")
    dev = _gpu("masked_fill", x, mask)
    out = _empty(list(x.shape), x.dtype, dev)
    m = mask.expand(x.shape) if list(mask.shape) != list(x.shape) else mask
    _lib.check(_L().mthip_masked_fill(dev, x.dtype.code, x.data_ptr(), _lib.int64_array(x.stride()), m.data_ptr(),
                                      _lib.int64_array(m.stride()), float(value), out.data_ptr(), x.dim(),
                                      _lib.int64_array(x.shape)))
    return out


def logical_not(x: Tensor) -> Tensor:
    """logical_not (tensor.cpp:14616) of a bool tensor: a new contiguous bool tensor."""
    if x.dtype is not T.bool_:
        raise NotImplementedError("mtorch_amd: logical_not is implemented for bool tensors")
    dev = _gpu("logical_not", x)
    x = x if x.is_contiguous() else x.contiguous()
    out = _empty(list(x.shape), T.bool_, dev)
    if x.numel():
        _lib.check(_L().mthip_logical_not(dev, x.data_ptr(), out.data_ptr(), x.numel()))
    return out


# ------------------------------------------------------------------------------ elementwise


def binary(a, b, op: str) -> Tensor:
    """binary_tensor_tensor / binary_tensor_scalar (tensor.cpp:18965-19176) for add/sub/mul/div."""
    a_t, b_t = isinstance(a, Tensor), isinstance(b, Tensor)
    if a_t and b_t:
        dev = _gpu(op, a, b)
        dt = T.promote_types(a.dtype, b.dtype)
        _float_dtype(op, dt)
        if a.dtype is not dt:
            a = cast(a, dt)
        if b.dtype is not dt:
            b = cast(b, dt)
        shape = T._broadcast_shape(list(a.shape), list(b.shape))
        out = _empty(shape, dt, dev)
        if out.numel() == 0:
            return out
        rank = len(shape)

        def aligned(t):
            pad = rank - t.dim()
            strides = [0] * pad + list(t.stride())
            sizes = [1] * pad + list(t.shape)
            return [0 if sizes[i] == 1 and shape[i] != 1 else strides[i] for i in range(rank)]

        _lib.check(_L().mthip_binary(dev, _BIN[op], dt.code, a.data_ptr(), _lib.int64_array(aligned(a)), b.data_ptr(),
                                     _lib.int64_array(aligned(b)), out.data_ptr(), rank, _lib.int64_array(shape)))
        return out
    if not a_t and not b_t:
        raise TypeError("binary op expects at least one tensor")
    t, scalar, scalar_first = (a, b, False) if a_t else (b, a, True)
    dev = _gpu(op, t)
    _float_dtype(op, t.dtype)
    src = t.contiguous()
    out = _empty(t.shape, t.dtype, dev)
    n = out.numel()
    if n:
        _lib.check(_L().mthip_binary_scalar(dev, _BIN[op], t.dtype.code, src.data_ptr(), float(scalar),
                                            1 if scalar_first else 0, out.data_ptr(), n))
    return out


def add(a, b, alpha=1):
    return binary(a, binary(b, alpha, "mul") if alpha != 1 else b, "add")


def unary(t: Tensor, name: str) -> Tensor:
    dev = _gpu(name, t)
    _float_dtype(name, t.dtype)
    src = t.contiguous()
    out = _empty(t.shape, t.dtype, dev)
    n = out.numel()
    if n:
        _lib.check(_L().mthip_unary(dev, _UNARY[name], t.dtype.code, src.data_ptr(), out.data_ptr(), n))
    return out


def gelu(t: Tensor, approximate="none") -> Tensor:
    """gelu (tensor.cpp:17207-17288)."""
    if approximate not in ("none", "tanh"):
        raise ValueError("gelu approximate must be 'none' or 'tanh'")
    return unary(t, "gelu" if approximate == "none" else "gelu_tanh")


def silu(t: Tensor) -> Tensor:
    """silu (tensor.cpp:16480-16613)."""
    return unary(t, "silu")


def geglu(t: Tensor) -> Tensor:
    """a * gelu(gate) for (a, gate) = t.chunk(2, -1): the SD feed-forward gate, with each op's
    own rounding (gelu narrowed, then the product narrowed)."""
    dev = _gpu("geglu", t)
    _float_dtype("geglu", t.dtype)
    two_d = t.shape[-1]
    if two_d % 2:
        raise ValueError("geglu expects an even last dimension")
    src = t.contiguous()
    out = _empty(list(t.shape[:-1]) + [two_d // 2], t.dtype, dev)
    rows = out.numel() // max(two_d // 2, 1)
    if out.numel():
        _lib.check(_L().mthip_geglu(dev, t.dtype.code, src.data_ptr(), out.data_ptr(), rows, two_d // 2))
    return out


# ------------------------------------------------------------------------------ contractions


def _rowmajor_2d(t: Tensor):
    """(tensor, ld) with unit stride on the last dim, copying only when needed."""
    if t.stride(-1) == 1 and (t.dim() < 2 or t.stride(-2) >= t.shape[-1] or t.shape[-2] <= 1):
        return t, (t.stride(-2) if t.dim() >= 2 and t.shape[-2] > 1 else t.shape[-1])
    c = t.contiguous()
    return c, c.shape[-1]


def _rows_view(x: Tensor):
    """x[..., K] as M rows of K with one row stride (lda), or None if not expressible."""
    K = x.shape[-1]
    if x.dim() == 1:
        return (1, K) if x.stride(0) == 1 or K <= 1 else None
    if x.stride(-1) != 1 and K > 1:
        return None
    outer = list(x.shape[:-1])
    ostr = list(x.stride()[:-1])
    # collapse the outer dims into one stride
    lda = None
    expect = None
    for size, stride in zip(reversed(outer), reversed(ostr)):
        if size == 1:
            continue
        if lda is None:
            lda = stride
            expect = stride * size
        elif stride != expect:
            return None
        else:
            expect = stride * size
    if lda is None:
        lda = K
    if lda < K:
        return None
    return T._numel(outer), lda


def linear(x: Tensor, w: Tensor, b: Tensor = None, act: int = ACT_NONE, residual: Tensor = None) -> Tensor:
    """mtorch::linear (tensor.cpp:31401-31694), binding py_linear (module.cpp:6778-6804).

    act/residual are fusions used by this package's modules: y = act(linear(x)) (+ residual),
    each step narrowed as the separate ops would be."""
    _same_dtype("linear", [x, w, b])
    dev = _gpu("linear", x, w, b, residual)
    if x.dim() < 1 or w.dim() != 2:
        raise ValueError("linear expects an input with at least 1 dimension and a 2-D weight")
    K = x.shape[-1]
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError("linear input and weight shapes cannot be multiplied")
    out_shape = list(x.shape[:-1]) + [N]
    if b is not None:
        try:
            if T._broadcast_shape(list(b.shape), out_shape) != out_shape:
                raise ValueError
        except ValueError:
            raise ValueError("linear bias is not broadcastable to the output shape") from None
    dt = x.dtype
    _float_dtype("linear", dt)
    rv = _rows_view(x)
    if rv is None:
        x = x.contiguous()
        rv = _rows_view(x)
    M, lda = rv
    w2, ldw = _rowmajor_2d(w)
    bias_vec = None
    post_bias = None
    if b is not None:
        if b.numel() == N and (b.dim() == 1 or all(s == 1 for s in b.shape[:-1])):
            bias_vec = b.reshape(N).contiguous()
        else:
            post_bias = b
    out = _empty(out_shape, dt, dev)
    res_ptr, ld_res = None, 0
    if residual is not None:
        if list(residual.shape) != out_shape:
            raise ValueError("linear residual must have the output shape")
        residual = residual.contiguous()
        res_ptr, ld_res = residual.data_ptr(), N
    if post_bias is not None and (act != ACT_NONE or residual is not None):
        raise ValueError("fused linear epilogues need a [out_features] bias")
    if out.numel():
        _lib.check(_L().mthip_linear(dev, dt.code, x.data_ptr(), lda, w2.data_ptr(), ldw, _ptr(bias_vec),
                                     out.data_ptr(), N, M, N, K, act, res_ptr, ld_res))
    if post_bias is not None:
        out = binary(out, post_bias, "add")
    return out


def linear_geglu(x: Tensor, w: Tensor, b: Tensor = None) -> Tensor:
    """a * gelu(gate) with (a, gate) = linear(x, w, b).chunk(2, dim=-1): the GEGLU projection of
    the SD feed-forward as one GEMM whose epilogue pairs each value column with its gate
    (mthip_linear_geglu); the weight/bias row interleave it needs is built once per weight
    version and kept on the weight's storage.  Shapes the fused kernel does not take run as
    linear then geglu."""
    _same_dtype("linear", [x, w, b])
    dev = _gpu("linear", x, w, b)
    if w.dim() != 2 or x.dim() < 1 or w.shape[1] != x.shape[-1]:
        raise ValueError("linear input and weight shapes cannot be multiplied")
    K, N2 = x.shape[-1], w.shape[0]
    vec = 8 if x.dtype is T.float16 else 4
    rv = _rows_view(x)
    if N2 % 64 or K % vec or (b is not None and list(b.shape) != [N2]) or rv is None or rv[1] % vec \
            or x.data_ptr() % 16 or not w.is_contiguous() or w.data_ptr() % 16:
        return geglu(linear(x, w, b))
    _float_dtype("linear", x.dtype)
    M, lda = rv
    N = N2 // 2
    wp, bp = _geglu_packed(w, b)
    out = _empty(list(x.shape[:-1]) + [N], x.dtype, dev)
    if out.numel():
        _lib.check(_L().mthip_linear_geglu(dev, x.dtype.code, x.data_ptr(), lda, wp.data_ptr(), _ptr(bp), out.data_ptr(),
                                           N, M, N, K))
    return out


def _geglu_packed(w: Tensor, b: Tensor):
    """w/b with rows interleaved in 32-row blocks (value block q, then gate block q), cached on
    w's storage and rebuilt after an in-place write to w or b."""
    st = w._storage
    N2, K = w.shape
    key = ("geglu", w._offset, N2, K, id(b._storage) if b is not None else None, b._offset if b is not None else 0)
    ver = (st.version, b._storage.version if b is not None else 0)
    if st.packs is None:
        st.packs = {}
    hit = st.packs.get(key)
    if hit is not None and hit[0] == ver:
        return hit[1], hit[2]
    q = N2 // 64
    wp = w.reshape(2, q, 32, K).permute(1, 0, 2, 3).contiguous().reshape(N2, K)
    bp = b.reshape(2, q, 32).permute(1, 0, 2).contiguous().reshape(N2) if b is not None else None
    st.packs[key] = (ver, wp, bp)
    return wp, bp


def _gemm(a: Tensor, b: Tensor, out: Tensor, batch, M, N, K, sa, sb, alpha=1.0, beta=0.0, c_in=None,
          c_rs=0, c_cs=0, c_bs=0):
    """out[batch,M,N] = alpha*a.b (+beta*c_in); a/b are [batch?, M, K] / [batch?, K, N] views."""
    dev = out._dev()
    # A: needs unit stride along K.
    if a.stride(-1) != 1 and K > 1:
        a = a.contiguous()
        sa = M * K if sa else 0
    lda = a.stride(-2) if M > 1 else K
    if lda < K:
        a = a.contiguous()
        lda, sa = K, (M * K if sa else 0)
    # B: [K, N] with unit stride along N (NN), or a transposed [N, K] matrix (NT).
    if b.stride(-1) == 1 or N == 1:
        b_trans, ldb = 0, (b.stride(-2) if K > 1 else N)
        if ldb < N:
            b = b.contiguous()
            b_trans, ldb, sb = 0, N, (K * N if sb else 0)
    elif b.stride(-2) == 1:
        b_trans, ldb = 1, b.stride(-1)
        if ldb < K:
            b = b.contiguous()
            b_trans, ldb, sb = 0, N, (K * N if sb else 0)
    else:
        b = b.contiguous()
        b_trans, ldb, sb = 0, N, (K * N if sb else 0)
    _lib.check(_L().mthip_gemm(dev, out.dtype.code, batch, M, N, K, a.data_ptr(), lda, sa, b.data_ptr(), ldb, sb,
                               b_trans, out.data_ptr(), N, M * N, float(alpha), float(beta), _ptr(c_in), c_rs, c_cs,
                               c_bs))


def _collapse_batch(t: Tensor, nb: int):
    """Single stride for the first nb (batch) dims, or None."""
    sizes, strides = list(t.shape[:nb]), list(t.stride()[:nb])
    stride, expect = None, None
    for s, st in zip(reversed(sizes), reversed(strides)):
        if s == 1:
            continue
        if stride is None:
            stride, expect = st, st * s
        elif st != expect:
            return None
        else:
            expect = st * s
    return 0 if stride is None else stride


def matmul(a: Tensor, b: Tensor) -> Tensor:
    """mtorch::matmul (tensor.cpp:24896-25064) incl. batched_matmul broadcasting (:24822)."""
    if not isinstance(a, Tensor) or not isinstance(b, Tensor):
        raise TypeError("matmul expected tensors")
    _same_dtype("matmul", [a, b])
    dev = _gpu("matmul", a, b)
    _float_dtype("matmul", a.dtype)
    if a.dim() == 0 or b.dim() == 0:
        raise ValueError("matmul expects both arguments to be at least 1-D")
    squeeze_m = a.dim() == 1
    squeeze_n = b.dim() == 1
    a2 = a.unsqueeze(0) if squeeze_m else a
    b2 = b.unsqueeze(1) if squeeze_n else b
    M, K = a2.shape[-2], a2.shape[-1]
    K2, N = b2.shape[-2], b2.shape[-1]
    if K != K2:
        raise ValueError("matmul shape mismatch")
    batch_shape = T._broadcast_shape(list(a2.shape[:-2]), list(b2.shape[:-2]))
    out_shape = batch_shape + [M, N]
    out = _empty(out_shape, a.dtype, dev)
    nb = len(batch_shape)
    bcount = T._numel(batch_shape)
    if out.numel():
        ae = a2.expand(batch_shape + [M, K])
        be = b2.expand(batch_shape + [K, N])
        sa = _collapse_batch(ae, nb) if nb else 0
        if sa is None:
            ae = ae.contiguous()
            sa = M * K
        sb = _collapse_batch(be, nb) if nb else 0
        if sb is None:
            be = be.contiguous()
            sb = K * N
        _gemm(ae, be, out, bcount, M, N, K, sa, sb)
    result_shape = list(out_shape)
    if squeeze_n:
        result_shape.pop(-1)
    if squeeze_m:
        result_shape.pop(-2 if not squeeze_n else -1)
    if result_shape != out_shape:
        out = out.reshape(result_shape)
    return out


def bmm(a: Tensor, b: Tensor) -> Tensor:
    if a.dim() != 3 or b.dim() != 3:
        raise ValueError("bmm expects 3-D tensors")
    if a.shape[0] != b.shape[0]:
        raise ValueError("bmm batch sizes must match")
    return matmul(a, b)


def addmm(inp: Tensor, m1: Tensor, m2: Tensor, beta=1.0, alpha=1.0) -> Tensor:
    """mtorch::addmm (tensor.cpp:25184-25366), binding py_addmm (module.cpp:6396-6419)."""
    _same_dtype("addmm", [inp, m1, m2])
    dev = _gpu("addmm", inp, m1, m2)
    _float_dtype("addmm", m1.dtype)
    if m1.dim() != 2 or m2.dim() != 2:
        raise ValueError("addmm expects 2-D mat1 and mat2 tensors")
    M, K = m1.shape
    K2, N = m2.shape
    if K != K2:
        raise ValueError("addmm matrix shapes cannot be multiplied")
    try:
        ok = T._broadcast_shape(list(inp.shape), [M, N]) == [M, N]
    except ValueError:
        ok = False
    if not ok:
        raise ValueError("addmm input is not broadcastable to the matrix product shape")
    e = inp.expand(M, N)
    out = _empty([M, N], m1.dtype, dev)
    if out.numel():
        # beta * input is stored even at beta = 0 (an inf/NaN input gives NaN, tensor.cpp:25256);
        # at alpha = 0 the library skips the product, as the reference does (tensor.cpp:25320).
        _gemm(m1, m2, out, 1, M, N, K, 0, 0, alpha, beta, e, e.stride(0), e.stride(1), 0)
    return out


def baddbmm(inp: Tensor, b1: Tensor, b2: Tensor, beta=1.0, alpha=1.0) -> Tensor:
    """baddbmm (tensor.cpp:25557): out[i] = beta*inp[i] + alpha*b1[i].b2[i]."""
    _same_dtype("baddbmm", [inp, b1, b2])
    dev = _gpu("baddbmm", inp, b1, b2)
    _float_dtype("baddbmm", b1.dtype)
    if b1.dim() != 3 or b2.dim() != 3 or b1.shape[0] != b2.shape[0] or b1.shape[2] != b2.shape[1]:
        raise ValueError("baddbmm expects batch1 [B,M,K] and batch2 [B,K,N]")
    B, M, K = b1.shape
    N = b2.shape[2]
    e = inp.expand(B, M, N)
    out = _empty([B, M, N], b1.dtype, dev)
    if out.numel():
        # beta * input always stored (tensor.cpp:1452); product skipped at alpha = 0 (:25621).
        sa = _collapse_batch(b1, 1)
        sb = _collapse_batch(b2, 1)
        _gemm(b1, b2, out, B, M, N, K, sa, sb, alpha, beta, e, e.stride(1), e.stride(2), e.stride(0))
    return out


def _pair(v, name):
    if isinstance(v, int):
        return (v, v)
    v = tuple(int(x) for x in v)
    if len(v) == 1:
        return (v[0], v[0])
    if len(v) != 2:
        raise ValueError(f"conv2d {name} must have 1 or 2 values")
    return v


def _conv2d_plan(x: Tensor, w: Tensor, b: Tensor, stride, padding, dilation, groups):
    """Argument checks and output geometry of mtorch::conv2d (tensor.cpp:26490-26560,
    conv2d_output_size :25941, normalize_conv2d_pair :25901); string padding resolved as the
    Python layer's _conv2d does (mtorch/__init__.py:3280-3287)."""
    if x.dim() not in (3, 4):
        raise ValueError("conv2d expects a 3-D or 4-D input tensor")
    if w.dim() != 4:
        raise ValueError("conv2d expects a 4-D weight tensor")
    if groups <= 0:
        raise ValueError("conv2d groups must be positive")
    sh, sw = _pair(stride, "stride")
    dh, dw = _pair(dilation, "dilation")
    if sh <= 0 or sw <= 0 or dh <= 0 or dw <= 0:
        raise ValueError("conv2d stride and dilation must be positive")
    unbatched = x.dim() == 3
    B, C, H, W = ([1] + list(x.shape)) if unbatched else list(x.shape)
    O, Cg, KH, KW = w.shape
    if isinstance(padding, str):
        if padding == "valid":
            ph = pw = 0
        elif padding == "same":
            if sh != 1 or sw != 1:
                raise ValueError("padding='same' is not supported for strided convolutions")
            th, tw = dh * (KH - 1), dw * (KW - 1)
            if th % 2 or tw % 2:
                raise NotImplementedError("asymmetric 'same' padding is not supported on the device")
            ph, pw = th // 2, tw // 2
        else:
            raise ValueError("padding must be 'same', 'valid' or an int/tuple")
    else:
        ph, pw = _pair(padding, "padding")
        if ph < 0 or pw < 0:
            raise ValueError("conv2d padding must be non-negative")
    if C != Cg * groups:
        raise ValueError("conv2d input channels must equal weight channels times groups")
    if O % groups != 0:
        raise ValueError("conv2d output channels must be divisible by groups")
    if b is not None and not (b.dim() == 1 and b.shape[0] == O):
        raise ValueError("conv2d bias must be 1-D with out_channels elements")
    OH = (H + 2 * ph - dh * (KH - 1) - 1) // sh + 1
    OW = (W + 2 * pw - dw * (KW - 1) - 1) // sw + 1
    if OH <= 0 or OW <= 0:
        raise ValueError("conv2d output size must be positive")
    _float_dtype("conv2d", x.dtype)
    return dict(B=B, C=C, H=H, W=W, O=O, KH=KH, KW=KW, sh=sh, sw=sw, ph=ph, pw=pw, dh=dh, dw=dw, OH=OH, OW=OW,
                unbatched=unbatched)


def conv2d(x: Tensor, w: Tensor, b: Tensor = None, stride=1, padding=0, dilation=1, groups=1,
           residual: Tensor = None) -> Tensor:
    """mtorch::conv2d (tensor.cpp:26490-27528), binding py_conv2d (module.cpp:6912-6961).
    `residual` (same shape as the output) is added after the conv result is narrowed."""
    _same_dtype("conv2d", [x, w, b], "tensors")
    dev = _gpu("conv2d", x, w, b, residual)
    p = _conv2d_plan(x, w, b, stride, padding, dilation, groups)
    B, C, H, W, O, KH, KW = p["B"], p["C"], p["H"], p["W"], p["O"], p["KH"], p["KW"]
    geo = (p["sh"], p["sw"], p["ph"], p["pw"], p["dh"], p["dw"])
    xc = (x.unsqueeze(0) if p["unbatched"] else x).contiguous()
    wc = w.contiguous()
    bc = _contig(b)
    out = _empty([B, O, p["OH"], p["OW"]], x.dtype, dev)
    rc = _conv_residual(residual, out)
    if out.numel():
        if groups == 1:
            wp = _conv_packed_weight(wc, dev, O, C, KH, KW)
            _lib.check(_L().mthip_conv2d_prepacked(dev, x.dtype.code, xc.data_ptr(), wp, _ptr(bc), out.data_ptr(), B,
                                                   C, H, W, O, KH, KW, *geo, _ptr(rc)))
        else:
            _lib.check(_L().mthip_conv2d(dev, x.dtype.code, xc.data_ptr(), wc.data_ptr(), _ptr(bc), out.data_ptr(), B,
                                         C, H, W, O, KH, KW, *geo, groups, _ptr(rc)))
    return out.squeeze(0) if p["unbatched"] else out


def _contig(t):
    return t.contiguous() if t is not None else None


def _conv_residual(residual, out):
    if residual is None:
        return None
    if list(residual.shape) != list(out.shape):
        raise ValueError("conv2d residual must have the output shape")
    return residual.contiguous()


def group_norm_silu_conv2d(x: Tensor, num_groups: int, gn_weight: Tensor, gn_bias: Tensor, eps, w: Tensor,
                           b: Tensor = None, stride=1, padding=0, dilation=1, residual: Tensor = None,
                           chan_add: Tensor = None) -> Tensor:
    """conv2d(silu(group_norm(x, num_groups, gn_weight, gn_bias, eps)), w, b, ...)
    (+ chan_add[:, :, None, None]) (+ residual): the GroupNorm -> SiLU -> conv chain of an SD
    ResNet block, with its time-embedding add (the reference runs these as separate ops,
    tensor.cpp:18643, 16480, 26490, 18965).  On the device the normalised activation is written
    once, channels-last, in the layout the implicit-GEMM conv reads (mthip_group_norm_nhwc then
    mthip_conv2d_nhwc), and the adds happen in the conv's epilogue; values equal the unfused
    sequence's.  chan_add is [B, O] (rows may be strided).  fp32 GroupNorm parameters over an fp16
    input mean the upcast pattern silu(group_norm(x.float(), ...).half())."""
    pdt = _norm_param_dtype("group_norm", x, gn_weight, gn_bias)
    _same_dtype("conv2d", [x, w, b, chan_add], "tensors")
    dev = _gpu("group_norm_silu_conv2d", x, gn_weight, gn_bias, w, b, residual, chan_add)
    if x.dim() != 4:
        raise ValueError("group_norm_silu_conv2d expects a 4-D input tensor")
    _group_norm_check(x, num_groups, gn_weight, gn_bias)
    p = _conv2d_plan(x, w, b, stride, padding, dilation, 1)
    B, C, H, W, O, KH, KW = p["B"], p["C"], p["H"], p["W"], p["O"], p["KH"], p["KW"]
    out = _empty([B, O, p["OH"], p["OW"]], x.dtype, dev)
    rc = _conv_residual(residual, out)
    ca, ca_ld = None, 0
    if chan_add is not None:
        if list(chan_add.shape) != [B, O]:
            raise ValueError("group_norm_silu_conv2d: chan_add must be [batch, out_channels]")
        ok = chan_add.stride(1) == 1 and (B == 1 or chan_add.stride(0) >= O)
        ca = chan_add if ok else chan_add.contiguous()
        ca_ld = ca.stride(0) if B > 1 else O
    if out.numel():
        L = _L()
        vec = 8 if x.dtype is T.float16 else 4
        Cp = -(-C // vec) * vec
        xn = T._DeviceBuffer(B * H * W * Cp * x.dtype.itemsize, dev)
        _lib.check(L.mthip_group_norm_nhwc(dev, x.dtype.code, x.contiguous().data_ptr(), _ptr(_contig(gn_weight)),
                                           _ptr(_contig(gn_bias)), xn.ptr, B, C, H * W, num_groups, float(eps), 1,
                                           pdt))
        wp = _conv_packed_weight(w.contiguous(), dev, O, C, KH, KW)
        _lib.check(L.mthip_conv2d_nhwc(dev, x.dtype.code, xn.ptr, wp, _ptr(_contig(b)), out.data_ptr(), B, C, H, W, O,
                                       KH, KW, p["sh"], p["sw"], p["ph"], p["pw"], p["dh"], p["dw"], _ptr(rc), _ptr(ca),
                                       ca_ld))
        del xn  # stream-ordered free: reused only by later work
    return out


def group_norm_silu_conv2d_cat(x0: Tensor, x1: Tensor, num_groups: int, gn_weight: Tensor, gn_bias: Tensor, eps,
                               w: Tensor, b: Tensor, padding, chan_add: Tensor, shortcut_w: Tensor, shortcut_b: Tensor):
    """The entry of an SD up-block ResBlock on x = cat([x0, x1], dim=1) (tensor.cpp:32141):
    returns (group_norm_silu_conv2d(x, ...), conv2d(x, shortcut_w, shortcut_b)) without the
    concatenated copy -- mthip_group_norm_nhwc_cat reads x0 and x1 in place and writes both the
    normalised activation and x itself channels-last, and the two convs read those.  Values
    equal the unfused cat -> group_norm -> silu -> conv2d / conv2d sequence's bit for bit.
    x1 = None: x = x0 (a ResBlock with a shortcut conv and one input; the shortcut then reads
    the GroupNorm's channels-last copy instead of a separate layout change).  Returns None when
    the inputs do not fit the channels-last fp16 kernel (the caller then concatenates)."""
    if x0.dtype is not T.float16 or x0.dim() != 4 or (x1 is not None and (x1.dtype is not T.float16 or x1.dim() != 4)):
        return None
    B, C0, H, W = x0.shape
    C1 = x1.shape[1] if x1 is not None else 0
    C = C0 + C1
    if (x1 is not None and list(x1.shape) != [B, C1, H, W]) or C % 8 or C0 % 2 or (H * W) % 8 or C % num_groups:
        return None
    pdt = _norm_param_dtype("group_norm", x0, gn_weight, gn_bias)
    _same_dtype("conv2d", [x0, x1, w, b, chan_add, shortcut_w, shortcut_b], "tensors")
    dev = _gpu("group_norm_silu_conv2d", x0, x1, gn_weight, gn_bias, w, b, chan_add, shortcut_w, shortcut_b)
    for t in (gn_weight, gn_bias):
        if t is not None and list(t.shape) != [C]:
            raise ValueError("group_norm weight and bias must have one entry per channel")
    O, KH, KW = w.shape[0], w.shape[2], w.shape[3]
    So = shortcut_w.shape[0]
    if list(w.shape[1:2]) != [C] or list(shortcut_w.shape[1:]) != [C, 1, 1]:
        raise ValueError("group_norm_silu_conv2d_cat: weight shapes do not match the concatenated input")
    ph, pw = _pair(padding, "padding")
    OH, OW = H + 2 * ph - KH + 1, W + 2 * pw - KW + 1
    out = _empty([B, O, OH, OW], x0.dtype, dev)
    sc = _empty([B, So, H, W], x0.dtype, dev)
    ca, ca_ld = None, 0
    if chan_add is not None:
        if list(chan_add.shape) != [B, O]:
            raise ValueError("group_norm_silu_conv2d: chan_add must be [batch, out_channels]")
        ok = chan_add.stride(1) == 1 and (B == 1 or chan_add.stride(0) >= O)
        ca = chan_add if ok else chan_add.contiguous()
        ca_ld = ca.stride(0) if B > 1 else O
    L = _L()
    xn = T._DeviceBuffer(B * H * W * C * 2, dev)
    raw = T._DeviceBuffer(B * H * W * C * 2, dev)
    _lib.check(L.mthip_group_norm_nhwc_cat(dev, x0.dtype.code, x0.contiguous().data_ptr(), C0,
                                           x1.contiguous().data_ptr() if x1 is not None else None, C1,
                                           _ptr(_contig(gn_weight)),
                                           _ptr(_contig(gn_bias)), xn.ptr, raw.ptr, B, H * W, num_groups, float(eps), 1,
                                           pdt))
    wp = _conv_packed_weight(w.contiguous(), dev, O, C, KH, KW)
    _lib.check(L.mthip_conv2d_nhwc(dev, x0.dtype.code, xn.ptr, wp, _ptr(_contig(b)), out.data_ptr(), B, C, H, W, O, KH,
                                   KW, 1, 1, ph, pw, 1, 1, None, _ptr(ca), ca_ld))
    swp = _conv_packed_weight(shortcut_w.contiguous(), dev, So, C, 1, 1)
    _lib.check(L.mthip_conv2d_nhwc(dev, x0.dtype.code, raw.ptr, swp, _ptr(_contig(shortcut_b)), sc.data_ptr(), B, C, H,
                                   W, So, 1, 1, 1, 1, 0, 0, 1, 1, None, None, 0))
    del xn, raw  # stream-ordered free: reused only by later work
    return out, sc


def upsample2x_conv2d(x: Tensor, w: Tensor, b: Tensor = None, padding=1) -> Tensor:
    """conv2d(interpolate(x, scale_factor=2, mode="nearest"), w, b, padding=padding) for fp16 NCHW
    x whose channel count is a whole number of 16-byte chunks: mthip_upsample2x_to_nhwc writes
    the upsampled input channels-last in one pass (no NCHW upsampled copy, no separate layout
    change) and mthip_conv2d_nhwc convolves it -- the SD decoder's Upsample block, bit for bit
    the two-op sequence.  Returns None where it does not apply (the caller runs the two ops)."""
    if x.dtype is not T.float16 or x.dim() != 4 or w.dim() != 4 or x.shape[1] % 8:
        return None
    _same_dtype("conv2d", [x, w, b], "tensors")
    dev = _gpu("conv2d", x, w, b)
    B, C, H, W = x.shape
    O, KH, KW = w.shape[0], w.shape[2], w.shape[3]
    if w.shape[1] != C:
        return None
    ph, pw = _pair(padding, "padding")
    H2, W2 = 2 * H, 2 * W
    OH, OW = H2 + 2 * ph - KH + 1, W2 + 2 * pw - KW + 1
    if OH <= 0 or OW <= 0:
        return None
    out = _empty([B, O, OH, OW], x.dtype, dev)
    L = _L()
    xp = T._DeviceBuffer(B * H2 * W2 * C * 2, dev)
    _lib.check(L.mthip_upsample2x_to_nhwc(dev, x.dtype.code, x.contiguous().data_ptr(), xp.ptr, B, C, C, H, W))
    wp = _conv_packed_weight(w.contiguous(), dev, O, C, KH, KW)
    _lib.check(L.mthip_conv2d_nhwc(dev, x.dtype.code, xp.ptr, wp, _ptr(_contig(b)), out.data_ptr(), B, C, H2, W2, O,
                                   KH, KW, 1, 1, ph, pw, 1, 1, None, None, 0))
    del xp  # stream-ordered free: reused only by later work
    return out


def conv2d_tokens(tok: Tensor, w: Tensor, b: Tensor, H: int, W: int, residual: Tensor = None) -> Tensor:
    """1x1 conv of a channels-last token tensor tok[B, H*W, C] to NCHW [B, O, H, W] (+ residual):
    conv2d(tok.reshape(B, H, W, C).permute(0, 3, 1, 2), w, b) without the permute -- the proj_out
    of an SD transformer block, whose epilogue adds the block's NCHW input."""
    _same_dtype("conv2d", [tok, w, b], "tensors")
    dev = _gpu("conv2d", tok, w, b, residual)
    B, L, C = tok.shape
    O = w.shape[0]
    if L != H * W or list(w.shape[1:]) not in ([C, 1, 1], [C]):
        raise ValueError("conv2d_tokens: token / weight shape mismatch")
    if C % (8 if tok.dtype is T.float16 else 4):
        raise ValueError("conv2d_tokens: the channel count must be a whole number of 16-byte chunks")
    out = _empty([B, O, H, W], tok.dtype, dev)
    rc = _conv_residual(residual, out)
    tc = tok.contiguous()
    wp = _conv_packed_weight(w.contiguous().reshape(O, C, 1, 1), dev, O, C, 1, 1)
    _lib.check(_L().mthip_conv2d_nhwc(dev, tok.dtype.code, tc.data_ptr(), wp, _ptr(_contig(b)), out.data_ptr(), B, C, H,
                                      W, O, 1, 1, 1, 1, 0, 0, 1, 1, _ptr(rc), None, 0))
    return out


def _conv_packed_weight(w: Tensor, dev: int, O: int, C: int, KH: int, KW: int) -> int:
    """Device pointer of w (contiguous [O, C, KH, KW]) packed for mthip_conv2d_prepacked.  The
    packed copy lives on w's storage, keyed by the view and tagged with the storage version, so
    it is rebuilt only after an in-place write to the weight (the role of the reference's
    Storage weight caches, tensor.h:65-78)."""
    st = w._storage
    key = ("conv2d", w._offset, O, C, KH, KW)
    if st.packs is None:
        st.packs = {}
    hit = st.packs.get(key)
    if hit is not None and hit[0] == st.version:
        return hit[1].ptr
    L = _L()
    nbytes = L.mthip_conv2d_packed_bytes(w.dtype.code, O, C, KH, KW)
    buf = T._DeviceBuffer(nbytes, dev)
    _lib.check(L.mthip_conv2d_pack_weight(dev, w.dtype.code, w.data_ptr(), buf.ptr, O, C, KH, KW))
    st.packs[key] = (st.version, buf)
    return buf.ptr


# ------------------------------------------------------------------------------ attention


def _batch_head_strides(t: Tensor, nprefix: int):
    """(batch_stride, head_stride) for prefix dims [*batch, heads], or None."""
    if nprefix == 0:
        return 0, 0
    head = t.stride(nprefix - 1) if t.shape[nprefix - 1] > 1 else 0
    if nprefix == 1:
        return 0, head
    bs = _collapse_batch(t, nprefix - 1)
    if bs is None:
        return None
    return bs, head


def scaled_dot_product_attention(query: Tensor, key: Tensor, value: Tensor, attn_mask: Tensor = None,
                                 dropout_p=0.0, is_causal=False, scale=None, enable_gqa=False) -> Tensor:
    """mtorch::scaled_dot_product_attention (tensor.cpp:30930-31324; sdpa_prefix_plan :30318-30391)."""
    for t in (query, key, value):
        if not t.dtype.is_floating_point:
            raise ValueError("scaled_dot_product_attention expects floating point query, key, and value")
    if query.dtype is not key.dtype or query.dtype is not value.dtype:
        raise ValueError("scaled_dot_product_attention query, key, and value must have the same dtype")
    if attn_mask is not None and attn_mask.dtype not in (T.bool_, T.float32, query.dtype):
        raise ValueError("scaled_dot_product_attention attn_mask must be bool, float32, or match query dtype")
    if dropout_p < 0.0 or dropout_p > 1.0:
        raise ValueError("scaled_dot_product_attention dropout_p must be between 0 and 1")
    dev = _gpu("scaled_dot_product_attention", query, key, value, attn_mask)
    _float_dtype("scaled_dot_product_attention", query.dtype)
    if query.dim() < 2 or key.dim() < 2 or value.dim() < 2:
        raise ValueError("scaled_dot_product_attention expects tensors with rank >= 2")
    if query.dim() != key.dim() or query.dim() != value.dim():
        raise ValueError("scaled_dot_product_attention query, key, and value ranks must match")
    rank = query.dim()
    E = query.shape[-1]
    if key.shape[-1] != E:
        raise ValueError("scaled_dot_product_attention query and key embedding dimensions must match")
    Lk = key.shape[-2]
    if value.shape[-2] != Lk:
        raise ValueError("scaled_dot_product_attention key and value sequence lengths must match")
    Lq, Ev = query.shape[-2], value.shape[-1]
    prefix = list(query.shape[:-2])
    if not enable_gqa:
        if list(key.shape[:-2]) != prefix or list(value.shape[:-2]) != prefix:
            raise ValueError("scaled_dot_product_attention leading dimensions must match")
        Hk_ratio = 1
    else:
        if rank < 3:
            raise ValueError("scaled_dot_product_attention enable_gqa requires a head dimension")
        if list(key.shape[:-3]) != prefix[:-1] or list(value.shape[:-3]) != prefix[:-1]:
            raise ValueError("scaled_dot_product_attention leading dimensions must match for enable_gqa")
        if key.shape[-3] != value.shape[-3]:
            raise ValueError("scaled_dot_product_attention key and value heads must match for enable_gqa")
        if key.shape[-3] <= 0 or query.shape[-3] % key.shape[-3] != 0:
            raise ValueError(
                "scaled_dot_product_attention query heads must be divisible by key/value heads for enable_gqa")
        Hk_ratio = query.shape[-3] // key.shape[-3]
    attn_shape = prefix + [Lq, Lk]
    if attn_mask is not None:
        try:
            okm = T._broadcast_shape(list(attn_mask.shape), attn_shape) == attn_shape and attn_mask.dim() <= len(attn_shape)
        except ValueError:
            okm = False
        if not okm:
            raise ValueError("scaled_dot_product_attention attn_mask is not broadcastable to attention weights")
    out = _empty(prefix + [Lq, Ev], query.dtype, dev)
    if out.numel() == 0:
        return out
    if dropout_p == 1.0:
        fill_(out, 0.0)
        return out
    if dropout_p != 0.0:
        raise ValueError("scaled_dot_product_attention dropout_p is only supported when it is 0 or 1")
    npre = len(prefix)
    H = prefix[-1] if npre else 1
    B = T._numel(prefix[:-1]) if npre else 1
    Hk = H // Hk_ratio

    def strides3(t):
        t2 = t if t.stride(-1) == 1 else t.contiguous()
        bh = _batch_head_strides(t2, npre)
        if bh is None:
            t2 = t2.contiguous()
            bh = _batch_head_strides(t2, npre)
        return t2, [bh[0], bh[1], t2.stride(-2)]

    q2, qs = strides3(query)
    k2, ks = strides3(key)
    v2, vs = strides3(value)
    mask_kind, mask_dt, mptr, ms = 0, 1, None, None
    m2 = None
    if attn_mask is not None:
        m2 = attn_mask
        if m2.dtype is not T.bool_ and m2.dtype is not query.dtype and m2.dtype is not T.float32:
            m2 = cast(m2, T.float32)
        full_rank = len(attn_shape)
        me = m2.expand(attn_shape)
        st = list(me.stride())
        # (b, h, q, k) strides; batch dims collapse to one stride
        if npre >= 2:
            bst = _collapse_batch(me, npre - 1)
            if bst is None:
                me = me.contiguous()
                st = list(me.stride())
                bst = _collapse_batch(me, npre - 1)
            hst = st[npre - 1]
        elif npre == 1:
            bst, hst = 0, st[0]
        else:
            bst, hst = 0, 0
        ms = [bst, hst, st[full_rank - 2], st[full_rank - 1]]
        m2 = me
        mask_kind = 1 if m2.dtype is T.bool_ else 2
        mask_dt = m2.dtype.code
        mptr = m2.data_ptr()
    _lib.check(_L().mthip_sdpa(dev, query.dtype.code, q2.data_ptr(), _lib.int64_array(qs), k2.data_ptr(),
                               _lib.int64_array(ks), v2.data_ptr(), _lib.int64_array(vs), out.data_ptr(), None, B, H,
                               Hk, Lq, Lk, E, Ev, mask_kind, mask_dt, mptr, _lib.int64_array(ms) if ms else None,
                               1 if is_causal else 0, 0 if scale is None else 1,
                               0.0 if scale is None else float(scale)))
    return out


# ------------------------------------------------------------------------------ normalisation


def _norm_param_dtype(op: str, x: Tensor, weight: Tensor, bias: Tensor) -> int:
    """dtype code of a norm's parameters: x's dtype, or float32 over a float16 input -- the
    upcast pattern norm(x.float(), w32, b32).half(), which the fused device paths run as one
    kernel.  (The public F.group_norm / F.layer_norm keep the reference's same-dtype rule.)"""
    dts = {t.dtype for t in (weight, bias) if t is not None}
    if not dts or dts == {x.dtype}:
        return x.dtype.code
    if dts == {T.float32} and x.dtype is T.float16:
        return T.float32.code
    raise RuntimeError(f"expected {op} tensors to have the same dtype")


def _group_norm_check(x: Tensor, num_groups: int, weight: Tensor, bias: Tensor):
    """Argument checks of mtorch::group_norm (tensor.cpp:18643-18700; binding module.cpp:7646-7693)."""
    if not x.dtype.is_floating_point:
        raise ValueError("group_norm expects a floating point input")
    if x.dim() < 2:
        raise ValueError("group_norm expected input rank of at least 2")
    if num_groups <= 0:
        raise ValueError("group_norm num_groups must be positive")
    C = x.shape[1]
    if C % num_groups != 0:
        raise ValueError("group_norm num_channels must be divisible by num_groups")
    inner = T._numel(x.shape[2:])
    if (C // num_groups) * inner <= 1:
        raise ValueError("group_norm expected more than 1 value per group")
    if weight is not None and list(weight.shape) != [C]:
        raise ValueError("group_norm weight must have shape [C]")
    if bias is not None and list(bias.shape) != [C]:
        raise ValueError("group_norm bias must have shape [C]")
    _float_dtype("group_norm", x.dtype)
    return inner


def group_norm(x: Tensor, num_groups: int, weight: Tensor = None, bias: Tensor = None, eps=1e-5,
               fuse_silu=False, allow_upcast=False) -> Tensor:
    """mtorch::group_norm (tensor.cpp:18643-18963), binding py_group_norm (module.cpp:7646-7693).
    allow_upcast: float32 parameters over a float16 input run group_norm(x.float(), w, b).half()."""
    if allow_upcast:
        pdt = _norm_param_dtype("group_norm", x, weight, bias)
    else:
        _same_dtype("group_norm", [x, weight, bias], "tensors")
        pdt = x.dtype.code
    dev = _gpu("group_norm", x, weight, bias)
    inner = _group_norm_check(x, num_groups, weight, bias)
    B, C = x.shape[0], x.shape[1]
    xc = x.contiguous()
    out = _empty(x.shape, x.dtype, dev)
    if out.numel():
        _lib.check(_L().mthip_group_norm(dev, x.dtype.code, xc.data_ptr(), _ptr(_contig(weight)), _ptr(_contig(bias)),
                                         out.data_ptr(), B, C, inner, num_groups, float(eps), 1 if fuse_silu else 0,
                                         pdt))
    return out


def layer_norm(x: Tensor, normalized_shape, weight: Tensor = None, bias: Tensor = None, eps=1e-5,
               allow_upcast=False) -> Tensor:
    """mtorch::layer_norm (tensor.cpp:17386-17708), binding py_layer_norm (module.cpp:7461-7516).
    allow_upcast: float32 parameters over a float16 input run layer_norm(x.float(), w, b).half()."""
    if isinstance(normalized_shape, int):
        normalized_shape = [normalized_shape]
    normalized_shape = [int(s) for s in normalized_shape]
    if allow_upcast:
        pdt = _norm_param_dtype("layer_norm", x, weight, bias)
    else:
        _same_dtype("layer_norm", [x, weight, bias], "tensors")
        pdt = x.dtype.code
    dev = _gpu("layer_norm", x, weight, bias)
    if not normalized_shape:
        raise ValueError("layer_norm normalized_shape must not be empty")
    if not x.dtype.is_floating_point:
        raise ValueError("layer_norm expects a floating point input")
    if len(normalized_shape) > x.dim():
        raise ValueError("layer_norm normalized_shape exceeds input rank")
    if list(x.shape[x.dim() - len(normalized_shape):]) != normalized_shape:
        raise ValueError("layer_norm normalized_shape must match the input tail dimensions")
    if weight is not None and list(weight.shape) != normalized_shape:
        raise ValueError("layer_norm weight shape must match normalized_shape")
    if bias is not None and list(bias.shape) != normalized_shape:
        raise ValueError("layer_norm bias shape must match normalized_shape")
    _float_dtype("layer_norm", x.dtype)
    N = T._numel(normalized_shape)
    rows = 0 if N == 0 else x.numel() // N
    xc = x.contiguous()
    out = _empty(x.shape, x.dtype, dev)
    if out.numel():
        _lib.check(_L().mthip_layer_norm(dev, x.dtype.code, xc.data_ptr(), _ptr(_contig(weight)),
                                         _ptr(_contig(bias)), out.data_ptr(), rows, N, float(eps), pdt))
    return out


def softmax(x: Tensor, dim=-1, dtype=None) -> Tensor:
    """mtorch::softmax (tensor.cpp:15145-15221)."""
    dev = _gpu("softmax", x)
    rank = x.dim()
    d = T._positive_dim(dim, rank)
    out_dt = T._as_dtype(dtype, x.dtype)
    if not x.dtype.is_floating_point or not out_dt.is_floating_point:
        raise RuntimeError("softmax(): input dtype must be floating point")
    _float_dtype("softmax", out_dt)
    # A dtype other than the input's takes the reference's generic path (tensor.cpp:15165-15207):
    # the input is read at its own precision and only the results are narrowed.  So a wider
    # output widens the input first (exact), a narrower one computes at the input's precision
    # and narrows the probabilities.
    narrowing = x.dtype is T.float32 and out_dt is T.float16
    src = x if (out_dt is x.dtype or narrowing) else cast(x, out_dt)
    if rank == 0:
        src = src.reshape(1)
        d = 0
    last = d == src.dim() - 1
    # fp32 rank<=2 kernels divide by the row total, the others multiply by its reciprocal
    # (tensor.cpp:7535-7537, 7581-7588, 7708-7710, 7789-7796); the generic path divides.
    divide = 1 if (out_dt is T.float32 and src.dim() <= 2) or not last or out_dt is not x.dtype else 0
    if not last:
        perm = [i for i in range(src.dim()) if i != d] + [d]
        moved = src.permute(perm).contiguous()
        res = softmax(moved, -1) if divide == 0 else _softmax_last(moved, dev, 1)
        inv = [0] * len(perm)
        for i, p in enumerate(perm):
            inv[p] = i
        out = res.permute(inv).contiguous()
    else:
        out = _softmax_last(src.contiguous(), dev, divide)
    if narrowing:
        out = cast(out, out_dt)
    return out.reshape(x.shape) if rank == 0 else out


def _softmax_last(src: Tensor, dev: int, divide: int) -> Tensor:
    out = _empty(src.shape, src.dtype, dev)
    cols = src.shape[-1] if src.dim() else 1
    rows = 0 if cols == 0 else src.numel() // cols
    if out.numel():
        _lib.check(_L().mthip_softmax_lastdim(dev, src.dtype.code, src.data_ptr(), out.data_ptr(), rows, cols, divide))
    return out


# ------------------------------------------------------------------------------ glue ops


def cat(tensors, dim=0) -> Tensor:
    """mtorch::cat (tensor.cpp:32141) along one dim of same-shaped device tensors."""
    tensors = list(tensors)
    if not tensors:
        raise ValueError("cat expects a non-empty list of tensors")
    dev = _gpu("cat", *tensors)
    dt = tensors[0].dtype
    if any(t.dtype is not dt for t in tensors):
        raise RuntimeError("expected cat tensors to have the same dtype")
    rank = tensors[0].dim()
    d = T._positive_dim(dim, rank)
    for t in tensors:
        if t.dim() != rank or any(t.shape[i] != tensors[0].shape[i] for i in range(rank) if i != d):
            raise ValueError("cat expects tensors with matching shapes outside the cat dimension")
    out_shape = list(tensors[0].shape)
    out_shape[d] = sum(t.shape[d] for t in tensors)
    out = _empty(out_shape, dt, dev)
    if out.numel():
        srcs = [t.contiguous() for t in tensors]
        ptrs = (ctypes.c_void_p * len(srcs))(*[s.data_ptr() for s in srcs])
        _lib.check(_L().mthip_cat(dev, dt.code, len(srcs), ptrs, _lib.int64_array([s.shape[d] for s in srcs]), rank,
                                  _lib.int64_array(out_shape), d, out.data_ptr()))
    return out


def interpolate(x: Tensor, size=None, scale_factor=None, mode="nearest", align_corners=None) -> Tensor:
    """interpolate(mode="nearest") (tensor.cpp:10897) for integer upsampling of NCHW input."""
    dev = _gpu("interpolate", x)
    if mode != "nearest":
        raise unsupported(f"interpolate(mode={mode!r})", "cuda")
    if x.dim() != 4:
        raise unsupported("interpolate on a non-4-D input", "cuda")
    B, C, H, W = x.shape
    if size is not None:
        oh, ow = (size, size) if isinstance(size, int) else tuple(size)
        if oh % H or ow % W:
            raise unsupported("interpolate with a non-integer scale", "cuda")
        sh, sw = oh // H, ow // W
    else:
        sf = (scale_factor, scale_factor) if not isinstance(scale_factor, (list, tuple)) else tuple(scale_factor)
        if any(float(s) != int(s) or int(s) < 1 for s in sf):
            raise unsupported("interpolate with a non-integer scale", "cuda")
        sh, sw = int(sf[0]), int(sf[1])
    _float_dtype("interpolate", x.dtype)
    xc = x.contiguous()
    out = _empty([B, C, H * sh, W * sw], x.dtype, dev)
    if out.numel():
        _lib.check(_L().mthip_upsample_nearest2d(dev, x.dtype.code, xc.data_ptr(), out.data_ptr(), B * C, H, W, sh, sw))
    return out


def arange(start, end=None, step=1, dtype=None, device=None) -> Tensor:
    """arange (tensor.h:150); values are computed on the host as start + i*step and moved."""
    if end is None:
        start, end = 0, start
    n = max(0, int(math.ceil((end - start) / step)))
    if dtype is None:
        dtype = T.int64 if all(isinstance(v, int) for v in (start, end, step)) else T.float32
    dt = T._as_dtype(dtype)
    vals = np.array([start + i * step for i in range(n)], dtype=np.float64)
    host = _random.host_cast(vals, T.float64, dt)
    t = Tensor(T.Storage(dt, n, T.device("cpu"), host=host), [n], [1])
    if device is not None and T.device(device).type != "cpu":
        t = t.to(device)
    return t
