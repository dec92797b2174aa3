"""The no-allocation group_norm entry point (mthip_group_norm_noalloc) against mthip_group_norm:
identical bits on calls in a row, each smaller than the one before (the scratch keeps the
previous call's partials), with no growth of the caching allocator; the one-pass kernel serves
batches whose partials would not fit the scratch; two-kernel sizes past the scratch are refused
with an error status."""

import numpy as np
import pytest

import mtorch_amd as mt
import oracle as orc
from mtorch_amd import _lib

pytestmark = pytest.mark.gpu


def _call(fn, x, w, b, groups, silu, param_dt):
    y = mt.empty(*x.shape, dtype=x.dtype, device="cuda")
    B, C = x.shape[0], x.shape[1]
    inner = x.numel() // (B * C)
    rc = fn(0, x.dtype.code, x.data_ptr(), w.data_ptr(), b.data_ptr(), y.data_ptr(), B, C, inner, groups, 1e-5,
            silu, param_dt.code)
    _lib.check(rc)
    return y


def _bits(t):
    return t.cpu().half_bits() if t.dtype is mt.float16 else t.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("dt,pdt", [("float16", "float16"), ("float32", "float32"), ("float16", "float32")])
def test_noalloc_group_norm_equals_group_norm(dt, pdt):
    L = _lib.lib()
    r = orc.Rng(123)
    # the one-pass kernel (512 (sample, group) pairs, no partials), then the two-kernel path on
    # the scratch, then a smaller two-kernel call
    cases = [((16, 320, 64, 64), 32, 1), ((2, 320, 64, 64), 32, 1), ((1, 64, 9, 7), 8, 0)]
    for shape, groups, silu in cases:
        dtype, ptype = getattr(mt, dt), getattr(mt, pdt)
        x = mt.from_numpy(r.randn(shape, dt), dtype=dtype).to("cuda")
        w = mt.from_numpy(r.randn((shape[1],), pdt), dtype=ptype).to("cuda")
        b = mt.from_numpy(r.randn((shape[1],), pdt), dtype=ptype).to("cuda")
        ref = _call(L.mthip_group_norm, x, w, b, groups, silu, ptype)
        y = mt.empty(*shape, dtype=dtype, device="cuda")
        mt.cuda.synchronize()
        before = (mt.cuda.memory_allocated(), mt.cuda.memory_reserved())
        B, C = shape[0], shape[1]
        inner = int(np.prod(shape[2:]))
        _lib.check(L.mthip_group_norm_noalloc(0, dtype.code, x.data_ptr(), w.data_ptr(), b.data_ptr(), y.data_ptr(), B,
                                              C, inner, groups, 1e-5, silu, ptype.code))
        mt.cuda.synchronize()
        # nothing taken from the caching allocator, nothing obtained from the driver
        assert (mt.cuda.memory_allocated(), mt.cuda.memory_reserved()) == before
        assert np.array_equal(_bits(y), _bits(ref)), (shape, dt, pdt)


def test_noalloc_group_norm_one_pass_beyond_the_scratch():
    """8192 (sample, group) pairs of 20 stats chunks would need 163840 partials, more than the
    scratch holds; the one-pass kernel needs none, so the call succeeds, bit for bit
    mthip_group_norm, without allocating."""
    L = _lib.lib()
    r = orc.Rng(321)
    part = mt.from_numpy(r.randn((16, 320, 64, 64), "float16"), dtype=mt.float16).to("cuda")
    x = mt.cat([part] * 16, dim=0)
    w = mt.from_numpy(r.randn((320,), "float16"), dtype=mt.float16).to("cuda")
    b = mt.from_numpy(r.randn((320,), "float16"), dtype=mt.float16).to("cuda")
    ref = _call(L.mthip_group_norm, x, w, b, 32, 1, mt.float16)
    y = mt.empty(*x.shape, dtype=mt.float16, device="cuda")
    mt.cuda.synchronize()
    before = (mt.cuda.memory_allocated(), mt.cuda.memory_reserved())
    _lib.check(L.mthip_group_norm_noalloc(0, _lib.F16, x.data_ptr(), w.data_ptr(), b.data_ptr(), y.data_ptr(), 256,
                                          320, 4096, 32, 1e-5, 1, _lib.F16))
    mt.cuda.synchronize()
    assert (mt.cuda.memory_allocated(), mt.cuda.memory_reserved()) == before
    assert np.array_equal(_bits(y), _bits(ref))


def test_noalloc_group_norm_refuses_more_partials_than_the_scratch():
    L = _lib.lib()
    # 4096 groups x 64 chunks of 2048 elements = 262144 partials > 131072
    B, C, inner, groups = 128, 32, 131072, 32
    x = mt.zeros(B, C, inner, dtype=mt.float16, device="cuda")
    y = mt.empty(B, C, inner, dtype=mt.float16, device="cuda")
    rc = L.mthip_group_norm_noalloc(0, _lib.F16, x.data_ptr(), None, None, y.data_ptr(), B, C, inner, groups, 1e-5, 0,
                                    _lib.F16)
    assert rc != 0
    assert b"scratch" in L.mthip_last_error()
