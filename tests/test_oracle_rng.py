"""Pins the oracle's restatement of mtorch's generator (module.cpp:47-183, 245-274, 335-365)
and checks the product generator (libmthip host code) against it bit for bit.

Pins: splitmix64's published test vectors; the 53-bit scaling of the uniform from the pinned
u64 stream; the polar pair's ordering/acceptance from the pinned uniforms; normality (KS);
the spare-normal bookkeeping across fp32 pair fills and fp16 per-element fills; and, where the
reference tree is present, the reference's own generator compiled from module.cpp
(oracle/_ref/libref_rng.so, built by `make -C oracle ref`) bit for bit over streams, odd and
even fills and interleaved fp32/fp16 draws."""

import ctypes
import math
import os

import numpy as np
import pytest
from scipy import stats

import mtorch_amd as mt


def test_splitmix64_published_vectors(orc):
    r = orc.Rng(1234567)
    assert [r.next_u64() for _ in range(5)] == [
        6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431, 16408922859458223821]
    r = orc.Rng(0)
    assert r.next_u64() == 0xE220A8397B1DCDAF


def test_uniform_is_top_53_bits(orc):
    a, b = orc.Rng(99), orc.Rng(99)
    for _ in range(1000):
        u = a.uniform_open()
        assert 0.0 < u < 1.0
        assert u == (b.next_u64() >> 11) * 2.0**-53


def test_polar_pair_order_and_acceptance(orc):
    for seed in range(20):
        g, u = orc.Rng(seed), orc.Rng(seed)
        first, second = g.normal_pair()
        while True:
            x = 2.0 * u.uniform_open() - 1.0
            y = 2.0 * u.uniform_open() - 1.0
            r2 = x * x + y * y
            if 0.0 < r2 < 1.0:
                break
        # z = (x, y) * s for one positive s: the pair is the accepted (u, v) scaled, u first
        assert math.copysign(1.0, first) == math.copysign(1.0, x)
        assert math.copysign(1.0, second) == math.copysign(1.0, y)
        assert first / second == pytest.approx(x / y, rel=1e-12)
        assert (first * first + second * second) == pytest.approx(-2.0 * math.log(r2), rel=1e-12)
        assert g.next_u64() == u.next_u64()  # same number of uniforms consumed


def test_normals_are_standard_normal(orc):
    z = orc.Rng(5).randn((200000,)).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    assert stats.kstest(z, "norm").pvalue > 1e-3


def test_spare_normal_bookkeeping(orc):
    # an odd fp32 fill leaves the second of its last pair as the spare
    a, b = orc.Rng(3), orc.Rng(3)
    x = a.randn((5,))
    pairs = [b.normal_pair() for _ in range(3)]
    flat = [v for p in pairs for v in p]
    assert np.array_equal(x, np.float32(flat[:5]))
    assert a.next_normal() == flat[5]
    # fp16 fills draw one normal per element from the same stream
    c, d = orc.Rng(4), orc.Rng(4)
    h = c.randn((7,), "float16")
    z = d.randn((7,), "float32")
    assert np.array_equal(h, orc.f2h(z))


@pytest.mark.parametrize("seed", [0, 1, 42, 2**63 + 5])
def test_product_generator_matches_oracle(orc, seed):
    o = orc.Rng(seed)
    mt.manual_seed(seed)
    seq = [("n", (3, 5), "float32"), ("n", (7,), "float16"), ("u", (11,), "float32"), ("n", (1,), "float32"),
           ("u", (4, 4), "float16"), ("n", (6,), "float32")]
    for kind, shape, dt in seq:
        if kind == "n":
            exp = o.randn(shape, dt)
            got = mt.randn(*shape, dtype=dt)
        else:
            exp = o.uniform(shape, 0.0, 1.0, dt)
            got = mt.rand(*shape, dtype=dt)
        arr = got.half_bits() if dt == "float16" else got.numpy()
        assert np.array_equal(arr.view(np.uint16 if dt == "float16" else np.uint32),
                              exp.view(np.uint16 if dt == "float16" else np.uint32)), (kind, shape, dt)


def test_product_normal_and_uniform_inplace_match_oracle(orc):
    o = orc.Rng(77)
    mt.manual_seed(77)
    w = mt.empty(6, 5)
    w.normal_(0.0, 0.02)
    assert np.array_equal(w.numpy(), o.randn((6, 5), "float32", 0.0, 0.02))
    b = mt.empty(9, dtype=mt.float16)
    b.uniform_(-0.5, 0.25)
    assert np.array_equal(b.half_bits(), o.uniform((9,), -0.5, 0.25, "float16"))


def test_kaiming_uniform_consumes_uniforms_with_default_bound(orc):
    """kaiming_uniform_(a=sqrt 5) draws U(-1/sqrt(fan_in), 1/sqrt(fan_in)) (mtorch/__init__.py:5487-5499)."""
    o = orc.Rng(9)
    mt.manual_seed(9)
    w = mt.empty(8, 4, 3, 3)
    mt.nn.init.kaiming_uniform_(w, a=math.sqrt(5))
    bound = math.sqrt(3.0) * math.sqrt(2.0 / 6.0) / math.sqrt(36.0)
    assert np.array_equal(w.numpy(), o.uniform((8, 4, 3, 3), -bound, bound))


# ------------------------------------------------------------------ against the reference build

_REF = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref", "libref_rng.so")


@pytest.fixture(scope="module")
def ref():
    if not os.path.exists(_REF):
        pytest.skip("oracle/_ref/libref_rng.so not built (needs the reference tree: make -C oracle ref)")
    lib = ctypes.CDLL(_REF)
    u64, dbl, vp, i64 = ctypes.c_uint64, ctypes.c_double, ctypes.c_void_p, ctypes.c_int64
    lib.ref_rng_new.restype, lib.ref_rng_new.argtypes = vp, [u64]
    lib.ref_rng_free.restype, lib.ref_rng_free.argtypes = None, [vp]
    lib.ref_rng_next_u64.restype, lib.ref_rng_next_u64.argtypes = u64, [vp]
    lib.ref_rng_next_uniform.restype, lib.ref_rng_next_uniform.argtypes = dbl, [vp]
    lib.ref_rng_next_normal.restype, lib.ref_rng_next_normal.argtypes = dbl, [vp]
    for name in ("ref_rng_fill_normal_f32", "ref_rng_fill_uniform_f32"):
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = None, [vp, vp, i64, dbl, dbl]
    return lib


class _RefRng:
    def __init__(self, lib, seed):
        self.lib, self.p = lib, lib.ref_rng_new(seed)

    def __del__(self):
        self.lib.ref_rng_free(self.p)

    def randn_f32(self, n, mean=0.0, std=1.0):
        out = np.empty(n, np.float32)
        self.lib.ref_rng_fill_normal_f32(self.p, out.ctypes.data, n, mean, std)
        return out

    def uniform_f32(self, n, a, b):
        out = np.empty(n, np.float32)
        self.lib.ref_rng_fill_uniform_f32(self.p, out.ctypes.data, n, a, b)
        return out


SEEDS = [0, 1, 42, 1234567, 2**63 + 5, 2**64 - 1]


@pytest.mark.parametrize("seed", SEEDS)
def test_oracle_streams_equal_the_reference_build(orc, ref, seed):
    """u64, open-uniform and standard-normal streams (the last with the spare carried between
    draws) from the reference's module.cpp equal the oracle's, draw for draw."""
    r, o = _RefRng(ref, seed), orc.Rng(seed)
    assert [ref.ref_rng_next_u64(r.p) for _ in range(1000)] == [o.next_u64() for _ in range(1000)]
    got = [ref.ref_rng_next_uniform(r.p) for _ in range(1000)]
    assert got == [o.uniform_open() for _ in range(1000)]
    got = [ref.ref_rng_next_normal(r.p) for _ in range(1001)]
    assert got == [o.next_normal() for _ in range(1001)]


@pytest.mark.parametrize("seed", SEEDS)
def test_oracle_fills_equal_the_reference_build(orc, ref, seed):
    """A sequence of contiguous fp32 normal fills of odd and even lengths (a fill that ends on
    the first of a pair leaves the second as the spare, and the next fill starts with it),
    uniform fills, single draws and fp16 per-element draws in between: the oracle equals the
    reference build bit for bit, array by array."""
    r, o = _RefRng(ref, seed), orc.Rng(seed)
    for kind, n, a, b in [("n", 5, 0.0, 1.0), ("n", 7, 0.5, 2.0), ("n", 1, 0.0, 1.0), ("n", 0, 0.0, 1.0),
                          ("u", 11, -1.0, 1.0), ("n", 10, -3.0, 0.25), ("h", 7, 0.0, 1.0), ("n", 3, 0.0, 1.0),
                          ("hu", 9, -0.5, 0.5), ("s", 1, 0.0, 1.0), ("n", 4096, 0.0, 1.0), ("u", 1000, 2.0, 5.0)]:
        if kind == "n":
            assert np.array_equal(o.randn((n,), "float32", a, b), r.randn_f32(n, a, b)), (kind, n)
        elif kind == "u":
            assert np.array_equal(o.uniform((n,), a, b, "float32"), r.uniform_f32(n, a, b)), (kind, n)
        elif kind == "h":
            # fp16 normal_: one standard normal per element, mean + std * z narrowed through float
            z = np.array([ref.ref_rng_next_normal(r.p) for _ in range(n)])
            assert np.array_equal(o.randn((n,), "float16", a, b), orc.f2h(np.float32(a + b * z))), (kind, n)
        elif kind == "hu":
            u = np.array([ref.ref_rng_next_uniform(r.p) for _ in range(n)])
            assert np.array_equal(o.uniform((n,), a, b, "float16"), orc.f2h(np.float32(a + (b - a) * u))), (kind, n)
        else:
            assert o.next_normal() == ref.ref_rng_next_normal(r.p)
