"""Pins the oracle's restatement of mtorch's generator (module.cpp:47-183, 245-274, 335-365)
and checks the product generator (libmthip host code) against it bit for bit.

Pins: splitmix64's published test vectors; the 53-bit scaling of the uniform from the pinned
u64 stream; the polar pair's ordering/acceptance from the pinned uniforms; normality (KS);
the spare-normal bookkeeping across fp32 pair fills and fp16 per-element fills."""

import math

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
