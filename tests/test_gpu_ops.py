"""GPU parity: every hot-path operator through libmthip's C ABI against the CPU oracle on the
same seeded inputs.

Tolerances: max |gpu - ref| / max |ref| <= 1e-4 for fp32 kernels and
<= 1e-2 for fp16 kernels (fp32 accumulate); bit-exact for dtype casts, copies and metadata."""

import os
import sys

import numpy as np
import pytest

import mtorch_amd as mt
import oracle as orc

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(__file__)
sys.path.insert(0, os.path.join(HERE, "golden"))
import closed_form  # noqa: E402

F = mt.nn.functional
TOL = {"float32": 1e-4, "float16": 1e-2}


def rel(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    if got.size == 0:
        return 0.0
    assert np.array_equal(np.isnan(got), np.isnan(ref)), "NaN pattern differs"
    m = ~np.isnan(ref)
    return float(np.max(np.abs(got[m] - ref[m])) / max(np.max(np.abs(ref[m])), 1e-30)) if m.any() else 0.0


class Gen:
    """Seeded inputs from mtorch's generator (via the oracle) in a given dtype."""

    def __init__(self, seed):
        self.r = orc.Rng(seed)

    def randn(self, shape, dt, std=1.0):
        return self.r.randn(shape, dt, 0.0, std)


def dev(a):
    return mt.from_numpy(a, dtype=mt.float16 if a.dtype == np.uint16 else None).to("cuda")


def host(t):
    return t.cpu().half_bits() if t.dtype is mt.float16 else t.cpu().numpy()


def val(a):
    return orc.h2f(a) if a.dtype == np.uint16 else a


@pytest.fixture(autouse=True)
def _no_grad():
    with mt.no_grad():
        yield


def test_device_visible():
    assert mt.cuda.is_available()
    name = mt.cuda.get_device_name(0)
    assert "gfx950" in name, name


# ------------------------------------------------------------------ data movement


def test_cast_bit_exact():
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    t = mt.from_numpy(x).to("cuda")
    got = t.to(mt.float16).cpu().half_bits()
    assert np.array_equal(got, orc.f2h(x))
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    back = mt.from_numpy(allh, dtype=mt.float16).to("cuda").to(mt.float32).cpu().numpy()
    assert np.array_equal(back.view(np.uint32), orc.h2f(allh).view(np.uint32))
    # odd sizes / offsets take the scalar path
    sub = t[3:1000]
    assert np.array_equal(sub.half().cpu().half_bits(), orc.f2h(x[3:1000]))


def test_strided_copies_bit_exact():
    rng = np.random.default_rng(4)
    a = rng.standard_normal((3, 37, 5, 41)).astype(np.float32)
    t = mt.from_numpy(a).to("cuda")
    for perm in [(0, 2, 1, 3), (0, 1, 3, 2), (3, 2, 1, 0), (1, 0, 2, 3)]:
        got = t.permute(*perm).contiguous().cpu().numpy()
        assert np.array_equal(got, np.ascontiguousarray(a.transpose(perm)))
    h = orc.f2h(a)
    th = dev(h)
    got = th.transpose(1, 2).contiguous().cpu().half_bits()
    assert np.array_equal(got, np.ascontiguousarray(h.transpose(0, 2, 1, 3)))
    assert np.array_equal(th[:, 5:20:3, :, ::2].contiguous().cpu().half_bits(), h[:, 5:20:3, :, ::2])


def test_view_metadata_matches_reference_rules():
    t = mt.zeros(2, 3, 4, device="cuda")
    assert t.transpose(0, 2).stride() == (1, 4, 12)
    r = t.transpose(1, 2).reshape(2, 12)  # not viewable -> copy, contiguous strides
    assert r.stride() == (12, 1) and r.is_contiguous()
    v = t.permute(0, 2, 1).unsqueeze(1)
    assert v.shape == (2, 1, 4, 3) and v.stride() == (12, 4, 1, 4)
    a, b = t.chunk(2, dim=-1)
    assert a.shape == (2, 3, 2) and b.storage_offset() == 2 and b.stride() == (12, 4, 1)


# ------------------------------------------------------------------ elementwise


@pytest.mark.parametrize("dt", ["float32", "float16"])
def test_binary_ops(dt):
    g = Gen(11)
    a = g.randn((4, 6, 9, 10), dt)
    b = g.randn((4, 6, 9, 10), dt)
    for op in ("add", "mul", "sub"):
        got = host({"add": dev(a) + dev(b), "mul": dev(a) * dev(b), "sub": dev(a) - dev(b)}[op])
        assert np.array_equal(got, orc.binary(a, b, op)), op  # same-shape ops are exact
    # broadcasts: channel bias [1,6,1,1], time embedding [4,6,1,1], row [10]
    for shape in [(1, 6, 1, 1), (4, 6, 1, 1), (10,), (9, 1)]:
        c = g.randn(shape, dt)
        got = host(dev(a) + dev(c))
        ref = orc.binary(a, np.broadcast_to(c, a.shape), "add")
        assert np.array_equal(got, ref), shape


@pytest.mark.parametrize("dt", ["float32", "float16"])
def test_activations(dt):
    g = Gen(12)
    x = g.randn((3, 1001), dt, 3.0)
    for name, fn, ref in [("silu", F.silu, orc.silu(x)), ("gelu", F.gelu, orc.gelu(x)),
                          ("gelu_tanh", lambda t: F.gelu(t, approximate="tanh"), orc.gelu(x, "tanh"))]:
        got = host(fn(dev(x)))
        assert rel(val(got), val(ref)) <= (2e-6 if dt == "float32" else 1e-3), name


def test_silu_fp16_every_half_is_bit_exact():
    """The fp16 SiLU (native 2^x and reciprocal with pinned exceptions) against the reference's
    f2h(x / (1 + expf(-x))) on all 65536 half inputs, NaNs and infinities included."""
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = host(F.silu(dev(allh)))
    ref = orc.silu(allh)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, [(hex(i), hex(got[i]), hex(ref[i])) for i in bad[:8]]


def test_silu_gelu_fp16_lds_table_path_is_bit_exact():
    """Buffers of >= 2^21 halves take the kernel that looks SiLU / erf-GELU up in an LDS copy of
    the 64 K-entry table: every half input, repeated past that size with a ragged 16-byte tail,
    gives the same bits as the scalar kernel on the same halves and, for SiLU, as the oracle."""
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    big = np.tile(allh, 40)[: 40 * 65536 - 3]  # 2,621,437 halves: table kernel + scalar tail
    t = dev(big)
    for name, fn in [("silu", F.silu), ("gelu", F.gelu)]:
        got = host(fn(t))
        ref = host(fn(dev(allh)[1:]))  # one element in: the unaligned scalar kernel
        ref = np.concatenate([host(fn(dev(allh[:1]))), ref])
        exp = np.tile(ref, 40)[: big.size]
        bad = np.nonzero(got != exp)[0]
        assert bad.size == 0, (name, [(int(big[i]), hex(got[i]), hex(exp[i])) for i in bad[:8]])
    got = host(F.silu(t))
    assert np.array_equal(got, np.tile(orc.silu(allh), 40)[: big.size])


@pytest.mark.parametrize("dt", ["float32", "float16"])
def test_unary_vector_path_equals_scalar_path(dt):
    """Aligned inputs go through the 16-byte-per-lane kernel (fp16 silu and erf-gelu as table
    lookups) with a scalar tail; a view one element in is misaligned and takes the scalar
    kernel.  Both give the same bits, on every half input for fp16."""
    if dt == "float16":
        x = (np.arange(65536 + 9, dtype=np.uint32) % 65536).astype(np.uint16)
    else:
        x = Gen(15).randn((65536 + 9,), dt, 4.0)
    t = dev(x)
    for name, fn in [("silu", F.silu), ("gelu", F.gelu), ("gelu_tanh", lambda u: F.gelu(u, approximate="tanh"))]:
        full = host(fn(t))
        off = host(fn(t[1:]))
        bad = np.nonzero(full[1:].view(np.uint32 if dt == "float32" else np.uint16)
                         != off.view(np.uint32 if dt == "float32" else np.uint16))[0]
        assert bad.size == 0, (name, bad[:8])


@pytest.mark.parametrize("dt", ["float32", "float16"])
@pytest.mark.parametrize("M,N,K,bias", [(77, 64, 40, True), (300, 320, 96, True), (128, 128, 64, False), (8192, 2560, 320, True)])
def test_linear_geglu_fused(dt, M, N, K, bias):
    """The GEGLU epilogue (value/gate pairing over interleaved weight rows, gelu table lookup)
    equals linear -> geglu bit for bit, and the oracle's linear -> chunk -> gelu -> mul within
    tolerance."""
    g = Gen(M + N + K)
    x = g.randn((M, K), dt)
    w = g.randn((2 * N, K), dt, 1.0 / np.sqrt(K))
    b = g.randn((2 * N,), dt) if bias else None
    xd, wd, bd = dev(x), dev(w), (dev(b) if bias else None)
    fused = host(F.linear_geglu(xd, wd, bd))
    unfused = host(F.geglu(F.linear(xd, wd, bd)))
    assert np.array_equal(fused, unfused)
    if M * N <= 300 * 320:
        lin = orc.linear(x, w, b)
        ref = orc.binary(np.ascontiguousarray(lin[:, :N]), orc.gelu(np.ascontiguousarray(lin[:, N:])), "mul")
        assert rel(val(fused), val(ref)) <= TOL[dt]


def test_norm_upcast_pattern():
    """fp32 norm parameters over fp16 data: norm(x.float(), w32, b32).half() in one kernel."""
    from mtorch_amd import _ops

    g = Gen(81)
    x = g.randn((2, 64, 8, 8), "float16")
    w = g.randn((64,), "float32")
    b = g.randn((64,), "float32")
    got = host(_ops.group_norm(dev(x), 8, dev(w), dev(b), 1e-5, allow_upcast=True))
    ref = orc.f2h(orc.group_norm(orc.h2f(x), 8, w, b, 1e-5))
    assert got.dtype == np.uint16 and rel(val(got), val(ref)) <= 2e-3
    got = host(_ops.group_norm(dev(x), 8, dev(w), dev(b), 1e-5, fuse_silu=True, allow_upcast=True))
    assert rel(val(got), val(orc.silu(ref))) <= 2e-3
    t = g.randn((3, 77, 320), "float16")
    lw = g.randn((320,), "float32")
    lb = g.randn((320,), "float32")
    got = host(_ops.layer_norm(dev(t), [320], dev(lw), dev(lb), 1e-5, allow_upcast=True))
    ref = orc.f2h(orc.layer_norm(orc.h2f(t), 320, lw, lb, 1e-5))
    assert rel(val(got), val(ref)) <= 2e-3
    # the SpatialTransformer shapes (8192 tokens x 320, 2048 x 640, 512 x 1280): rows of five
    # 16-byte chunks per lane over 8/16/32 lanes
    for rows, n in [(8192, 320), (2048, 640), (2050, 1280)]:
        t2 = g.randn((rows, n), "float16", 2.0)
        w2 = g.randn((n,), "float32")
        b2 = g.randn((n,), "float32")
        got = host(_ops.layer_norm(dev(t2), [n], dev(w2), dev(b2), 1e-5, allow_upcast=True))
        ref = orc.f2h(orc.layer_norm(orc.h2f(t2), n, w2, b2, 1e-5))
        assert rel(val(got), val(ref)) <= 2e-3, (rows, n)
    with pytest.raises(RuntimeError, match="same dtype"):
        F.layer_norm(dev(t), [320], dev(lw), dev(lb))  # the public op keeps the same-dtype rule


def test_geglu_matches_chunk_gelu_mul():
    g = Gen(13)
    x = g.randn((2, 17, 64), "float16", 2.0)
    got = host(F.geglu(dev(x)))
    a, gate = x[..., :32], x[..., 32:]
    ref = orc.binary(np.ascontiguousarray(a), orc.gelu(np.ascontiguousarray(gate)), "mul")
    assert rel(val(got), val(ref)) <= 1e-3


def _finite_halves():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    return h[(h & 0x7C00) != 0x7C00]


def test_fp16_mul_keeps_the_sign_of_zero_products():
    """fp16 products narrowed on the device keep mtorch's signed zeros (a -0 product stays 0x8000,
    tiny products flush to a zero of their sign), bit for bit against the oracle for every finite
    half times a set of multipliers, the zeros included."""
    a = _finite_halves()
    for bm in [0x3C00, 0xBC00, 0x0000, 0x8000, 0x0001, 0x8001, 0x7BFF, 0x3555]:
        b = np.full(a.shape, bm, np.uint16)
        got = host(dev(a) * dev(b))
        ref = orc.binary(a, b, "mul")
        bad = np.nonzero(got != ref)[0]
        assert bad.size == 0, (hex(bm), [(hex(a[i]), hex(got[i]), hex(ref[i])) for i in bad[:6]])


def test_geglu_bit_exact_over_every_gate():
    """geglu(value, gate) = value * gelu(gate) in fp16 equals the oracle's chunk -> gelu -> mul
    bit for bit for every finite gate half (large negative gates give -0 gelus, whose products
    keep the sign), with positive and negative values."""
    gate = _finite_halves()
    for vm in [0x3C00, 0xBC00, 0x2CAA, 0x0000]:
        value = np.full(gate.shape, vm, np.uint16)
        x = np.concatenate([value, gate]).reshape(1, 2 * gate.size)
        got = host(F.geglu(dev(x))).reshape(-1)
        ref = orc.binary(value, orc.gelu(gate), "mul")
        bad = np.nonzero(got != ref)[0]
        assert bad.size == 0, (hex(vm), [(hex(gate[i]), hex(got[i]), hex(ref[i])) for i in bad[:6]])


def test_scalar_ops_and_unary_math():
    g = Gen(14)
    x = g.randn((1000,), "float32")
    t = dev(x)
    assert rel(host(t * 0.125), x.astype(np.float64) * 0.125) <= 1e-7
    assert rel(host(2.0 - t), 2.0 - x.astype(np.float64)) <= 1e-7
    assert rel(host(t.exp()), np.exp(x.astype(np.float64))) <= 1e-6
    assert rel(host(t.sin()), np.sin(x.astype(np.float64))) <= 1e-6


# ------------------------------------------------------------------ contractions


@pytest.mark.parametrize("dt", ["float32", "float16"])
@pytest.mark.parametrize("M,N,K", [(37, 23, 19), (128, 320, 320), (200, 130, 72), (2, 1280, 320), (64, 77, 768)])
def test_linear(dt, M, N, K):
    g = Gen(M * 7 + N)
    x = g.randn((M, K), dt)
    w = g.randn((N, K), dt, 1.0 / np.sqrt(K))
    b = g.randn((N,), dt)
    got = host(F.linear(dev(x), dev(w), dev(b)))
    assert rel(val(got), val(orc.linear(x, w, b))) <= TOL[dt]


@pytest.mark.parametrize("M,N,K,res", [(8192, 960, 320, False), (8192, 320, 320, True), (2048, 640, 2560, True),
                                        (512, 3840, 1280, False), (512, 1280, 1280, True), (77, 96, 640, True),
                                        (1000, 48, 320, False)])
@pytest.mark.parametrize("bt", ["64", "128"])
def test_linear_streamed_kernel(M, N, K, res, bt, monkeypatch):
    """fp16 linears with K a multiple of 320 can take the streamed kernel (persistent workgroups
    over 80-channel x 64- or 128-token units -- four or eight compute waves, one or two producer
    waves -- K split and reduction where the model picks it); MTHIP_GEMM_STREAM=2 sends every
    such shape there.  Checked against the oracle on a
    strided subset of rows that includes the last, with bias and with the residual, including
    partial channel and token tiles; 64- and 128-token units (MTHIP_GEMM_STREAM_BT)."""
    monkeypatch.setenv("MTHIP_GEMM_STREAM", "2")
    monkeypatch.setenv("MTHIP_GEMM_STREAM_BT", bt)
    g = Gen(M + N + K)
    x = g.randn((M, K), "float16")
    w = g.randn((N, K), "float16", 1.0 / np.sqrt(K))
    b = g.randn((N,), "float16")
    r = g.randn((M, N), "float16") if res else None
    if res:
        got = host(F.linear_residual(dev(x), dev(w), dev(b), dev(r)))
    else:
        got = host(F.linear(dev(x), dev(w), dev(b)))
    rows = np.unique(np.r_[np.arange(0, M, max(1, M // 60)), M - 1])
    ref = orc.linear(np.ascontiguousarray(x[rows]), w, b)
    if res:
        ref = orc.binary(ref, np.ascontiguousarray(r[rows]), "add")
    assert rel(val(got[rows]), val(ref)) <= TOL["float16"]


@pytest.mark.parametrize("M,N,K", [(8192, 1280, 320), (512, 1280, 1280), (2048, 640, 2560), (77, 96, 640)])
@pytest.mark.parametrize("bt", ["64", "128"])
def test_linear_gelu_streamed_kernel(M, N, K, bt, monkeypatch):
    """fp16 linear+GELU on the streamed kernel (the gelu of each narrowed value looked up in the
    fp16 table in its epilogue, or in the K-split reduction's): bit for bit gelu(linear(...)) of
    the same kernel -- every value through the table, so every gate input is covered where the
    outputs span them -- and the oracle's values on a strided subset of rows; 64- and 128-token
    units, the planner's K splits, partial channel and token tiles."""
    monkeypatch.setenv("MTHIP_GEMM_STREAM", "2")
    monkeypatch.setenv("MTHIP_GEMM_STREAM_BT", bt)
    g = Gen(M * 3 + N + K)
    x = g.randn((M, K), "float16")
    w = g.randn((N, K), "float16", 2.0 / np.sqrt(K))
    b = g.randn((N,), "float16")
    fused = host(F.linear_gelu(dev(x), dev(w), dev(b)))
    unfused = host(F.gelu(F.linear(dev(x), dev(w), dev(b))))
    assert np.array_equal(fused, unfused)
    rows = np.unique(np.r_[np.arange(0, M, max(1, M // 40)), M - 1])
    ref = orc.gelu(orc.linear(np.ascontiguousarray(x[rows]), w, b))
    assert rel(val(fused[rows]), val(ref)) <= TOL["float16"]


@pytest.mark.parametrize("M,N,res", [(8192, 320, True), (8192, 960, False), (1000, 240, True), (77, 96, False)])
def test_linear_streamed_token_tiles_agree_bit_for_bit(M, N, res, monkeypatch):
    """With one K slice (K = 320) every output's fp32 sum runs over the same k order whether its
    unit holds 64 tokens (four compute waves, one producer) or 128 (eight compute waves, two
    producers), so the two give the same bits; a stage refilled while a compute wave still
    reads it, or a token row read from the wrong wave's fragment, would show here."""
    monkeypatch.setenv("MTHIP_GEMM_STREAM", "2")
    g = Gen(M + 3 * N)
    K = 320
    x, w, b = dev(g.randn((M, K), "float16")), dev(g.randn((N, K), "float16", 1.0 / np.sqrt(K))), dev(g.randn((N,), "float16"))
    r = dev(g.randn((M, N), "float16")) if res else None
    outs = []
    for bt in ("64", "128"):
        monkeypatch.setenv("MTHIP_GEMM_STREAM_BT", bt)
        outs.append(host(F.linear_residual(x, w, b, r) if res else F.linear(x, w, b)))
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("dt", ["float32", "float16"])
def test_linear_strided_vector_input(dt):
    """A 1-D input with a non-unit stride (x[::2]) is one row read after a dense copy."""
    g = Gen(5)
    x = g.randn((2 * 96,), dt)
    w = g.randn((40, 96), dt, 0.1)
    b = g.randn((40,), dt)
    got = host(F.linear(dev(x)[::2], dev(w), dev(b)))
    ref = orc.linear(np.ascontiguousarray(x[::2]).reshape(1, 96), w, b).reshape(40)
    assert rel(val(got), val(ref)) <= TOL[dt]


@pytest.mark.parametrize("dt", ["float32", "float16"])
def test_linear_fused_epilogues(dt):
    g = Gen(21)
    x = g.randn((3, 50, 96), dt)
    w = g.randn((128, 96), dt, 0.1)
    b = g.randn((128,), dt)
    r = g.randn((3, 50, 128), dt)
    lin = orc.linear(x, w, b)
    got = host(F.linear_gelu(dev(x), dev(w), dev(b)))
    assert rel(val(got), val(orc.gelu(lin))) <= TOL[dt]
    got = host(F.linear_silu(dev(x), dev(w), dev(b)))
    assert rel(val(got), val(orc.silu(lin))) <= TOL[dt]
    got = host(F.linear_residual(dev(x), dev(w), dev(b), dev(r)))
    assert rel(val(got), val(orc.binary(lin, r, "add"))) <= TOL[dt]


def test_linear_strided_input_and_transposed_weight():
    g = Gen(22)
    x = g.randn((40, 2, 64), "float32")
    w = g.randn((64, 48), "float32", 0.1)  # used as w.t()
    xt = dev(x).transpose(0, 1)  # [2, 40, 64] non-contiguous
    got = host(F.linear(xt, dev(w).t()))
    ref = orc.linear(np.ascontiguousarray(x.transpose(1, 0, 2)), np.ascontiguousarray(w.T))
    assert rel(got, ref) <= 1e-4


@pytest.mark.parametrize("dt", ["float32", "float16"])
def test_matmul_batched_broadcast_and_transposes(dt):
    g = Gen(31)
    a = g.randn((2, 3, 33, 20), dt)
    b = g.randn((3, 20, 45), dt)
    got = host(mt.matmul(dev(a), dev(b)))
    ref = orc.matmul(a.reshape(6, 33, 20), np.broadcast_to(b[None], (2, 3, 20, 45)).reshape(6, 20, 45))
    assert rel(val(got), val(ref.reshape(2, 3, 33, 45))) <= TOL[dt]
    # attention-style: q @ k^T with k^T a transposed view
    k = g.randn((3, 45, 20), dt)
    got = host(mt.matmul(dev(a[0]), dev(k).transpose(-2, -1)))
    ref = orc.matmul(a[0], np.ascontiguousarray(k.transpose(0, 2, 1)))
    assert rel(val(got), val(ref)) <= TOL[dt]
    v = g.randn((20,), dt)
    got = host(mt.matmul(dev(a[0, 0]), dev(v)))
    assert rel(val(got), val(orc.matmul(a[0, 0], v.reshape(20, 1)).reshape(33))) <= TOL[dt]


@pytest.mark.parametrize("dt", ["float32", "float16"])
@pytest.mark.parametrize("K", [77, 1, 9, 13])
def test_matmul_unaligned_depth_every_row(dt, K):
    """K not a whole number of 16-byte chunks: A is staged through a zero-padded copy and its
    last row's final chunk must still be read (probabilities @ values over 77 text tokens)."""
    g = Gen(33 + K)
    a = g.randn((3, 64, K), dt)
    b = g.randn((3, K, 40), dt)
    got = val(host(mt.bmm(dev(a), dev(b))))
    ref = val(orc.matmul(a, b))
    for r in (0, 62, 63):
        assert rel(got[:, r], ref[:, r]) <= TOL[dt], r
    assert rel(got, ref) <= TOL[dt]


@pytest.mark.parametrize("dt", ["float32", "float16"])
def test_addmm_and_baddbmm(dt):
    g = Gen(32)
    inp = g.randn((40,), dt)
    m1 = g.randn((25, 30), dt)
    m2 = g.randn((30, 40), dt)
    got = host(mt.addmm(dev(inp), dev(m1), dev(m2), beta=0.5, alpha=2.0))
    assert rel(val(got), val(orc.addmm(inp, m1, m2, 0.5, 2.0))) <= TOL[dt]
    bi = g.randn((4, 25, 40), dt)
    b1 = g.randn((4, 25, 30), dt)
    b2 = g.randn((4, 30, 40), dt)
    got = host(mt.baddbmm(dev(bi), dev(b1), dev(b2), beta=1.0, alpha=0.25))
    ref = np.stack([orc.addmm(bi[i], b1[i], b2[i], 1.0, 0.25) for i in range(4)])
    assert rel(val(got), val(ref)) <= TOL[dt]


@pytest.mark.parametrize("dt", ["float32", "float16"])
def test_addmm_and_baddbmm_non_finite_beta0_alpha0(dt):
    """The Linux path's semantics at beta = 0 and alpha = 0 (tensor.cpp:25253-25258, 25320,
    1452, 25621): beta*input is stored even at beta = 0, so an inf/NaN input element gives NaN;
    alpha = 0 skips the product, so NaN/inf operands leave exactly beta*input (bit for bit)."""
    g = Gen(34)
    inp = g.randn((25, 40), dt)
    bits = 0x7C00 if dt == "float16" else np.float32(np.inf)
    nanb = 0x7E00 if dt == "float16" else np.float32(np.nan)
    inp[3, 5], inp[7, 0] = bits, nanb
    m1 = g.randn((25, 30), dt)
    m2 = g.randn((30, 40), dt)
    got = host(mt.addmm(dev(inp), dev(m1), dev(m2), beta=0.0, alpha=1.5))
    ref = orc.addmm(inp, m1, m2, 0.0, 1.5)
    assert rel(val(got), val(ref)) <= TOL[dt]
    assert np.isnan(val(got)[3, 5]) and np.isnan(val(got)[7, 0])
    m1n = m1.copy()
    m1n[0, 0], m1n[10, 29] = nanb, bits
    got = host(mt.addmm(dev(inp), dev(m1n), dev(m2), beta=0.75, alpha=0.0))
    assert np.array_equal(val(got), val(orc.addmm(inp, m1n, m2, 0.75, 0.0)), equal_nan=True)
    bi = np.stack([inp] * 3)
    b1 = np.stack([m1n] * 3)
    b2 = np.stack([m2] * 3)
    got = host(mt.baddbmm(dev(bi), dev(b1), dev(b2), beta=0.75, alpha=0.0))
    want = orc.addmm(inp, m1n, m2, 0.75, 0.0)
    for i in range(3):
        assert np.array_equal(val(got[i]), val(want), equal_nan=True)
    got = host(mt.baddbmm(dev(bi), dev(np.stack([m1] * 3)), dev(b2), beta=0.0, alpha=1.0))
    assert np.isnan(val(got)[:, 3, 5]).all() and np.isnan(val(got)[:, 7, 0]).all()
    assert rel(val(got[1]), val(orc.addmm(inp, m1, m2, 0.0, 1.0))) <= TOL[dt]


CONV_CASES = [
    dict(B=2, C=32, H=16, W=16, O=48, k=3, stride=1, padding=1, dilation=1, groups=1),
    dict(B=1, C=40, H=15, W=13, O=24, k=3, stride=2, padding=1, dilation=1, groups=1),
    dict(B=2, C=4, H=12, W=12, O=32, k=3, stride=1, padding=1, dilation=1, groups=1),
    dict(B=2, C=32, H=9, W=11, O=4, k=3, stride=1, padding=1, dilation=1, groups=1),
    dict(B=1, C=64, H=8, W=8, O=64, k=1, stride=1, padding=0, dilation=1, groups=1),
    dict(B=1, C=12, H=10, W=10, O=8, k=3, stride=1, padding=2, dilation=2, groups=1),
    dict(B=1, C=8, H=7, W=9, O=6, k=3, stride=1, padding=1, dilation=1, groups=2),
]


@pytest.mark.parametrize("dt", ["float32", "float16"])
@pytest.mark.parametrize("cfg", CONV_CASES, ids=lambda c: f"C{c['C']}O{c['O']}k{c['k']}s{c['stride']}d{c['dilation']}g{c['groups']}")
def test_conv2d(dt, cfg):
    g = Gen(41 + cfg["C"])
    x = g.randn((cfg["B"], cfg["C"], cfg["H"], cfg["W"]), dt)
    w = g.randn((cfg["O"], cfg["C"] // cfg["groups"], cfg["k"], cfg["k"]), dt, 1.0 / np.sqrt(cfg["C"] * 9))
    b = g.randn((cfg["O"],), dt)
    kw = dict(stride=cfg["stride"], padding=cfg["padding"], dilation=cfg["dilation"], groups=cfg["groups"])
    got = host(F.conv2d(dev(x), dev(w), dev(b), **kw))
    assert rel(val(got), val(orc.conv2d(x, w, b, **kw))) <= TOL[dt]


def test_fp16_narrowing_in_gemm_epilogue_is_exact():
    """K = 1 makes every output an exact fp32 product x*w, so the only rounding is the fp16
    narrowing in the epilogue: it must reproduce mtorch's half-away-from-zero rule bit for bit
    on every finite half times factors that create ties (normal and subnormal results) and
    overflow."""
    bits = np.arange(65536, dtype=np.uint16)
    finite = bits[(bits & 0x7C00) != 0x7C00]
    factors = np.array([1.0, 1.0 + 2.0**-10, 1.5, 0.75 + 2.0**-11, 3.0, 2.0**-10, 2.0**-13 * 3, 2.0**-20,
                        1.0 + 2.0**-5, 0.1, 2.0**10 + 1.0, 33.0], dtype=np.float32)
    x = finite.reshape(-1, 1)
    w = orc.f2h(factors).reshape(-1, 1)
    got = host(F.linear(dev(x), dev(w)))
    ref = orc.linear(x, w)
    assert got.dtype == np.uint16 and np.array_equal(got, ref)


def _same_halves(got, ref):
    """Bit-equal fp16 arrays, except that +0 and -0 match (the sign of a zero sum depends on
    the summation order, not on the narrowing) and NaNs match NaNs."""
    g, r = val(got), val(ref)
    gn, rn = np.isnan(g), np.isnan(r)
    zero = (g == 0) & (r == 0)
    bad = (gn != rn) | (~gn & ~rn & ~zero & (got != ref))
    assert not bad.any(), (int(bad.sum()), np.argwhere(bad)[:5], got[bad][:5], ref[bad][:5])


@pytest.mark.parametrize("B,H,W,O", [(2, 64, 64, 80), (1, 63, 64, 100), (2, 32, 32, 80), (1, 16, 16, 80),
                                     (2, 8, 8, 80)])
def test_conv3x3_halo_epilogue_narrowing_is_exact(B, H, W, O):
    """One-hot centre-tap weights (output channel o reads input channel o % 64 times a factor)
    make every conv sum a single exact fp32 product, so the epilogue's narrowings are the only
    rounding: conv + bias, then + residual, each narrowed half-away-from-zero must match the
    oracle bit for bit over every finite half input, on ties (normal and subnormal results),
    subnormal and zero results, overflow to inf, and residual infinities and NaNs (waves that
    meet those redo their values on the general path).  Every latent width's kernel, a partial
    last row block (H = 63) and a partial channel tile (O = 100)."""
    C = 64
    bits = np.arange(65536, dtype=np.uint16)
    finite = bits[(bits & 0x7C00) != 0x7C00]
    n = B * C * H * W
    x = np.resize(finite, n).reshape(B, C, H, W)
    factors = orc.f2h(np.array([1.0, 1.0 + 2.0**-10, 1.5, 0.75 + 2.0**-11, 3.0, 2.0**-10, 2.0**-13 * 3, 2.0**-20,
                                1.0 + 2.0**-5, 0.1, 2.0**10 + 1.0, 33.0, -1.0 - 2.0**-10], dtype=np.float32))
    w = np.zeros((O, C, 3, 3), np.uint16)
    for o in range(O):
        w[o, o % C, 1, 1] = factors[o % len(factors)]
    g = Gen(B * 100 + H + O)
    b = g.randn((O,), "float16")
    b[::3] = 0
    b[1::7] = orc.f2h(np.float32(2.0**-20))
    r = g.randn((B, O, H, W), "float16")
    r[0, 5, H // 2, 7], r[0, O - 1, H - 1, 3], r[B - 1, 33, 0, 0] = 0x7C00, 0xFC00, 0x7E00
    r[0, 7, 2, :8] = 0x7BFF  # 65504: large conv outputs overflow after the add
    ref_conv = orc.conv2d(x, w, b, padding=1)
    got = host(F.conv2d(dev(x), dev(w), dev(b), padding=1))
    _same_halves(got, ref_conv)
    got = host(F.conv2d_residual(dev(x), dev(w), dev(b), dev(r), padding=1))
    _same_halves(got, orc.binary(ref_conv, r, "add"))


@pytest.mark.parametrize("bt", ["64", "128"])
def test_streamed_epilogue_narrowing_is_exact(bt, monkeypatch):
    """The streamed kernel's epilogue (row-major linear and the NCHW 1x1-conv mode, 64- and
    128-token units) on one-hot weights: each output is one exact fp32 product, so + bias,
    narrowed, (+ residual, narrowed) must match the oracle bit for bit over every finite half
    input -- ties, subnormal and zero results, overflow, residual infinities and NaN."""
    from mtorch_amd import _ops
    monkeypatch.setenv("MTHIP_GEMM_STREAM", "2")
    monkeypatch.setenv("MTHIP_CONV_STREAM", "2")
    monkeypatch.setenv("MTHIP_GEMM_STREAM_BT", bt)
    bits = np.arange(65536, dtype=np.uint16)
    finite = bits[(bits & 0x7C00) != 0x7C00]
    factors = orc.f2h(np.array([1.0, 1.0 + 2.0**-10, 1.5, 0.75 + 2.0**-11, 3.0, 2.0**-10, 2.0**-13 * 3, 2.0**-20,
                                1.0 + 2.0**-5, 0.1, 2.0**10 + 1.0, 33.0, -1.0 - 2.0**-10], dtype=np.float32))
    M, K, N = 1024, 320, 200
    x = np.resize(finite, M * K).reshape(M, K)
    w = np.zeros((N, K), np.uint16)
    w[np.arange(N), np.arange(N) % K] = factors[np.arange(N) % len(factors)]
    g = Gen(int(bt))
    b = g.randn((N,), "float16")
    b[::3] = 0
    r = g.randn((M, N), "float16")
    r[5, 7], r[M - 1, N - 1], r[300, 33] = 0x7C00, 0xFC00, 0x7E00
    ref = orc.linear(x, w, b)
    _same_halves(host(F.linear(dev(x), dev(w), dev(b))), ref)
    _same_halves(host(F.linear_residual(dev(x), dev(w), dev(b), dev(r))), orc.binary(ref, r, "add"))
    B, H, W, O = 2, 16, 16, 160
    tok = np.resize(finite[::-1], B * H * W * K).reshape(B, H * W, K)
    xc = np.ascontiguousarray(tok.reshape(B, H, W, K).transpose(0, 3, 1, 2))
    wc = np.zeros((O, K, 1, 1), np.uint16)
    wc[np.arange(O), np.arange(O) % K, 0, 0] = factors[np.arange(O) % len(factors)]
    rc = g.randn((B, O, H, W), "float16")
    rc[1, 3, 4, 5], rc[0, O - 1, 0, 0] = 0x7E00, 0x7C00
    refc = orc.conv2d(xc, wc, b[:O])
    _same_halves(host(_ops.conv2d_tokens(dev(tok), dev(wc), dev(b[:O]), H, W)), refc)
    _same_halves(host(_ops.conv2d_tokens(dev(tok), dev(wc), dev(b[:O]), H, W, residual=dev(rc))),
                 orc.binary(refc, rc, "add"))


def test_tile_gemm_epilogue_narrowing_is_exact(monkeypatch):
    """The tile GEMM's epilogue (fp16 linear with bias and residual, MTHIP_GEMM_STREAM=0 keeping
    the streamed kernel out, and the implicit-GEMM conv with bias and residual: width 24 is not
    a halo-kernel width) on one-hot weights, so each output is one exact product: the
    narrowings must match the oracle bit for bit over every finite half input, ties, subnormal
    and zero results, overflow and residual infinities and NaN included."""
    monkeypatch.setenv("MTHIP_GEMM_STREAM", "0")
    bits = np.arange(65536, dtype=np.uint16)
    finite = bits[(bits & 0x7C00) != 0x7C00]
    factors = orc.f2h(np.array([1.0, 1.0 + 2.0**-10, 1.5, 0.75 + 2.0**-11, 3.0, 2.0**-10, 2.0**-13 * 3, 2.0**-20,
                                1.0 + 2.0**-5, 0.1, 2.0**10 + 1.0, 33.0, -1.0 - 2.0**-10], dtype=np.float32))
    M, K, N = 1024, 64, 256
    x = np.resize(finite, M * K).reshape(M, K)
    w = np.zeros((N, K), np.uint16)
    w[np.arange(N), np.arange(N) % K] = factors[np.arange(N) % len(factors)]
    g = Gen(91)
    b = g.randn((N,), "float16")
    b[::3] = 0
    r = g.randn((M, N), "float16")
    r[5, 7], r[M - 1, N - 1], r[300, 33] = 0x7C00, 0xFC00, 0x7E00
    ref = orc.linear(x, w, b)
    _same_halves(host(F.linear(dev(x), dev(w), dev(b))), ref)
    _same_halves(host(F.linear_residual(dev(x), dev(w), dev(b), dev(r))), orc.binary(ref, r, "add"))
    B, C, H, W, O = 2, 64, 16, 24, 128
    xc = np.resize(finite[::-1], B * C * H * W).reshape(B, C, H, W)
    wc = np.zeros((O, C, 3, 3), np.uint16)
    wc[np.arange(O), np.arange(O) % C, 1, 1] = factors[np.arange(O) % len(factors)]
    bc = b[:O]
    rc = g.randn((B, O, H, W), "float16")
    rc[1, 3, 4, 5], rc[0, O - 1, 0, 0] = 0x7E00, 0x7C00
    refc = orc.conv2d(xc, wc, bc, padding=1)
    _same_halves(host(F.conv2d(dev(xc), dev(wc), dev(bc), padding=1)), refc)
    _same_halves(host(F.conv2d_residual(dev(xc), dev(wc), dev(bc), dev(rc), padding=1)), orc.binary(refc, rc, "add"))


@pytest.mark.parametrize("dt", ["float32", "float16"])
def test_split_k_paths(dt):
    """Shapes whose output tiles cannot fill the chip while K is long take the split-K path
    (fp32 slices reduced in order, then the epilogue): conv with bias + residual, linear with a
    fused activation + residual and a ragged N, and a 2-D addmm."""
    g = Gen(61)
    x = g.randn((1, 256, 4, 4), dt)
    w = g.randn((96, 256, 3, 3), dt, 1.0 / 48)
    b = g.randn((96,), dt)
    r = g.randn((1, 96, 4, 4), dt)
    got = host(F.conv2d_residual(dev(x), dev(w), dev(b), dev(r), padding=1))
    ref = orc.binary(orc.conv2d(x, w, b, padding=1), r, "add")
    assert rel(val(got), val(ref)) <= TOL[dt]
    xl = g.randn((8, 2048), dt)
    wl = g.randn((70, 2048), dt, 1.0 / 45)
    bl = g.randn((70,), dt)
    rl = g.randn((8, 70), dt)
    lin = orc.linear(xl, wl, bl)
    assert rel(val(host(F.linear_gelu(dev(xl), dev(wl), dev(bl)))), val(orc.gelu(lin))) <= TOL[dt]
    got = host(F.linear_residual(dev(xl), dev(wl), dev(bl), dev(rl)))
    assert rel(val(got), val(orc.binary(lin, rl, "add"))) <= TOL[dt]
    inp = g.randn((36,), dt)
    m1 = g.randn((8, 4096), dt)
    m2 = g.randn((4096, 36), dt, 1.0 / 64)
    got = host(mt.addmm(dev(inp), dev(m1), dev(m2), beta=0.5, alpha=1.5))
    assert rel(val(got), val(orc.addmm(inp, m1, m2, 0.5, 1.5))) <= TOL[dt]


@pytest.mark.parametrize("tile", range(6))
def test_direct_to_lds_tile_shapes(tile, monkeypatch):
    """Every direct-to-LDS tile shape and stage count the launcher can pick (forced through
    MTHIP_GEMM_DTL_TILE), on shapes with ragged M/N edges, a K tail, split K, the conv's padded
    taps and channel edges, and the bias/residual/activation epilogues, against the oracle."""
    monkeypatch.setenv("MTHIP_GEMM_DTL_TILE", str(tile))
    g = Gen(90 + tile)
    dt = "float16"
    x = g.randn((203, 328), dt)  # K = 328: 5 whole K tiles and an 8-wide tail
    w = g.randn((150, 328), dt, 1.0 / 18)
    b = g.randn((150,), dt)
    r = g.randn((203, 150), dt)
    lin = orc.linear(x, w, b)
    assert rel(val(host(F.linear(dev(x), dev(w), dev(b)))), val(lin)) <= TOL[dt]
    got = host(F.linear_residual(dev(x), dev(w), dev(b), dev(r)))
    assert rel(val(got), val(orc.binary(lin, r, "add"))) <= TOL[dt]
    assert rel(val(host(F.linear_gelu(dev(x), dev(w), dev(b)))), val(orc.gelu(lin))) <= TOL[dt]
    xl = g.randn((24, 3072), dt)  # long K, few tiles: split K
    wl = g.randn((200, 3072), dt, 1.0 / 55)
    assert rel(val(host(F.linear(dev(xl), dev(wl)))), val(orc.linear(xl, wl, None))) <= TOL[dt]
    xc = g.randn((2, 128, 13, 11), dt)  # channel count a multiple of the K tile: fast im2col
    wc = g.randn((136, 128, 3, 3), dt, 1.0 / 34)
    bc = g.randn((136,), dt)
    rc = g.randn((2, 136, 13, 11), dt)
    got = host(F.conv2d_residual(dev(xc), dev(wc), dev(bc), dev(rc), padding=1))
    ref = orc.binary(orc.conv2d(xc, wc, bc, padding=1), rc, "add")
    assert rel(val(got), val(ref)) <= TOL[dt]
    got = host(F.conv2d(dev(xc), dev(wc), dev(bc), stride=2, padding=1))
    assert rel(val(got), val(orc.conv2d(xc, wc, bc, stride=2, padding=1))) <= TOL[dt]


@pytest.mark.parametrize("dt", ["float32", "float16"])
def test_conv2d_packed_weight_follows_inplace_writes(dt):
    """The packed weight cached on the weight's storage is rebuilt after copy_/fill_."""
    g = Gen(62)
    x = g.randn((2, 24, 9, 9), dt)
    w1 = g.randn((16, 24, 3, 3), dt, 0.1)
    w2 = g.randn((16, 24, 3, 3), dt, 0.1)
    xd, wd = dev(x), dev(w1)
    first = host(F.conv2d(xd, wd, padding=1))
    assert np.array_equal(first, host(F.conv2d(xd, wd, padding=1)))
    assert rel(val(first), val(orc.conv2d(x, w1, None, padding=1))) <= TOL[dt]
    wd.copy_(dev(w2))
    assert rel(val(host(F.conv2d(xd, wd, padding=1))), val(orc.conv2d(x, w2, None, padding=1))) <= TOL[dt]
    wd.fill_(0.25)
    w3 = np.full_like(w2, orc.f2h(np.float32(0.25)) if dt == "float16" else 0.25)
    assert rel(val(host(F.conv2d(xd, wd, padding=1))), val(orc.conv2d(x, w3, None, padding=1))) <= TOL[dt]


@pytest.mark.parametrize("dt", ["float32", "float16"])
def test_conv2d_residual_epilogue(dt):
    g = Gen(51)
    x = g.randn((2, 16, 10, 10), dt)
    w = g.randn((16, 16, 3, 3), dt, 0.1)
    b = g.randn((16,), dt)
    got = host(F.conv2d_residual(dev(x), dev(w), dev(b), dev(x), padding=1))
    ref = orc.binary(x, orc.conv2d(x, w, b, padding=1), "add")
    assert rel(val(got), val(ref)) <= TOL[dt]


# ------------------------------------------------------------------ attention


@pytest.mark.parametrize("dt", ["float16", "float32"])
@pytest.mark.parametrize("Lq,Lk,E", [(256, 256, 40), (300, 77, 40), (130, 130, 80), (64, 200, 160), (33, 17, 64), (5, 9, 7),
                                     (200, 1100, 40), (96, 1024, 32)])
def test_sdpa(dt, Lq, Lk, E):
    """(200, 1100, 40) and (96, 1024, 32) take the two-key-group kernel (>= 1024 keys, head dim
    <= 48): an odd number of 64-key tiles, a ragged last tile, and a query block past Lq."""
    g = Gen(Lq + Lk + E)
    q = g.randn((2, 3, Lq, E), dt)
    k = g.randn((2, 3, Lk, E), dt)
    v = g.randn((2, 3, Lk, E), dt)
    got = host(F.scaled_dot_product_attention(dev(q), dev(k), dev(v)))
    assert rel(val(got), val(orc.sdpa(q, k, v))) <= TOL[dt]


@pytest.mark.parametrize("L,Lk,E", [(4096, 4096, 40), (4096, 77, 40), (1024, 1024, 80), (256, 256, 160)])
def test_sdpa_sd_shapes_query_subset(L, Lk, E):
    """BASELINE.json configs[2] shapes ([2,8,L,E] fp16).  Every query row is independent, so the
    oracle checks a strided subset of rows of the full-size GPU result."""
    g = Gen(L + Lk + E)
    q = g.randn((2, 8, L, E), "float16")
    k = g.randn((2, 8, Lk, E), "float16")
    v = g.randn((2, 8, Lk, E), "float16")
    got = host(F.scaled_dot_product_attention(dev(q), dev(k), dev(v)))
    rows = np.arange(0, L, max(1, L // 48))
    ref = orc.sdpa(np.ascontiguousarray(q[:, :, rows]), k, v)
    assert rel(val(got[:, :, rows]), val(ref)) <= 1e-2


@pytest.mark.parametrize("dt", ["float16", "float32"])
def test_sdpa_masks_causal_scale(dt):
    g = Gen(61)
    q = g.randn((2, 4, 70, 40), dt)
    k = g.randn((2, 4, 90, 40), dt)
    v = g.randn((2, 4, 90, 40), dt)
    rng = np.random.default_rng(0)
    bmask = rng.random((2, 1, 70, 90)) > 0.4
    bmask[..., 0] = True
    amask = (rng.standard_normal((70, 90)) * 2).astype(np.float32)
    cases = [
        dict(attn_mask=bmask, is_causal=False, scale=None),
        dict(attn_mask=amask, is_causal=False, scale=0.2),
        dict(attn_mask=None, is_causal=True, scale=None),
        dict(attn_mask=bmask, is_causal=True, scale=0.3),
    ]
    for c in cases:
        m = c["attn_mask"]
        md = None if m is None else mt.from_numpy(m).to("cuda")
        got = host(F.scaled_dot_product_attention(dev(q), dev(k), dev(v), attn_mask=md, is_causal=c["is_causal"],
                                                  scale=c["scale"]))
        ref = orc.sdpa(q, k, v, m, c["is_causal"], c["scale"])
        assert rel(val(got), val(ref)) <= TOL[dt], c


@pytest.mark.parametrize("dt,E,Lk", [("float16", 40, 1100), ("float16", 40, 77), ("float16", 80, 150),
                                     ("float16", 160, 90), ("float32", 40, 90), ("float32", 160, 77)])
def test_sdpa_explicit_scale(dt, E, Lk):
    """An explicit scale is used as given (tensor.cpp:31019, 31182): 0 (softmax of the mask alone:
    the mean of V over the unmasked keys), a negative scale and a positive one, on the flash
    kernel (fp16; head dims 40/80/160; 1100 keys take the two-key-group instance, 77 a ragged
    tile) and the row-wise kernel (fp32), unmasked, with bool and additive masks and causal."""
    g = Gen(E + Lk + (1 if dt == "float16" else 2))
    q = g.randn((2, 2, 70, E), dt)
    k = g.randn((2, 2, Lk, E), dt)
    v = g.randn((2, 2, Lk, E), dt)
    rng = np.random.default_rng(E + Lk)
    bmask = rng.random((2, 1, 70, Lk)) > 0.4
    bmask[..., 1] = True
    amask = (rng.standard_normal((70, Lk)) * 2).astype(np.float32)
    for scale in (0.0, -0.125, 0.3):
        for m, causal in ((None, False), (bmask, False), (amask, False), (None, True)):
            md = None if m is None else mt.from_numpy(m).to("cuda")
            got = host(F.scaled_dot_product_attention(dev(q), dev(k), dev(v), attn_mask=md, is_causal=causal,
                                                      scale=scale))
            ref = orc.sdpa(q, k, v, m, causal, scale)
            assert rel(val(got), val(ref)) <= TOL[dt], (scale, m is None, causal)
    # scale 0 without a mask: every query gets the mean of V
    got = val(host(F.scaled_dot_product_attention(dev(q), dev(k), dev(v), scale=0.0))).astype(np.float64)
    mean = val(v).astype(np.float64).mean(2, keepdims=True)
    assert rel(got, np.broadcast_to(mean, got.shape)) <= TOL[dt]


@pytest.mark.parametrize("Lq,Lk,E,split", [(1024, 1024, 80, None), (256, 256, 160, None), (1024, 77, 80, None),
                                           (256, 77, 160, "2"), (200, 1100, 40, "3"), (300, 700, 64, "8"),
                                           (130, 520, 160, "5"), (96, 200, 40, "1")])
def test_sdpa_key_splits(Lq, Lk, E, split, monkeypatch):
    """Small query grids split the keys over workgroups (each writes its unnormalised accumulator
    and running max/sum) and a combine kernel merges them: the SD 32x32 / 16x16 self and cross
    shapes at the default split count, and forced counts with a ragged last split, the
    two-key-group instance (1100 keys), dim parts (head dim 160), masks and causal."""
    if split is not None:
        monkeypatch.setenv("MTHIP_FLASH_SPLIT", split)
    g = Gen(Lq + Lk + E + 7)
    q = g.randn((2, 4, Lq, E), "float16")
    k = g.randn((2, 4, Lk, E), "float16")
    v = g.randn((2, 4, Lk, E), "float16")
    rng = np.random.default_rng(Lq + Lk)
    bmask = rng.random((2, 1, Lq, Lk)) > 0.3
    bmask[..., -1] = True
    amask = (rng.standard_normal((Lq, Lk)) * 2).astype(np.float32)
    rows = np.arange(0, Lq, max(1, Lq // 40))
    for m, causal in ((None, False), (bmask, False), (amask, False), (None, True)):
        md = None if m is None else mt.from_numpy(m).to("cuda")
        got = host(F.scaled_dot_product_attention(dev(q), dev(k), dev(v), attn_mask=md, is_causal=causal))
        mr = None if m is None else np.ascontiguousarray(np.broadcast_to(m, (2, 4, Lq, Lk))[:, :, rows])
        if causal:  # the oracle's causal mask counts query positions: evaluate on all rows
            ref = orc.sdpa(q, k, v, None, True)[:, :, rows]
        else:
            ref = orc.sdpa(np.ascontiguousarray(q[:, :, rows]), k, v, mr)
        assert rel(val(got[:, :, rows]), val(ref)) <= TOL["float16"], (m is None, causal)


@pytest.mark.parametrize("Lq,Lk,E,Ev", [(70, 90, 136, 136), (33, 200, 96, 96), (64, 77, 160, 120), (130, 64, 160, 160)])
def test_sdpa_dim_parts(Lq, Lk, E, Ev):
    """Head dims above 80 run four dim parts per 32-query block (each wave: the block's scores, a
    quarter of the output dims): parts with fewer or no 32-dim blocks (136, 96), a value dim
    narrower than the key dim, ragged query blocks, masks and causal."""
    g = Gen(Lq + Lk + E + Ev)
    q = g.randn((2, 3, Lq, E), "float16")
    k = g.randn((2, 3, Lk, E), "float16")
    v = g.randn((2, 3, Lk, Ev), "float16")
    rng = np.random.default_rng(Lq)
    bmask = rng.random((2, 1, Lq, Lk)) > 0.3
    bmask[..., 0] = True
    amask = (rng.standard_normal((Lq, Lk)) * 2).astype(np.float32)
    for m, causal in ((None, False), (bmask, False), (amask, False), (None, True), (bmask, True)):
        md = None if m is None else mt.from_numpy(m).to("cuda")
        got = host(F.scaled_dot_product_attention(dev(q), dev(k), dev(v), attn_mask=md, is_causal=causal))
        assert rel(val(got), val(orc.sdpa(q, k, v, m, causal))) <= TOL["float16"], (m is None, causal)


def test_sdpa_fully_masked_row_is_nan_and_gqa():
    g = Gen(62)
    q = g.randn((1, 4, 40, 40), "float16")
    k = g.randn((1, 2, 50, 40), "float16")
    v = g.randn((1, 2, 50, 40), "float16")
    m = np.ones((40, 50), bool)
    m[7, :] = False
    out = host(F.scaled_dot_product_attention(dev(q), dev(k), dev(v), attn_mask=mt.from_numpy(m).to("cuda"),
                                              enable_gqa=True))
    kr = np.repeat(k, 2, axis=1)
    vr = np.repeat(v, 2, axis=1)
    ref = orc.sdpa(q, kr, vr, m)
    assert rel(val(out), val(ref)) <= 1e-2


def test_sd_cross_attention_scenario_fixture():
    """Reference scenario tests/compat/test_tensor_ops.py:2105-2158 in fp16 on the GPU."""
    c = closed_form.sd_cross_attention_inputs()
    exp = np.load(os.path.join(HERE, "golden", "sd_cross_attention_2x64x77x320.npz"))["attended"]
    h = lambda a: dev(orc.f2h(a))  # noqa: E731
    q = F.linear(h(c["hidden"]), h(c["qw"]), h(c["bias"])).reshape(2, 64, 8, 40).transpose(1, 2).reshape(16, 64, 40)
    k = F.linear(h(c["enc"]), h(c["kw"]), h(c["bias"])).reshape(2, 77, 8, 40).transpose(1, 2).reshape(16, 77, 40)
    v = F.linear(h(c["enc"]), h(c["vw"]), h(c["bias"])).reshape(2, 77, 8, 40).transpose(1, 2).reshape(16, 77, 40)
    att = F.scaled_dot_product_attention(q, k, v, attn_mask=mt.from_numpy(c["mask"]).to("cuda"), scale=0.125)
    assert np.allclose(orc.h2f(host(att)), exp, rtol=4e-3, atol=4e-3)  # the reference test's tolerance


# ------------------------------------------------------------------ normalisation / softmax


@pytest.mark.parametrize("dt", ["float32", "float16"])
@pytest.mark.parametrize("shape,groups", [((2, 64, 16, 16), 32), ((1, 40, 7, 9), 8), ((3, 32, 5), 4), ((2, 320, 64, 64), 32)])
def test_group_norm(dt, shape, groups):
    g = Gen(71 + shape[1])
    x = g.randn(shape, dt)
    w = g.randn((shape[1],), dt)
    b = g.randn((shape[1],), dt)
    got = host(F.group_norm(dev(x), groups, dev(w), dev(b), 1e-5))
    ref = orc.group_norm(x, groups, w, b, 1e-5)
    assert rel(val(got), val(ref)) <= TOL[dt]
    got = host(F.group_norm_silu(dev(x), groups, dev(w), dev(b), 1e-5))
    assert rel(val(got), val(orc.silu(ref))) <= TOL[dt]


@pytest.mark.parametrize("dt", ["float16", "float32"])
@pytest.mark.parametrize("shape,groups", [((16, 320, 64, 64), 32), ((24, 320, 32, 32), 32), ((8, 64, 59, 104), 64),
                                          ((40, 64, 9, 16), 16)])
def test_group_norm_single_pass_large_batch(dt, shape, groups, monkeypatch):
    """With >= 2 (sample, group) pairs per CU, NCHW GroupNorm runs in one pass (a workgroup holds
    its whole group in registers, four 256-thread parts replaying the stats kernel): bit for bit
    the two-kernel result (MTHIP_GN_SINGLE=0), with
    and without the fused SiLU, with fp16 or fp32 affine parameters, including a last stats chunk
    shorter than the rest (one-channel groups of 59x104 pixels), and checked against the oracle on
    a few samples.  (Groups of 9x16 pixels take the two-kernel path: chunks shorter than a
    workgroup's vector sweep.)"""
    from mtorch_amd import _ops
    g = Gen(sum(shape) + groups)
    x = g.randn(shape, dt)
    C = shape[1]
    w, b = g.randn((C,), dt), g.randn((C,), dt)
    w32, b32 = g.randn((C,), "float32"), g.randn((C,), "float32")
    runs = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("MTHIP_GN_SINGLE", mode)
        runs[mode] = [host(F.group_norm(dev(x), groups, dev(w), dev(b), 1e-5)),
                      host(F.group_norm_silu(dev(x), groups, dev(w), dev(b), 1e-5)),
                      host(F.group_norm(dev(x), groups, None, None, 1e-5))]
        if dt == "float16":
            runs[mode].append(host(_ops.group_norm(dev(x), groups, dev(w32), dev(b32), 1e-5, allow_upcast=True)))
    for got, want in zip(runs["1"], runs["0"]):
        assert np.array_equal(got, want)
    xs = np.ascontiguousarray(x[::7])
    ref = orc.group_norm(xs, groups, w, b, 1e-5)
    assert rel(val(runs["1"][0][::7]), val(ref)) <= TOL[dt]
    assert rel(val(runs["1"][1][::7]), val(orc.silu(ref))) <= TOL[dt]


GN1_CASES = [
    # B, C0, C1, H, W, groups, parameter dtype, silu, workgroups per group (None: the default)
    (2, 320, 0, 64, 64, 32, "float16", 1, None),  # the bench sub-block
    (2, 320, 0, 64, 64, 32, "float32", 1, None),
    (2, 320, 0, 64, 64, 32, "float16", 0, "1"),
    (2, 320, 0, 64, 64, 32, "float16", 1, "2"),
    (2, 640, 0, 32, 32, 32, "float32", 1, None),
    (2, 1280, 0, 32, 32, 32, "float32", 1, None),
    (2, 1280, 0, 16, 16, 32, "float32", 0, None),
    (2, 1280, 0, 8, 8, 32, "float32", 1, None),
    (2, 2560, 0, 8, 8, 32, "float32", 1, None),
    (2, 640, 320, 32, 32, 32, "float32", 1, None),  # up-block cat inputs, read in place
    (2, 1280, 640, 16, 16, 32, "float32", 1, None),
    (2, 1280, 1280, 16, 16, 32, "float32", 1, None),
    (2, 1280, 1280, 8, 8, 32, "float32", 1, "4"),
    (2, 640, 320, 64, 64, 32, "float32", 1, None),  # 60 stats chunks per group (15 per part)
    (2, 320, 320, 64, 64, 32, "float32", 1, None),  # 40
    (2, 1280, 640, 32, 32, 32, "float32", 1, None),  # 30 (8 per part)
    (1, 640, 0, 64, 64, 32, "float16", 1, None),  # 40, one source, against the oracle too
    (3, 36, 0, 12, 20, 6, "float16", 1, None),  # channel padding (Cp 40 > C), 6-channel groups
    (1, 18, 22, 8, 8, 4, "float16", 1, None),  # a group straddling the two sources
    (4, 64, 0, 16, 24, 8, "float16", 1, None),  # 16-byte stores (8-channel groups)
    (2, 160, 160, 64, 64, 32, "float16", 1, None),  # 10-channel groups at 64x64, concatenated input
    (1, 310, 0, 64, 64, 31, "float16", 1, None),  # ... with channel padding (Cp 312), 31 groups
]


@pytest.mark.parametrize("B,C0,C1,H,W,G,pdt,silu,split", GN1_CASES)
def test_group_norm_nhwc_one_launch_equals_two_kernels(B, C0, C1, H, W, G, pdt, silu, split, monkeypatch):
    """The one-launch channels-last GroupNorm (a 1024-thread workgroup per (sample, group) or
    per part of one, replaying the stats kernel's sums) against the stats + apply kernels
    (MTHIP_GN_ONEPASS=0): the normalised (+SiLU) output and, for the concatenated input, the raw
    channels-last copy, bit for bit, including the zero padding channels; the one-source fp16
    cases also against the oracle."""
    from mtorch_amd import _lib
    L = _lib.lib()
    g = Gen(B + C0 + C1 + H + W + G)
    C, HW = C0 + C1, H * W
    Cp = -(-C // 8) * 8
    x0 = dev(g.randn((B, C0, H, W), "float16"))
    x1 = dev(g.randn((B, C1, H, W), "float16")) if C1 else None
    pt = getattr(mt, pdt)
    w = mt.from_numpy(g.randn((C,), pdt), dtype=pt).to("cuda")
    b = mt.from_numpy(g.randn((C,), pdt), dtype=pt).to("cuda")
    if split is not None:
        monkeypatch.setenv("MTHIP_GN1_SPLIT", split)
    outs = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("MTHIP_GN_ONEPASS", mode)
        y = mt.full((B, HW, Cp), 7.0, dtype=mt.float16, device="cuda")  # padding must come back zero
        r = mt.full((B, HW, Cp), 7.0, dtype=mt.float16, device="cuda")
        if C1:
            _lib.check(L.mthip_group_norm_nhwc_cat(0, _lib.F16, x0.data_ptr(), C0, x1.data_ptr(), C1, w.data_ptr(),
                                                   b.data_ptr(), y.data_ptr(), r.data_ptr(), B, HW, G, 1e-5, silu,
                                                   pt.code))
        else:
            _lib.check(L.mthip_group_norm_nhwc(0, _lib.F16, x0.data_ptr(), w.data_ptr(), b.data_ptr(), y.data_ptr(), B,
                                               C, HW, G, 1e-5, silu, pt.code))
        outs[mode] = (host(y), host(r) if C1 else None)
    assert np.array_equal(outs["1"][0], outs["0"][0])
    if C1:
        assert np.array_equal(outs["1"][1], outs["0"][1])
    if Cp > C:
        assert not outs["1"][0][..., C:].any()
    if not C1 and pdt == "float16":
        xs = host(x0)[:1]
        ref = orc.group_norm(xs, G, host(w), host(b), 1e-5)
        if silu:
            ref = orc.silu(ref)
        got = outs["1"][0][:1, :, :C].transpose(0, 2, 1).reshape(1, C, H, W)
        assert rel(val(got), val(ref)) <= TOL["float16"]


@pytest.mark.parametrize("shape", [(16, 320, 64, 64), (2, 320, 64, 64)])
def test_group_norm_leaves_allocated_bytes_unchanged(shape, monkeypatch):
    """Neither GroupNorm path keeps device memory past the call: the one-pass kernel (16 samples:
    512 (sample, group) pairs) needs no partials buffer, the two-kernel path (2 samples) returns
    its partials block to the cache.  Checked through the C ABI into existing outputs and through
    F.group_norm / F.group_norm_silu with their outputs dropped."""
    monkeypatch.setenv("MTHIP_GN_SINGLE", "1")
    g = Gen(sum(shape))
    xd = dev(g.randn(shape, "float16"))
    wd, bd = dev(g.randn((shape[1],), "float16")), dev(g.randn((shape[1],), "float16"))
    y1 = F.group_norm(xd, 32, wd, bd, 1e-5)  # warm the caches (tables, blocks)
    y2 = F.group_norm_silu(xd, 32, wd, bd, 1e-5)
    mt.cuda.synchronize()
    before = mt.cuda.memory_allocated()
    for _ in range(3):
        _ops_gn_into(xd, wd, bd, y1, silu=False)
        _ops_gn_into(xd, wd, bd, y2, silu=True)
    mt.cuda.synchronize()
    assert mt.cuda.memory_allocated() == before
    for _ in range(3):
        t = F.group_norm(xd, 32, wd, bd, 1e-5)
        u = F.group_norm_silu(xd, 32, wd, bd, 1e-5)
        assert np.array_equal(host(t), host(y1)) and np.array_equal(host(u), host(y2))
        del t, u
    mt.cuda.synchronize()
    assert mt.cuda.memory_allocated() == before


def _ops_gn_into(xd, wd, bd, y, silu):
    """mthip_group_norm into an existing output (so the count sees only the call's own memory)."""
    from mtorch_amd import _lib
    B, C = xd.shape[0], xd.shape[1]
    inner = xd.numel() // (B * C)
    _lib.check(_lib.lib().mthip_group_norm(0, xd.dtype.code, xd.data_ptr(), wd.data_ptr(), bd.data_ptr(),
                                           y.data_ptr(), B, C, inner, 32, 1e-5, 1 if silu else 0, xd.dtype.code))


@pytest.mark.parametrize("dt", ["float32", "float16"])
@pytest.mark.parametrize("B,C,H,W,O,G", [(2, 64, 16, 16, 48, 32), (1, 12, 9, 11, 8, 4), (2, 40, 8, 8, 40, 8)])
def test_group_norm_silu_conv2d_channels_last_handoff(dt, B, C, H, W, O, G):
    """GN -> SiLU written channels-last and consumed by the conv equals the three-op sequence
    (channel padding, ragged pixel tiles and the residual epilogue included)."""
    g = Gen(B * 1000 + C + O)
    x = g.randn((B, C, H, W), dt)
    gamma = g.randn((C,), dt)
    beta = g.randn((C,), dt)
    w = g.randn((O, C, 3, 3), dt, 1.0 / np.sqrt(9 * C))
    b = g.randn((O,), dt)
    r = g.randn((B, O, H, W), dt)
    h = orc.silu(orc.group_norm(x, G, gamma, beta, 1e-5))
    ref = orc.binary(orc.conv2d(h, w, b, padding=1), r, "add")
    got = host(F.group_norm_silu_conv2d(dev(x), G, dev(gamma), dev(beta), 1e-5, dev(w), dev(b), padding=1,
                                        residual=dev(r)))
    assert rel(val(got), val(ref)) <= TOL[dt]
    got = host(F.group_norm_silu_conv2d(dev(x), G, dev(gamma), dev(beta), 1e-5, dev(w), None, stride=2, padding=1))
    assert rel(val(got), val(orc.conv2d(h, w, None, stride=2, padding=1))) <= TOL[dt]


@pytest.mark.parametrize("B,C,H,W,O", [(2, 64, 64, 64, 80), (1, 128, 5, 64, 100), (2, 64, 32, 32, 160),
                                         (2, 192, 16, 16, 96), (1, 320, 8, 8, 80), (2, 60, 9, 16, 64),
                                         (1, 128, 3, 32, 240)])
def test_conv3x3_halo_kernel_shapes(B, C, H, W, O):
    """fp16 3x3 s1 p1 convs of 64-channel blocks take the halo kernel: every latent width (64,
    32, 16, 8), a partial last row block, a partial last channel tile, padded input channels and
    the channel-block split with its reduction; with bias, residual and the channel addend."""
    g = Gen(B * 7000 + C * 13 + H * 3 + O)
    x = g.randn((B, C, H, W), "float16")
    w = g.randn((O, C, 3, 3), "float16", 1.0 / np.sqrt(9 * C))
    b = g.randn((O,), "float16")
    r = g.randn((B, O, H, W), "float16")
    t = g.randn((B, O), "float16")
    got = host(F.conv2d_residual(dev(x), dev(w), dev(b), dev(r), padding=1))
    conv = orc.conv2d(x, w, b, padding=1)
    assert rel(val(got), val(orc.binary(conv, r, "add"))) <= 1e-2
    got = host(F.conv2d(dev(x), dev(w), None, padding=1))
    assert rel(val(got), val(orc.conv2d(x, w, None, padding=1))) <= 1e-2
    # through the channels-last hand-off, with the time-embedding addend fused
    gamma = g.randn((C,), "float16")
    beta = g.randn((C,), "float16")
    groups = 4
    fused = host(F.group_norm_silu_conv2d(dev(x), groups, dev(gamma), dev(beta), 1e-5, dev(w), dev(b), padding=1,
                                          chan_add=dev(t), residual=dev(r)))
    h = orc.silu(orc.group_norm(x, groups, gamma, beta, 1e-5))
    ref = val(orc.conv2d(h, w, b, padding=1)).astype(np.float64) + val(t)[:, :, None, None] + val(r)
    assert rel(val(fused), ref) <= 1e-2


@pytest.mark.parametrize("C,H", [(640, 16), (1280, 16), (1280, 13)])
def test_conv3x3_halo_whole_image_tiles(C, H):
    """Wide convs at width 16 (SD's 1280-channel 16x16 latent) run 48-channel units over a whole
    16-row image with the channel blocks split over K and reduced: checked against the oracle on
    a strided subset of output channels that includes the partial last 48-channel tile, with
    bias and residual, and with the time-embedding addend through the fused GroupNorm path."""
    B, W, O = 2, 16, 1280
    g = Gen(C + H + 77)
    x = g.randn((B, C, H, W), "float16")
    w = g.randn((O, C, 3, 3), "float16", 1.0 / np.sqrt(9 * C))
    b = g.randn((O,), "float16")
    r = g.randn((B, O, H, W), "float16")
    t = g.randn((B, O), "float16")
    sel = np.r_[np.arange(0, O, 37), np.arange(O - 40, O)]
    ws, bs = np.ascontiguousarray(w[sel]), np.ascontiguousarray(b[sel])
    got = host(F.conv2d_residual(dev(x), dev(w), dev(b), dev(r), padding=1))[:, sel]
    ref = orc.binary(orc.conv2d(x, ws, bs, padding=1), np.ascontiguousarray(r[:, sel]), "add")
    assert rel(val(got), val(ref)) <= 1e-2
    got = host(F.conv2d(dev(x), dev(w), None, padding=1))[:, sel]
    assert rel(val(got), val(orc.conv2d(x, ws, None, padding=1))) <= 1e-2
    gamma = g.randn((C,), "float16")
    beta = g.randn((C,), "float16")
    fused = host(F.group_norm_silu_conv2d(dev(x), 32, dev(gamma), dev(beta), 1e-5, dev(w), dev(b), padding=1,
                                          chan_add=dev(t)))[:, sel]
    h = orc.silu(orc.group_norm(x, 32, gamma, beta, 1e-5))
    ref = val(orc.conv2d(h, ws, bs, padding=1)).astype(np.float64) + val(t)[:, sel, None, None]
    assert rel(val(fused), ref) <= 1e-2


@pytest.mark.parametrize("B,C,H,W,O", [(2, 320, 8, 8, 320), (2, 640, 4, 4, 640), (2, 960, 6, 6, 320),
                                         (1, 1920, 4, 5, 640), (2, 320, 8, 8, 1280), (1, 640, 2, 6, 48),
                                         (2, 320, 64, 64, 320)])
@pytest.mark.parametrize("bt", ["64", "128"])
def test_conv1x1_streamed_nchw(B, C, H, W, O, bt, monkeypatch):
    """fp16 1x1 convs of a channels-last activation with K a multiple of 320 take the streamed
    kernel in its NCHW mode (the SD transformer's proj_out, the ResBlock shortcuts), through
    conv2d_tokens (bias + residual, and no bias) and through conv2d on an NCHW input: checked
    against the oracle on a strided subset of output channels, as is the implicit-GEMM path
    (MTHIP_CONV_STREAM=0; its fp32 sums are grouped differently, so the two agree to rounding,
    not bit for bit).  Covers partial 80-channel and 64/128-token tiles (MTHIP_GEMM_STREAM_BT),
    images that split a token tile (6x6, and 8x8 under 128-token units), K splits with the conv
    reduction (K = 1920 over few pixels), forced, 1280 output channels, and the 64x64 proj_out."""
    from mtorch_amd import _ops
    monkeypatch.setenv("MTHIP_GEMM_STREAM_BT", bt)
    g = Gen(B + C + H + W + O)
    x = g.randn((B, C, H, W), "float16")
    w = g.randn((O, C, 1, 1), "float16", 1.0 / np.sqrt(C))
    b = g.randn((O,), "float16")
    r = g.randn((B, O, H, W), "float16")
    tok = np.ascontiguousarray(x.transpose(0, 2, 3, 1).reshape(B, H * W, C))
    sel = np.unique(np.r_[np.arange(0, O, 7), O - 1])
    ws, bs = np.ascontiguousarray(w[sel]), np.ascontiguousarray(b[sel])
    refs = (orc.binary(orc.conv2d(x, ws, bs), np.ascontiguousarray(r[:, sel]), "add"), orc.conv2d(x, ws, None),
            orc.conv2d(x, ws, bs))
    for mode in ("2", "0"):
        monkeypatch.setenv("MTHIP_CONV_STREAM", mode)
        outs = (host(_ops.conv2d_tokens(dev(tok), dev(w), dev(b), H, W, residual=dev(r))),
                host(_ops.conv2d_tokens(dev(tok), dev(w), None, H, W)), host(F.conv2d(dev(x), dev(w), dev(b))))
        for got, ref in zip(outs, refs):
            assert got.shape == (B, O, H, W)
            assert rel(val(got[:, sel]), val(ref)) <= 1e-2


@pytest.mark.parametrize("dt", ["float32", "float16"])
@pytest.mark.parametrize("B,C,H,W,O,G", [(2, 64, 16, 16, 48, 32), (2, 40, 9, 7, 40, 8), (1, 16, 8, 8, 24, 4)])
def test_group_norm_silu_conv2d_channel_add_is_the_separate_add(dt, B, C, H, W, O, G):
    """The time-embedding add fused into the conv epilogue (chan_add, here a strided slice of a
    wider projection) gives exactly the unfused conv -> add (-> residual add) sequence, and both
    match the oracle."""
    g = Gen(B * 2000 + C + O)
    x = g.randn((B, C, H, W), dt)
    gamma = g.randn((C,), dt)
    beta = g.randn((C,), dt)
    w = g.randn((O, C, 3, 3), dt, 1.0 / np.sqrt(9 * C))
    b = g.randn((O,), dt)
    r = g.randn((B, O, H, W), dt)
    proj = dev(g.randn((B, O + 24), dt))
    t = proj[:, 16:16 + O]  # row stride O + 24
    args = (G, dev(gamma), dev(beta), 1e-5, dev(w), dev(b))
    xd, rd = dev(x), dev(r)
    plain = F.group_norm_silu_conv2d(xd, *args, padding=1)
    sep = plain + t.unsqueeze(-1).unsqueeze(-1)
    fused = F.group_norm_silu_conv2d(xd, *args, padding=1, chan_add=t)
    assert np.array_equal(host(fused).view(np.uint8), host(sep).view(np.uint8))
    sep_res = sep + rd
    fused_res = F.group_norm_silu_conv2d(xd, *args, padding=1, chan_add=t, residual=rd)
    assert np.array_equal(host(fused_res).view(np.uint8), host(sep_res).view(np.uint8))
    h = orc.silu(orc.group_norm(x, G, gamma, beta, 1e-5))
    tt = np.asarray(val(host(t)), dtype=np.float64)[:, :, None, None]
    ref = val(orc.conv2d(h, w, b, padding=1)) + tt + val(r)
    assert rel(val(host(fused_res)), ref) <= TOL[dt]


@pytest.mark.parametrize("B,C0,C1,H,W,O,G,pdt", [(2, 640, 320, 16, 16, 320, 32, "float16"),
                                                 (2, 64, 64, 8, 8, 48, 32, "float16"),
                                                 (1, 48, 16, 9, 8, 32, 8, "float32"),
                                                 (1, 320, 0, 32, 32, 640, 32, "float16"),
                                                 (1, 640, 0, 16, 16, 1280, 32, "float16")])
def test_group_norm_silu_conv2d_cat_equals_cat_then_ops(B, C0, C1, H, W, O, G, pdt):
    """An up-block ResBlock entry on cat([x0, x1], dim=1) read in place (groups straddling the
    two inputs at C0=640, C1=320: 30-channel groups) gives the explicit cat -> GN -> SiLU -> conv
    (+ time add) and the 1x1 shortcut conv on the concatenation bit for bit, and the oracle's
    values; fp32 GN parameters are the upcast pattern.  C1 = 0 (x1 None): the down-block
    ResBlocks whose shortcut reads the GroupNorm's channels-last copy of their one input."""
    from mtorch_amd import _ops

    g = Gen(B * 300 + C0 + C1 + O)
    x0 = g.randn((B, C0, H, W), "float16")
    x1 = g.randn((B, C1, H, W), "float16") if C1 else None
    C = C0 + C1
    gamma, beta = g.randn((C,), pdt), g.randn((C,), pdt)
    w, b = g.randn((O, C, 3, 3), "float16", 1.0 / np.sqrt(9 * C)), g.randn((O,), "float16")
    sw, sb = g.randn((O, C, 1, 1), "float16", 1.0 / np.sqrt(C)), g.randn((O,), "float16")
    t = dev(g.randn((B, O), "float16"))
    xd = mt.cat([dev(x0), dev(x1)], dim=1) if C1 else dev(x0)
    x1d = dev(x1) if C1 else None
    args = (G, dev(gamma), dev(beta), 1e-5)
    r = _ops.group_norm_silu_conv2d_cat(dev(x0), x1d, *args, dev(w), dev(b), 1, t, dev(sw), dev(sb))
    assert r is not None
    out, sc = r
    ref_out = F.group_norm_silu_conv2d(xd, *args, dev(w), dev(b), padding=1, chan_add=t)
    ref_sc = F.conv2d(xd, dev(sw), dev(sb))
    assert np.array_equal(host(out), host(ref_out)) and np.array_equal(host(sc), host(ref_sc))
    xc = np.concatenate([x0, x1], axis=1) if C1 else x0
    if pdt == "float16":
        h = orc.silu(orc.group_norm(xc, G, gamma, beta, 1e-5))
    else:
        h = orc.silu(orc.f2h(orc.group_norm(orc.h2f(xc), G, gamma, beta, 1e-5)))
    ref = val(orc.conv2d(h, w, b, padding=1)) + np.asarray(val(host(t)), np.float64)[:, :, None, None]
    assert rel(val(host(out)), ref) <= 1e-2
    assert rel(val(host(sc)), val(orc.conv2d(xc, sw, sb))) <= 1e-2
    # shapes the channels-last fp16 kernel cannot take are declined (the caller concatenates)
    assert _ops.group_norm_silu_conv2d_cat(dev(x0)[:, :C0 - 1], x1d, *args, dev(w), dev(b), 1, t, dev(sw),
                                           dev(sb)) is None


@pytest.mark.parametrize("B,C,H,W,O", [(2, 1280, 8, 8, 1280), (2, 1280, 16, 16, 1280), (1, 640, 32, 32, 640),
                                         (1, 24, 5, 7, 16)])
def test_upsample2x_conv2d_equals_interpolate_then_conv(B, C, H, W, O):
    """The SD decoder's Upsample block through mthip_upsample2x_to_nhwc + the channels-last conv
    gives interpolate(nearest, x2) -> conv2d 3x3 bit for bit (the halo kernel at 16x16, 32x32
    and 64x64 outputs, the implicit GEMM for a ragged small one); the staging entry itself
    against numpy's repeat + transpose, with zero padding channels (Cp > C), for fp16 and fp32."""
    from mtorch_amd import _lib, _ops

    g = Gen(B * 17 + C + H * 5 + W + O)
    x = g.randn((B, C, H, W), "float16")
    w, b = g.randn((O, C, 3, 3), "float16", 1.0 / np.sqrt(9 * C)), g.randn((O,), "float16")
    got = _ops.upsample2x_conv2d(dev(x), dev(w), dev(b), padding=1)
    assert got is not None
    ref = F.conv2d(F.interpolate(dev(x), scale_factor=2, mode="nearest"), dev(w), dev(b), padding=1)
    assert np.array_equal(host(got).view(np.uint16), host(ref).view(np.uint16))
    L = _lib.lib()
    for dt, code in (("float16", _lib.F16), ("float32", _lib.F32)):
        xs = g.randn((B, C, H, W), dt)
        Cp = C + 8
        xp = mt.full((B, 4 * H * W, Cp), 7.0, dtype=getattr(mt, dt), device="cuda")
        _lib.check(L.mthip_upsample2x_to_nhwc(0, code, dev(xs).data_ptr(), xp.data_ptr(), B, C, Cp, H, W))
        up = xs.repeat(2, axis=2).repeat(2, axis=3).reshape(B, C, 4 * H * W).transpose(0, 2, 1)
        want = np.concatenate([up, np.zeros((B, 4 * H * W, 8), up.dtype)], axis=2)
        assert np.array_equal(host(xp), want)


@pytest.mark.parametrize("shape,groups", [((2, 320, 64, 64), 32), ((1, 640, 16, 16), 32), ((2, 64, 7, 9), 8)])
def test_group_norm_silu_fp16_equals_group_norm_then_silu(shape, groups):
    """The fused fp16 GroupNorm+SiLU (SiLU applied to the narrowed halves) writes exactly the
    halves of group_norm followed by silu."""
    g = Gen(sum(shape) + groups)
    x = g.randn(shape, "float16", 2.0)
    w, b = g.randn((shape[1],), "float16"), g.randn((shape[1],), "float16")
    fused = host(F.group_norm_silu(dev(x), groups, dev(w), dev(b), 1e-5))
    sep = host(F.silu(F.group_norm(dev(x), groups, dev(w), dev(b), 1e-5)))
    assert np.array_equal(fused, sep)


@pytest.mark.parametrize("B,C,H,W,G,pdt", [(2, 1280, 8, 8, 32, "float16"), (2, 640, 16, 16, 32, "float16"),
                                            (2, 960, 16, 16, 32, "float32"), (1, 64, 8, 8, 8, "float16"),
                                            (2, 320, 32, 32, 32, "float16"), (2, 2560, 8, 8, 32, "float16")])
def test_group_norm_channels_last_equals_nchw_bit_for_bit(B, C, H, W, G, pdt):
    """The channels-last GroupNorm (stats + transposing apply) writes exactly the values of the
    NCHW group_norm, permuted, at every SD latent size."""
    from mtorch_amd import sd_unet

    g = Gen(B + C + H)
    x = g.randn((B, C, H, W), "float16")
    gamma, beta = g.randn((C,), pdt), g.randn((C,), pdt)

    class Norm:
        weight, bias, groups, eps = dev(gamma), dev(beta), G, 1e-5

    tok = host(sd_unet._tokens_nhwc(dev(x), Norm))
    from mtorch_amd import _ops

    ref = host(_ops.group_norm(dev(x), G, dev(gamma), dev(beta), 1e-5, allow_upcast=True))
    assert np.array_equal(tok, np.ascontiguousarray(ref.transpose(0, 2, 3, 1)).reshape(B, H * W, C))


def test_sd_group_norm_scenario_fixture():
    hidden, w, b = closed_form.sd_group_norm_inputs()
    exp = np.load(os.path.join(HERE, "golden", "sd_group_norm_1x320x16x16.npz"))["y"]
    got = host(F.group_norm(dev(orc.f2h(hidden)), 32, dev(orc.f2h(w)), dev(orc.f2h(b)), eps=1e-5))
    assert np.allclose(orc.h2f(got), exp, rtol=3e-3, atol=3e-3)
    got32 = host(F.group_norm(dev(hidden), 32, dev(w), dev(b), eps=1e-5))
    assert np.allclose(got32, exp, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("dt", ["float32", "float16"])
@pytest.mark.parametrize("rows,n", [(2048, 320), (2049, 320), (1000, 640), (77, 768), (50, 1280), (13, 3000), (9, 100),
                                    (4096, 640), (2050, 1280)])
def test_layer_norm(dt, rows, n):
    g = Gen(81 + n)
    x = g.randn((rows, n), dt, 2.0)
    w = g.randn((n,), dt)
    b = g.randn((n,), dt)
    got = host(F.layer_norm(dev(x), (n,), dev(w), dev(b), 1e-5))
    assert rel(val(got), val(orc.layer_norm(x, n, w, b, 1e-5))) <= TOL[dt]


@pytest.mark.parametrize("dt", ["float32", "float16"])
@pytest.mark.parametrize("shape", [(4, 3, 77), (64, 1024), (2, 5000), (3, 4, 4096), (7,), (5, 320), (3, 2048)])
def test_softmax(dt, shape):
    g = Gen(91 + shape[-1])
    x = g.randn(shape, dt, 3.0)
    got = host(F.softmax(dev(x), dim=-1))
    assert rel(val(got), val(orc.softmax_lastdim(x))) <= TOL[dt]


@pytest.mark.parametrize("shape", [(64, 1024), (333, 77), (3, 5000)])
def test_softmax_fp16_within_one_ulp(shape):
    """The 16-bit softmax takes e^d as the native 2^(d log2 e): every output stays within one
    fp16 ulp of the oracle's (tensor.cpp:15145-15221), on each of the three kernels -- rows of
    whole 16-byte chunks in registers, short ragged rows, rows past 4096 columns."""
    g = Gen(97 + shape[-1])
    x = g.randn(shape, "float16", 4.0)
    got = host(F.softmax(dev(x), dim=-1))
    ref = orc.softmax_lastdim(x)
    assert got.dtype == np.uint16 and ref.dtype == np.uint16
    # outputs are >= +0, so the distance in ulps is the difference of the bit patterns
    d = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    assert d.max() <= 1, (int(d.max()), int((d > 1).sum()))
    assert (d == 0).mean() > 0.99


@pytest.mark.parametrize("src,out", [("float32", "float16"), ("float16", "float32")])
def test_softmax_with_another_output_dtype(src, out):
    """softmax(x, dtype=...) reads x at its own precision and narrows only the results
    (tensor.cpp:15165-15207), so large logits that one fp16 value cannot tell apart still get
    their own probabilities."""
    g = Gen(93)
    x = g.randn((64, 77), src, 4.0)
    if src == "float32":
        x[0, :2] = [1000.0, 1000.3]
        x[0, 2:] = -np.inf
    got = host(F.softmax(dev(x), dim=-1, dtype=getattr(mt, out)))
    ref = orc.softmax_generic(x, out)
    assert rel(val(got), val(ref)) <= TOL[out]
    if src == "float32":
        assert abs(float(val(got)[0, 1]) - 0.5742) < 1e-3


def test_copy_into_strided_views():
    """copy_/item assignment of a tensor into a non-contiguous device view, with broadcasting
    and an overlapping source (Tensor::copy_from, tensor.cpp:8292-8340)."""
    g = Gen(94)
    a = g.randn((6, 10), "float32")
    d = dev(a)
    src = g.randn((6, 4), "float32")
    d[:, 3:7] = dev(src)
    exp = a.copy()
    exp[:, 3:7] = src
    assert np.array_equal(host(d), exp)
    row = g.randn((5,), "float32")
    d[1:, ::2] = dev(row)  # broadcast over rows, every other column
    exp[1:, ::2] = row
    assert np.array_equal(host(d), exp)
    d[:, 1:] = d[:, :-1]  # overlapping shift: staged, so every value is read before it is overwritten
    exp[:, 1:] = exp[:, :-1].copy()
    assert np.array_equal(host(d), exp)
    h = dev(g.randn((4, 8), "float16"))
    hx = host(h).copy()
    v = g.randn((4, 3), "float32")
    h[:, 2:8:2][:, :3] = dev(v)  # dtype conversion on the way in
    hx[:, 2:8:2] = orc.f2h(v)
    assert np.array_equal(host(h), hx)


def test_copy_into_expanded_destination_last_write_wins():
    """A destination with zero strides (an expanded view) overlaps itself.  The reference writes
    every index in row-major order (tensor.cpp:8335-8338), so each element ends as the value of
    the last index along the expanded dims; the device copy gives exactly that."""
    g = Gen(95)
    base = dev(np.zeros((3, 1, 5), np.float32))
    src = g.randn((3, 4, 5), "float32")
    base.expand(3, 4, 5).copy_(dev(src))
    assert np.array_equal(host(base), src[:, 3:4, :])
    row = dev(np.zeros((1, 6), np.float32))
    s2 = g.randn((5, 6), "float32")
    row.expand(5, 6).copy_(dev(s2).transpose(0, 1).transpose(0, 1))
    assert np.array_equal(host(row), s2[4:5])


def test_softmax_other_dim():
    g = Gen(92)
    x = g.randn((5, 6, 7), "float32")
    got = host(F.softmax(dev(x), dim=1))
    e = np.exp(x.astype(np.float64) - x.max(1, keepdims=True))
    assert rel(got, e / e.sum(1, keepdims=True)) <= 1e-6


# ------------------------------------------------------------------ glue + graphs


def test_cat_and_upsample():
    g = Gen(101)
    a = g.randn((2, 3, 4, 5), "float16")
    b = g.randn((2, 6, 4, 5), "float16")
    got = host(mt.cat([dev(a), dev(b)], dim=1))
    assert np.array_equal(got, np.concatenate([a, b], axis=1))
    got = host(F.interpolate(dev(a), scale_factor=2, mode="nearest"))
    assert np.array_equal(got, a.repeat(2, axis=2).repeat(2, axis=3))


@pytest.mark.parametrize("dt", ["float16", "float32"])
@pytest.mark.parametrize("shape,scale", [((2, 640, 32, 32), 2), ((2, 1280, 8, 8), 2), ((1, 3, 5, 12), 2),
                                         ((2, 4, 6, 8), 3), ((1, 2, 3, 5), 2)])
def test_upsample_nearest_rows(dt, shape, scale):
    """Nearest upsampling is a copy: bit-exact against numpy's repeat, at the SD decoder shapes
    (2x, width a multiple of 4: the vectorised row kernel) and off them (odd widths, 3x)."""
    a = Gen(sum(shape) + scale).randn(shape, dt)
    got = host(F.interpolate(dev(a), scale_factor=scale, mode="nearest"))
    assert np.array_equal(got, a.repeat(scale, axis=2).repeat(scale, axis=3))


def test_graph_capture_replay_matches_eager():
    g = Gen(111)
    x = dev(g.randn((2, 32, 8, 8), "float16"))
    w = dev(g.randn((32, 32, 3, 3), "float16", 0.05))
    gamma = dev(g.randn((32,), "float16"))
    beta = dev(g.randn((32,), "float16"))

    def step():
        h = F.group_norm_silu(x, 8, gamma, beta)
        return F.conv2d_residual(h, w, None, x, padding=1)

    eager = host(step())
    step()  # warm the allocator cache so capture reuses blocks
    graph = mt.cuda.CUDAGraph()
    graph.capture_begin()
    out = step()
    graph.capture_end()
    for _ in range(3):
        graph.replay()
        mt.cuda.synchronize()
        assert np.array_equal(host(out), eager)
        _ = host(step())  # eager work between replays
    graph.reset()
