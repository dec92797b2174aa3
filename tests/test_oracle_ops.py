"""Pins the oracle's operator restatements against independent evaluations.

The reference's Linux path accumulates in double and rounds once (linear, matmul, addmm,
conv2d, SDPA), so float64 evaluations by numpy/torch-CPU pin those to within one final
rounding.  GELU/SiLU/softmax are pinned against closed forms with error bounds tight enough
that a wrong coefficient, sign or operand fails; the normalisations against torch float64 and
against the reference's SD scenario fixtures (tests/golden)."""

import math
import os
import sys

import numpy as np
import pytest
import torch

HERE = os.path.dirname(__file__)
sys.path.insert(0, os.path.join(HERE, "golden"))
import closed_form  # noqa: E402

F = torch.nn.functional


def ulps32(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


def ulps16(orc, a_bits, b_bits):
    a = a_bits.astype(np.int64)
    b = b_bits.astype(np.int64)
    a = np.where(a & 0x8000, -(a & 0x7FFF), a)
    b = np.where(b & 0x8000, -(b & 0x7FFF), b)
    return np.abs(a - b)


@pytest.fixture
def rng():
    return np.random.default_rng(1234)


# ------------------------------------------------------------------ contractions


def test_linear_fp32_is_double_sum_rounded_once(orc, rng):
    x = rng.standard_normal((33, 70)).astype(np.float32)
    w = rng.standard_normal((21, 70)).astype(np.float32)
    b = rng.standard_normal(21).astype(np.float32)
    got = orc.linear(x, w, b)
    ref = (x.astype(np.float64) @ w.astype(np.float64).T + b).astype(np.float32)
    assert ulps32(got, ref).max() <= 1


def test_linear_fp16_rounds_double_then_half(orc, rng):
    xh = orc.f2h(rng.standard_normal((17, 40)).astype(np.float32))
    wh = orc.f2h(rng.standard_normal((9, 40)).astype(np.float32) * 0.2)
    got = orc.linear(xh, wh)
    ref = orc.f2h((orc.h2f(xh).astype(np.float64) @ orc.h2f(wh).astype(np.float64).T).astype(np.float32))
    assert ulps16(orc, got, ref).max() <= 1


def test_matmul_batched_and_broadcast(orc, rng):
    a = rng.standard_normal((3, 5, 7)).astype(np.float32)
    b = rng.standard_normal((1, 7, 4)).astype(np.float32)
    got = orc.matmul(a, b)
    ref = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
    assert ulps32(got, ref).max() <= 1


def test_addmm_rounds_beta_term_first(orc, rng):
    inp = rng.standard_normal(6).astype(np.float32)
    m1 = rng.standard_normal((4, 5)).astype(np.float32)
    m2 = rng.standard_normal((5, 6)).astype(np.float32)
    got = orc.addmm(inp, m1, m2, beta=0.3, alpha=1.7)
    base = (0.3 * np.broadcast_to(inp, (4, 6)).astype(np.float64)).astype(np.float32)
    ref = (base.astype(np.float64) + 1.7 * (m1.astype(np.float64) @ m2.astype(np.float64))).astype(np.float32)
    assert ulps32(got, ref).max() <= 1


@pytest.mark.parametrize("dt", ["float32", "float16"])
def test_addmm_non_finite_beta0_alpha0(orc, rng, dt):
    """The Linux path stores beta*input even at beta = 0 (tensor.cpp:25253-25258), so an inf or
    NaN input gives NaN there (IEEE 0*inf), and skips the product at alpha = 0 (:25320), so a NaN
    or inf in mat1/mat2 never reaches the output, which is then beta*input narrowed once."""
    cast = (lambda a: orc.f2h(a)) if dt == "float16" else (lambda a: a)
    back = (lambda a: orc.h2f(a)) if dt == "float16" else (lambda a: a)
    inp = rng.standard_normal((4, 6)).astype(np.float32)
    inp[1, 2], inp[3, 0] = np.inf, np.nan
    m1 = rng.standard_normal((4, 5)).astype(np.float32)
    m2 = rng.standard_normal((5, 6)).astype(np.float32)
    inp, m1, m2 = cast(inp), cast(m1), cast(m2)
    got = back(orc.addmm(inp, m1, m2, beta=0.0, alpha=1.0))
    nonfinite = ~np.isfinite(back(inp))
    assert np.array_equal(np.isnan(got), nonfinite)
    prod = back(m1).astype(np.float64) @ back(m2).astype(np.float64)
    assert np.allclose(got[~nonfinite], prod[~nonfinite], rtol=2e-3 if dt == "float16" else 1e-6, atol=1e-3)
    # alpha = 0 with NaN/inf operands: exactly beta*input, narrowed once
    m1b = back(m1).copy()
    m1b[0, 0], m1b[2, 4] = np.nan, np.inf
    got = back(orc.addmm(inp, cast(m1b), m2, beta=0.5, alpha=0.0))
    ref = back(cast((0.5 * back(inp).astype(np.float64)).astype(np.float32)))
    assert np.array_equal(got, ref, equal_nan=True)


@pytest.mark.parametrize("cfg", [
    dict(C=5, O=7, H=9, W=8, k=3, stride=1, padding=1, dilation=1, groups=1),
    dict(C=6, O=4, H=10, W=7, k=3, stride=2, padding=1, dilation=1, groups=1),
    dict(C=4, O=6, H=9, W=9, k=3, stride=1, padding=2, dilation=2, groups=2),
    dict(C=8, O=5, H=6, W=5, k=1, stride=1, padding=0, dilation=1, groups=1),
])
def test_conv2d_fp32_matches_float64(orc, rng, cfg):
    x = rng.standard_normal((2, cfg["C"], cfg["H"], cfg["W"])).astype(np.float32)
    w = rng.standard_normal((cfg["O"], cfg["C"] // cfg["groups"], cfg["k"], cfg["k"])).astype(np.float32)
    b = rng.standard_normal(cfg["O"]).astype(np.float32)
    kw = dict(stride=cfg["stride"], padding=cfg["padding"], dilation=cfg["dilation"], groups=cfg["groups"])
    got = orc.conv2d(x, w, b, **kw)
    ref = F.conv2d(torch.from_numpy(x).double(), torch.from_numpy(w).double(), torch.from_numpy(b).double(), **kw)
    assert ulps32(got, ref.float().numpy()).max() <= 1


@pytest.mark.parametrize("O,k", [(8, 3), (3, 3), (6, 1)])
def test_conv2d_fp16_paths(orc, rng, O, k):
    """3x3 with O > 4 widens to fp32 (double accumulate); O <= 4 and 1x1 accumulate in float."""
    x = orc.f2h(rng.standard_normal((1, 12, 7, 6)).astype(np.float32))
    w = orc.f2h((rng.standard_normal((O, 12, k, k)) * 0.2).astype(np.float32))
    b = orc.f2h(rng.standard_normal(O).astype(np.float32))
    got = orc.conv2d(x, w, b, padding=k // 2)
    ref = F.conv2d(torch.from_numpy(orc.h2f(x)).double(), torch.from_numpy(orc.h2f(w)).double(),
                   torch.from_numpy(orc.h2f(b)).double(), padding=k // 2).float().numpy()
    assert ulps16(orc, got, orc.f2h(ref)).max() <= 1


# ------------------------------------------------------------------ attention


def _torch_sdpa(q, k, v, mask=None, causal=False, scale=None):
    m = None if mask is None else torch.from_numpy(mask if mask.dtype == np.bool_ else mask.astype(np.float64))
    return F.scaled_dot_product_attention(torch.from_numpy(q).double(), torch.from_numpy(k).double(),
                                          torch.from_numpy(v).double(), attn_mask=m, is_causal=causal,
                                          scale=scale).numpy()


@pytest.mark.parametrize("Lq,Lk,E,Ev", [(9, 13, 8, 6), (16, 77, 40, 40), (5, 5, 3, 7)])
def test_sdpa_fp32_matches_float64(orc, rng, Lq, Lk, E, Ev):
    q = rng.standard_normal((2, 3, Lq, E)).astype(np.float32)
    k = rng.standard_normal((2, 3, Lk, E)).astype(np.float32)
    v = rng.standard_normal((2, 3, Lk, Ev)).astype(np.float32)
    got = orc.sdpa(q, k, v)
    ref = _torch_sdpa(q, k, v).astype(np.float32)
    assert ulps32(got, ref).max() <= 2


def test_sdpa_masks_and_causal(orc, rng):
    q = rng.standard_normal((2, 6, 8)).astype(np.float32)
    k = rng.standard_normal((2, 10, 8)).astype(np.float32)
    v = rng.standard_normal((2, 10, 5)).astype(np.float32)
    bmask = rng.random((2, 6, 10)) > 0.3
    bmask[:, :, 0] = True
    fmask = rng.standard_normal((1, 6, 10)).astype(np.float32)
    tril = np.tril(np.ones((6, 10), bool))
    for mask, causal in [(bmask, False), (fmask, False), (None, True), (bmask, True)]:
        got = orc.sdpa(q, k, v, mask, causal, 0.3)
        if mask is not None and causal:  # torch takes one or the other: combine them
            ref = _torch_sdpa(q, k, v, mask & tril, False, 0.3).astype(np.float32)
        else:
            ref = _torch_sdpa(q, k, v, mask, causal, 0.3).astype(np.float32)
        assert np.allclose(got, ref, rtol=1e-6, atol=1e-6)
    # a masked key gets exactly zero weight: changing its value changes nothing
    v2 = v.copy()
    v2[:, 9, :] = 1e6
    m = np.ones((2, 6, 10), bool)
    m[:, :, 9] = False
    assert np.array_equal(orc.sdpa(q, k, v, m), orc.sdpa(q, k, v2, m))
    # a fully masked row is NaN (softmax of all -inf), as in the reference
    m[:, 2, :] = False
    out = orc.sdpa(q, k, v, m)
    assert np.isnan(out[:, 2]).all() and not np.isnan(out[:, 1]).any()


@pytest.mark.parametrize("dt", ["float32", "float16"])
def test_sdpa_explicit_scale_closed_forms(orc, rng, dt):
    """An explicit scale multiplies the scores as given (tensor.cpp:31019, 31182), zero and
    negative values included; scale=None is 1/sqrt(E).  Pinned by what the mathematics fixes:
    scale 0 leaves softmax(mask) -- the mean of V over the unmasked keys for a bool mask, the
    mask's own softmax weights for an additive one; a negative scale is the positive one on -q
    (negation is exact, so bit for bit); None equals an explicit 1/sqrt(E) bit for bit."""
    cast = (lambda a: orc.f2h(a)) if dt == "float16" else (lambda a: a)
    back = (lambda a: orc.h2f(a)) if dt == "float16" else (lambda a: a)
    q = cast(rng.standard_normal((2, 7, 12)).astype(np.float32))
    k = cast(rng.standard_normal((2, 11, 12)).astype(np.float32))
    v = cast(rng.standard_normal((2, 11, 6)).astype(np.float32))
    vf = back(v).astype(np.float64)
    tol = 1e-6 if dt == "float32" else 1e-3
    # scale 0, no mask: the mean of V over all keys, for every query
    got = back(orc.sdpa(q, k, v, scale=0.0)).astype(np.float64)
    assert np.allclose(got, np.broadcast_to(vf.mean(1, keepdims=True), got.shape), rtol=tol, atol=tol)
    # scale 0, bool mask: the mean over the unmasked keys
    bmask = rng.random((2, 7, 11)) > 0.5
    bmask[:, :, 3] = True
    got = back(orc.sdpa(q, k, v, bmask, scale=0.0)).astype(np.float64)
    ref = np.einsum("pqk,pke->pqe", bmask / bmask.sum(-1, keepdims=True), vf)
    assert np.allclose(got, ref, rtol=tol, atol=tol)
    # scale 0, additive mask: softmax of the mask alone
    fmask = (rng.standard_normal((2, 7, 11)) * 3).astype(np.float32)
    w = np.exp(fmask - fmask.max(-1, keepdims=True))
    w = w / w.sum(-1, keepdims=True)
    got = back(orc.sdpa(q, k, v, fmask, scale=0.0)).astype(np.float64)
    assert np.allclose(got, np.einsum("pqk,pke->pqe", w, vf), rtol=tol, atol=tol)
    # scale 0 with causal: the mean over keys 0..i
    got = back(orc.sdpa(q, k, v, is_causal=True, scale=0.0)).astype(np.float64)
    ref = np.stack([vf[:, : i + 1].mean(1) for i in range(7)], axis=1)
    assert np.allclose(got, ref, rtol=tol, atol=tol)
    # a negative scale is the positive one on -q, bit for bit, with and without masks
    nq = (q ^ np.uint16(0x8000)) if dt == "float16" else -q
    for m in (None, bmask, fmask):
        assert np.array_equal(orc.sdpa(q, k, v, m, scale=-0.125), orc.sdpa(nq, k, v, m, scale=0.125))
    # None is 1/sqrt(E)
    assert np.array_equal(orc.sdpa(q, k, v), orc.sdpa(q, k, v, scale=1.0 / math.sqrt(12)))
    if dt == "float32":  # and against torch in float64 at the non-positive scales
        for s in (0.0, -0.125, -1.5):
            ref = _torch_sdpa(q, k, v, fmask, False, s).astype(np.float32)
            assert np.allclose(orc.sdpa(q, k, v, fmask, scale=s), ref, rtol=1e-6, atol=1e-6), s


def test_sd_cross_attention_fixture(orc):
    """Reference scenario tests/compat/test_tensor_ops.py:2105-2158 through the oracle (fp32)."""
    c = closed_form.sd_cross_attention_inputs()
    exp = np.load(os.path.join(HERE, "golden", "sd_cross_attention_2x64x77x320.npz"))["attended"]
    q = orc.linear(c["hidden"], c["qw"], c["bias"]).reshape(2, 64, 8, 40).transpose(0, 2, 1, 3).reshape(16, 64, 40)
    k = orc.linear(c["enc"], c["kw"], c["bias"]).reshape(2, 77, 8, 40).transpose(0, 2, 1, 3).reshape(16, 77, 40)
    v = orc.linear(c["enc"], c["vw"], c["bias"]).reshape(2, 77, 8, 40).transpose(0, 2, 1, 3).reshape(16, 77, 40)
    got = orc.sdpa(q, k, v, c["mask"], scale=0.125)
    assert np.allclose(got, exp, rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------------ normalisation


def test_group_norm_matches_float64_and_fixture(orc, rng):
    x = rng.standard_normal((2, 8, 5, 6)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(8)).astype(np.float32)
    b = (0.1 * rng.standard_normal(8)).astype(np.float32)
    got = orc.group_norm(x, 4, w, b)
    ref = F.group_norm(torch.from_numpy(x).double(), 4, torch.from_numpy(w).double(), torch.from_numpy(b).double()).numpy()
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-5)
    hidden, gw, gb = closed_form.sd_group_norm_inputs()
    exp = np.load(os.path.join(HERE, "golden", "sd_group_norm_1x320x16x16.npz"))["y"]
    assert np.allclose(orc.group_norm(hidden, 32, gw, gb), exp, rtol=1e-4, atol=1e-4)
    got16 = orc.h2f(orc.group_norm(orc.f2h(hidden), 32, orc.f2h(gw), orc.f2h(gb)))
    assert np.allclose(got16, exp, rtol=3e-3, atol=3e-3)  # the reference test's tolerance


def test_layer_norm_two_pass_fp16_one_pass_fp32(orc, rng):
    x = (rng.standard_normal((7, 96)) * 2 + 3).astype(np.float32)
    w = rng.standard_normal(96).astype(np.float32)
    b = rng.standard_normal(96).astype(np.float32)
    ref = F.layer_norm(torch.from_numpy(x).double(), (96,), torch.from_numpy(w).double(), torch.from_numpy(b).double()).numpy()
    assert np.allclose(orc.layer_norm(x, 96, w, b), ref, rtol=1e-5, atol=2e-5)
    xh = orc.f2h(x)
    refh = F.layer_norm(torch.from_numpy(orc.h2f(xh)).double(), (96,), torch.from_numpy(orc.h2f(orc.f2h(w))).double(),
                        torch.from_numpy(orc.h2f(orc.f2h(b))).double()).numpy()
    assert ulps16(orc, orc.layer_norm(xh, 96, orc.f2h(w), orc.f2h(b)), orc.f2h(refh.astype(np.float32))).max() <= 1


def test_softmax_rows(orc, rng):
    x = rng.standard_normal((4, 3, 50)).astype(np.float32) * 4
    got = orc.softmax_lastdim(x)
    e = np.exp(x.astype(np.float64) - x.max(-1, keepdims=True))
    ref = e / e.sum(-1, keepdims=True)
    assert np.allclose(got, ref, rtol=2e-6, atol=1e-9)
    assert np.allclose(got.sum(-1), 1.0, atol=1e-5)
    got2 = orc.softmax_lastdim(x[0])  # rank 2 divides
    assert np.allclose(got2, ref[0], rtol=2e-6, atol=1e-9)
    h = orc.f2h(x)
    xr = orc.h2f(h).astype(np.float64)
    e = np.exp(xr - xr.max(-1, keepdims=True))
    ref16 = (e / e.sum(-1, keepdims=True)).astype(np.float32)
    assert ulps16(orc, orc.softmax_lastdim(h), orc.f2h(ref16)).max() <= 1


def test_softmax_with_another_output_dtype(orc, rng):
    """The generic path reads the input at its own precision and narrows only the results."""
    # closed form: softmax([a, a + 0.3]) = (1/(1+e^0.3), 1/(1+e^-0.3)); rounding the logits to
    # fp16 first would make both 1000.0 and give (0.5, 0.5)
    got = orc.h2f(orc.softmax_generic(np.array([[1000.0, 1000.3]], np.float32), "float16"))
    d = float(np.float32(1000.3)) - 1000.0
    exp = orc.f2h(np.array([1 / (1 + math.exp(d)), 1 / (1 + math.exp(-d))], np.float32))
    assert np.array_equal(orc.f2h(got[0]), exp)
    x = rng.standard_normal((6, 77)).astype(np.float32) * 5
    e = np.exp(x.astype(np.float64) - x.max(-1, keepdims=True))
    ref = e / e.sum(-1, keepdims=True)
    # e rounded to fp16, then the quotient rounded again: within one fp16 ulp of the exact value
    assert ulps16(orc, orc.softmax_generic(x, "float16"), orc.f2h(ref.astype(np.float32))).max() <= 1
    h = orc.f2h(x)
    xr = orc.h2f(h).astype(np.float64)
    e = np.exp(xr - xr.max(-1, keepdims=True))
    ref = e / e.sum(-1, keepdims=True)
    assert np.allclose(orc.softmax_generic(h, "float32"), ref, rtol=2e-7, atol=1e-12)


# ------------------------------------------------------------------ activations


def test_fast_erf_within_abramowitz_stegun_bound(orc):
    xs = np.linspace(-4, 4, 4001, dtype=np.float32)
    got = np.array([orc.lib().orc_fast_erf_float(float(v)) for v in xs])
    ref = np.array([math.erf(float(v)) for v in xs])
    # A&S 7.1.26 bounds the formula's error by 1.5e-7; evaluating it in float adds up to a few
    # float ulps of 1 - poly*exp(-x^2).  A wrong coefficient or sign costs >= 1e-4.
    assert np.max(np.abs(got - ref)) < 5e-7


def test_gelu_fp32_close_to_erf_gelu(orc):
    xs = np.linspace(-6, 6, 24001, dtype=np.float32)
    got = orc.gelu(xs)
    ref = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in xs.astype(np.float64)])
    assert np.max(np.abs(got - ref)) < 2e-6
    unit = np.abs(xs) <= 1
    assert np.max(np.abs(got[unit] - ref[unit])) < 1e-6  # truncated series region


def test_gelu_fp16_exhaustive_double_erf(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = orc.h2f(h).astype(np.float64)
    finite = np.isfinite(x)
    ref = np.array([0.5 * v * (1 + math.erf(v * 0.70710678118654752440)) for v in x[finite]], dtype=np.float64)
    got = orc.gelu(h)[finite]
    assert np.array_equal(got, orc.f2h(ref.astype(np.float32)))


def test_silu(orc, rng):
    x = (rng.standard_normal(5000) * 5).astype(np.float32)
    ref = x.astype(np.float64) / (1 + np.exp(-x.astype(np.float64)))
    assert ulps32(orc.silu(x), ref.astype(np.float32)).max() <= 2
    h = orc.f2h(x)
    xr = orc.h2f(h).astype(np.float64)
    assert ulps16(orc, orc.silu(h), orc.f2h((xr / (1 + np.exp(-xr))).astype(np.float32))).max() <= 1


def test_binary_fp16_is_float_op_then_half(orc, rng):
    a = orc.f2h(rng.standard_normal(10000).astype(np.float32))
    b = orc.f2h(rng.standard_normal(10000).astype(np.float32))
    fa, fb = orc.h2f(a), orc.h2f(b)
    assert np.array_equal(orc.binary(a, b, "add"), orc.f2h(fa + fb))
    assert np.array_equal(orc.binary(a, b, "mul"), orc.f2h(fa * fb))
