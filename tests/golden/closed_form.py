"""Closed-form inputs of the reference's SD scenario tests (sin/cos of arange), shared by
make_golden.py and the tests so fixtures only need to hold expected outputs."""

import numpy as np


def sd_group_norm_inputs():
    """tests/compat/test_tensor_ops.py:2161-2177 (reference)."""
    base = np.arange(0, 1 * 320 * 16 * 16, dtype=np.float32).reshape(1, 320, 16, 16)
    hidden = (np.sin(base * np.float32(0.013)) * np.float32(0.25)).astype(np.float32)
    w = (1.0 + np.arange(320, dtype=np.float32) * np.float32(0.0007)).astype(np.float32)
    b = (np.arange(320, dtype=np.float32) * np.float32(0.0003) - np.float32(0.04)).astype(np.float32)
    return hidden, w, b


def sd_cross_attention_inputs():
    """tests/compat/test_tensor_ops.py:2105-2158 (reference): 2x64 queries, 77 text tokens,
    320 channels, 8 heads, last 7 tokens masked, scale 0.125."""
    batch, qt, kt, ch = 2, 64, 77, 320
    hb = np.arange(batch * qt * ch, dtype=np.float32).reshape(batch, qt, ch)
    eb = np.arange(batch * kt * ch, dtype=np.float32).reshape(batch, kt, ch)
    hidden = (np.sin(hb * np.float32(0.013)) * np.float32(0.2)).astype(np.float32)
    enc = (np.cos(eb * np.float32(0.011)) * np.float32(0.2)).astype(np.float32)
    wb = np.arange(ch * ch, dtype=np.float32).reshape(ch, ch)
    qw = (np.sin(wb * np.float32(0.007)) / np.float32(64.0)).astype(np.float32)
    kw = (np.cos(wb * np.float32(0.009)) / np.float32(64.0)).astype(np.float32)
    vw = (np.sin(wb * np.float32(0.011)) / np.float32(64.0)).astype(np.float32)
    bias = (np.arange(ch, dtype=np.float32) / np.float32(4096.0) - np.float32(0.03)).astype(np.float32)
    mask = np.ones((2 * 8, 1, kt), dtype=bool)
    mask[:, :, kt - 7:] = False
    return dict(hidden=hidden, enc=enc, qw=qw, kw=kw, vw=vw, bias=bias, mask=mask)
