"""Writes the golden fixtures under tests/golden/ (run in the build container, where torch-CPU
2.10 -- the reference's own test oracle -- is installed).  The fixtures are data only: inputs
from the reference tests' literal values / closed-form generators and expected outputs.

    python tests/golden/make_golden.py
"""

import json
import os

import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

import closed_form  # noqa: E402


def fp16_rounding_boundaries():
    # Inputs of tests/compat/test_tensor_ops.py:1308-1320 (reference); expected = torch's fp16
    # cast, which the reference test compares against (ties here round the same either way).
    import torch

    values = [3.99853515625, 3.9990234375, 7.99853515625, 7.9990234375, -7.99853515625, float("inf")]
    expected = torch.tensor(values, dtype=torch.float32).to(torch.float16).to(torch.float32).tolist()
    with open(os.path.join(HERE, "fp16_rounding_boundaries.json"), "w") as fh:
        json.dump({"source": "reference tests/compat/test_tensor_ops.py:1308-1320", "input": values,
                   "expected": expected}, fh, indent=1)


def sd_group_norm():
    # Expected output for the closed-form inputs of tests/compat/test_tensor_ops.py:2161-2177
    # (reference), from torch in float64, rounded to float32 (tolerance-level fixture).
    import torch

    hidden, w, b = closed_form.sd_group_norm_inputs()
    out = torch.nn.functional.group_norm(torch.from_numpy(hidden).double(), 32, torch.from_numpy(w).double(),
                                         torch.from_numpy(b).double(), eps=1e-5).float().numpy()
    np.savez_compressed(os.path.join(HERE, "sd_group_norm_1x320x16x16.npz"), y=out)


def sd_cross_attention():
    # Expected attention output for the closed-form scenario of
    # tests/compat/test_tensor_ops.py:2105-2158 (reference), from torch in float64.
    import torch

    c = closed_form.sd_cross_attention_inputs()
    batch, qt, kt, ch, heads = 2, 64, 77, 320, 8
    hd = ch // heads
    t = lambda a: torch.from_numpy(a).double()  # noqa: E731
    F = torch.nn.functional
    q = F.linear(t(c["hidden"]), t(c["qw"]), t(c["bias"])).reshape(batch, qt, heads, hd).transpose(1, 2)
    k = F.linear(t(c["enc"]), t(c["kw"]), t(c["bias"])).reshape(batch, kt, heads, hd).transpose(1, 2)
    v = F.linear(t(c["enc"]), t(c["vw"]), t(c["bias"])).reshape(batch, kt, heads, hd).transpose(1, 2)
    q = q.reshape(batch * heads, qt, hd)
    k = k.reshape(batch * heads, kt, hd)
    v = v.reshape(batch * heads, kt, hd)
    att = F.scaled_dot_product_attention(q, k, v, attn_mask=torch.from_numpy(c["mask"]), scale=0.125)
    np.savez_compressed(os.path.join(HERE, "sd_cross_attention_2x64x77x320.npz"), attended=att.float().numpy())


if __name__ == "__main__":
    fp16_rounding_boundaries()
    sd_group_norm()
    sd_cross_attention()
    print("golden fixtures written to", HERE)
