"""The device fp16 narrowings (csrc/common.h f2h_fast / f2h_generic / f2h_nonnan / f2h_rtz_prep)
against mtorch's rounding rule on all 2^32 float patterns, through a C model of the same integer
steps with F16C standing in for the hardware's round-to-nearest-even and round-toward-zero
conversions (f2h_fast_model.c).  CPU only (~60 s)."""

import os
import shutil
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(__file__)


def _has_f16c():
    try:
        with open("/proc/cpuinfo") as fh:
            flags = fh.read()
        return " f16c" in flags and " fma" in flags
    except OSError:
        return False


@pytest.mark.skipif(shutil.which("gcc") is None or not _has_f16c(), reason="needs gcc and an F16C/FMA CPU")
def test_f2h_fast_equals_reference_rounding_on_all_floats():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "f2h_model")
        subprocess.run(["gcc", "-O2", "-mf16c", "-mfma", "-o", exe, os.path.join(HERE, "f2h_fast_model.c")], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout
    assert "fast!=generic 0, reference!=generic 0, nonnan!=generic 0" in out.stdout
