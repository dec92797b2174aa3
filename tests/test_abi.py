"""The C-ABI boundary without a GPU: the library loads, exports exactly what include/mthip.h
declares, the ctypes binding covers every declaration, argument validation fails with a status
and a message before any device work, and the device path refuses to run without the library
(no CPU fallback)."""

import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest

import mtorch_amd as mt
from mtorch_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mthip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    names = re.findall(r"\b(mthip_\w+)\s*\(", text)
    return sorted(set(names))


def exported_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True)
    return {line.split()[-1] for line in out.stdout.splitlines() if " T " in line}


def test_header_declares_the_hot_path_entry_points():
    names = header_functions()
    for needed in ["mthip_linear", "mthip_gemm", "mthip_conv2d", "mthip_conv2d_prepacked", "mthip_sdpa",
                   "mthip_group_norm", "mthip_layer_norm", "mthip_softmax_lastdim", "mthip_unary", "mthip_binary",
                   "mthip_cast", "mthip_malloc", "mthip_memcpy_h2d", "mthip_device_count"]:
        assert needed in names


def test_library_exports_every_declared_symbol():
    missing = set(header_functions()) - exported_symbols()
    assert not missing, f"declared in include/mthip.h but not exported: {sorted(missing)}"


def test_binding_covers_exactly_the_header():
    assert sorted(_lib.declared_symbols()) == header_functions()


def test_library_loads_and_reports_no_device_here():
    L = _lib.lib()
    assert L.mthip_version().decode().startswith("libmthip")
    n = ctypes.c_int(-1)
    assert L.mthip_device_count(ctypes.byref(n)) == 0
    if not os.path.exists("/dev/kfd"):
        assert n.value == 0
        assert mt.cuda.is_available() is False


def test_invalid_arguments_return_status_and_message():
    L = _lib.lib()
    rc = L.mthip_linear(0, 7, None, 4, None, 4, None, None, 4, 2, 2, 4, 0, None, 0)
    assert rc == 1  # MTHIP_ERR_INVALID
    assert "dtype" in L.mthip_last_error().decode()
    with pytest.raises(RuntimeError, match="dtype"):
        _lib.check(rc)
    rc = L.mthip_conv2d(0, 0, None, None, None, None, 1, 4, 8, 8, 4, 3, 3, 0, 1, 1, 1, 1, 1, 1, None)
    assert rc == 1 and "stride" in L.mthip_last_error().decode()
    assert L.mthip_linear(0, 0, None, 4, None, 4, None, None, 4, 2, 2, 4, 9, None, 0) == 1  # unknown activation


def test_packed_conv_weight_size():
    L = _lib.lib()
    assert L.mthip_conv2d_packed_bytes(0, 320, 320, 3, 3) == 320 * 9 * 320 * 2
    assert L.mthip_conv2d_packed_bytes(0, 320, 4, 3, 3) == 320 * 9 * 8 * 2  # channels padded to 8
    assert L.mthip_conv2d_packed_bytes(1, 16, 3, 1, 1) == 16 * 4 * 4
    assert L.mthip_conv2d_packed_bytes(5, 16, 3, 1, 1) == -1


def test_host_generator_matches_oracle_stream():
    import oracle as orc

    L = _lib.lib()
    g = L.mthip_generator_create(1234)
    try:
        out = np.empty(1001, np.float32)
        assert L.mthip_rng_normal(g, 1, out.ctypes.data, out.size, 0.0, 1.0) == 0
        ref = orc.Rng(1234).randn((1001,), "float32", 0.0, 1.0)
        assert np.array_equal(out, ref)
    finally:
        L.mthip_generator_destroy(g)


def test_device_ops_fail_loudly_without_the_library(tmp_path):
    """A fresh interpreter whose binding points at a missing library: creating a device
    tensor raises instead of computing on the CPU."""
    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "from mtorch_amd import _lib\n"
        "_lib.LIB_PATH = %r\n"
        "import mtorch_amd as mt\n"
        "try:\n"
        "    mt.zeros(4).to('cuda')\n"
        "except RuntimeError as e:\n"
        "    print('RAISED', e)\n"
    ) % (ROOT, str(tmp_path / "libmthip.so"))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert "RAISED" in out.stdout and "not built" in out.stdout, out.stdout + out.stderr
