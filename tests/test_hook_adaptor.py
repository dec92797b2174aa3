"""The C++ adaptor that mtorch's core calls on a GPU tensor (mtorch_amd/hook/mtorch_hip.cpp), compiled
against the reference's own tensor.h and this repository's include/mthip.h.

Compilation only: the reference core (tensor.cpp) does not build on Linux, so the adaptor is not
linked or run here.  The checks are that it compiles warning-free, that every libmthip symbol it
calls is declared in include/mthip.h, and that each mirrored op has exactly the public op's
signature (so the dispatch hook in tensor.cpp can forward its arguments unchanged).  Skipped when
the reference tree is absent (the GPU box)."""

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_CPP = "/root/reference/cpp"
TENSOR_H = os.path.join(REF_CPP, "mtorch", "core", "tensor.h")
HOOK = os.path.join(ROOT, "mtorch_amd", "hook")
SRC = os.path.join(HOOK, "mtorch_hip.cpp")

pytestmark = pytest.mark.skipif(not os.path.exists(TENSOR_H) or shutil.which("g++") is None,
                                reason="needs the reference tree's tensor.h and g++")

# ops whose hip:: entry must have the public op's exact type (tensor.h declarations)
MIRRORED = ["to", "binary_tensor_tensor", "binary_tensor_scalar", "binary_scalar_tensor", "silu", "gelu", "linear",
            "matmul", "bmm", "addmm", "baddbmm", "conv2d", "scaled_dot_product_attention", "group_norm",
            "layer_norm", "softmax"]


def compile_cmd(src, out):
    return ["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-O1", "-fPIC", "-c", "-I", REF_CPP, "-I",
            os.path.join(ROOT, "include"), "-I", HOOK, src, "-o", out]


def header_functions():
    text = open(os.path.join(ROOT, "include", "mthip.h")).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return set(re.findall(r"\b(mthip_\w+)\s*\(", text))


def test_adaptor_compiles_against_reference_header(tmp_path):
    obj = str(tmp_path / "mtorch_hip.o")
    r = subprocess.run(compile_cmd(SRC, obj), capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    nm = subprocess.run(["nm", "-u", obj], capture_output=True, text=True, check=True).stdout
    called = set(re.findall(r"\b(mthip_\w+)\b", nm))
    assert called, "the adaptor calls no libmthip entry point"
    assert called <= header_functions(), sorted(called - header_functions())
    for needed in ["mthip_linear", "mthip_gemm", "mthip_conv2d_prepacked", "mthip_sdpa", "mthip_group_norm",
                   "mthip_layer_norm", "mthip_softmax_lastdim", "mthip_unary", "mthip_binary", "mthip_cast",
                   "mthip_memcpy_h2d", "mthip_memcpy_d2h"]:
        assert needed in called, needed


def test_adaptor_mirrors_public_signatures(tmp_path):
    lines = ['#include <type_traits>', '#include "mtorch_hip.h"']
    for op in MIRRORED:
        lines.append(f"static_assert(std::is_same_v<decltype(&mtorch::{op}), decltype(&mtorch::hip::{op})>, "
                     f'"hip::{op} differs from mtorch::{op}");')
    src = tmp_path / "signatures.cpp"
    src.write_text("\n".join(lines) + "\n")
    r = subprocess.run(compile_cmd(str(src), str(tmp_path / "signatures.o")), capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
