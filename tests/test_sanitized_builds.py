"""AddressSanitizer + UndefinedBehaviorSanitizer builds of the CPU-side code.

* The oracle (oracle/oracle.c) and the product's host generator (mtorch_amd/csrc/rng.cpp) are
  compiled with -fsanitize=address,undefined -fno-sanitize-recover=all together with
  tests/sanitize_driver.cpp, which calls every oracle function and every generator entry point
  over ragged, empty and edge-case shapes with exactly sized buffers, and then run: any
  out-of-bounds access, overflow or invalid shift aborts the run.
* The C++ adaptor that the reference core would call (mtorch_amd/hook/mtorch_hip.cpp) is compiled
  with the same instrumentation against the reference's tensor.h (it cannot be linked: the
  reference core does not build on Linux), which checks that it is sanitizer-clean at compile
  time; skipped where the reference tree is absent.

CPU only; a few seconds."""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]

needs_gcc = pytest.mark.skipif(shutil.which("gcc") is None or shutil.which("g++") is None, reason="needs gcc/g++")


@needs_gcc
def test_oracle_and_generator_under_asan_ubsan(tmp_path):
    oracle_o = str(tmp_path / "oracle.o")
    rng_o = str(tmp_path / "rng.o")
    exe = str(tmp_path / "sanitize_driver")
    subprocess.run(["gcc", "-std=c11", "-ffp-contract=off", *SAN, "-c", os.path.join(ROOT, "oracle", "oracle.c"),
                    "-o", oracle_o], check=True)
    subprocess.run(["g++", "-std=c++17", "-ffp-contract=off", *SAN, "-c",
                    os.path.join(ROOT, "mtorch_amd", "csrc", "rng.cpp"), "-o", rng_o], check=True)
    subprocess.run(["g++", "-std=c++17", *SAN, os.path.join(ROOT, "tests", "sanitize_driver.cpp"), oracle_o, rng_o,
                    "-o", exe, "-lm"], check=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=600, env=env)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-6000:])
    assert "clean" in r.stdout
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-6000:]


TENSOR_H = "/root/reference/cpp/mtorch/core/tensor.h"


@needs_gcc
@pytest.mark.skipif(not os.path.exists(TENSOR_H), reason="needs the reference tree's tensor.h")
def test_hook_adaptor_compiles_under_asan_ubsan(tmp_path):
    hook = os.path.join(ROOT, "mtorch_amd", "hook")
    r = subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-fPIC", *SAN, "-c", "-I",
                        "/root/reference/cpp", "-I", os.path.join(ROOT, "include"), "-I", hook,
                        os.path.join(hook, "mtorch_hip.cpp"), "-o", str(tmp_path / "mtorch_hip.o")],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
