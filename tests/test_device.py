"""Device-string parsing and the device surface, as the reference's tests/test_device.py:8-18
pins it, plus the GPU type this backend adds.  Runs on the CPU (no device allocation)."""

import pytest

import mtorch_amd as mt


def test_cpu_device_keyword_creates_cpu_tensor():
    tensor = mt.zeros((2, 3), dtype=mt.float32, device=mt.device("cpu"))
    assert tensor.device == "cpu"


def test_metal_device_is_parsed_but_storage_is_not_implemented():
    assert str(mt.device("metal")) == "mps"
    with pytest.raises(NotImplementedError):
        mt.zeros((1,), device=mt.device("mps"))
    with pytest.raises(NotImplementedError):
        mt.randn(2, device="mps")
    with pytest.raises(NotImplementedError):
        mt.zeros(3).to("mps")


def test_device_strings_and_indices():
    assert repr(mt.device("mps:1")) == "device(type='mps', index=1)"
    assert str(mt.device("hip")) == "cuda"
    assert str(mt.device("cuda:0")) == "cuda:0"
    assert mt.device("cuda") == "cuda:0"
    assert str(mt.device(0)) == "cuda:0"
    with pytest.raises(NotImplementedError):
        mt.device("xla")
