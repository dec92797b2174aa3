"""Host-side checks (no GPU) for the composed-attention and lifecycle surface: the save/load file
format (mtorch/__init__.py:6101-6151), its unpickler, MultiheadAttention's deterministic
initialisation (mtorch/__init__.py:4297-4385) and the argument checks of einsum and masked_fill
that run before any device work."""

import io
import pickle
from collections import OrderedDict

import numpy as np
import pytest

import mtorch_amd as mt


def test_save_writes_the_reference_payload():
    """The payload the reference writes for this object, spelled out from its format: tensors as
    {"__mtorch_tensor__", "data", "dtype", "requires_grad"}, OrderedDict and tuple markers."""
    t = mt.tensor([[1.5, -2.0], [0.25, 3.0]], dtype=mt.float16)
    b = mt.tensor([True, False])
    obj = OrderedDict([("w", t), ("meta", (b, 7, "x"))])
    buf = io.BytesIO()
    mt.save(obj, buf)
    payload = pickle.loads(buf.getvalue())
    assert payload == {
        "__mtorch_ordered_dict__": True,
        "items": [
            ("w", {"__mtorch_tensor__": True, "data": [[1.5, -2.0], [0.25, 3.0]], "dtype": "float16",
                   "requires_grad": False}),
            ("meta", {"__mtorch_tuple__": True, "items": [
                {"__mtorch_tensor__": True, "data": [True, False], "dtype": "bool", "requires_grad": False}, 7, "x"]}),
        ],
    }
    assert buf.getvalue()[:2] == b"\x80\x02"  # pickle protocol 2


def test_load_reads_a_reference_payload():
    payload = {"a": {"__mtorch_tensor__": True, "data": [0.1, -65504.0, 1e-8], "dtype": "float16",
                     "requires_grad": True},
               "b": {"__mtorch_tensor__": True, "data": [[1, 2], [3, 4]], "dtype": "int64", "requires_grad": False},
               "c": {"__mtorch_tensor__": True, "data": 2.5, "dtype": "unknown_dtype", "requires_grad": False},
               "d": {"__mtorch_tuple__": True, "items": [1, [2, {"__mtorch_ordered_dict__": True, "items": [("k", 3)]}]]}}
    out = mt.load(io.BytesIO(pickle.dumps(payload, protocol=2)))
    a = out["a"]
    assert a.dtype is mt.float16 and a.requires_grad and list(a.shape) == [3]
    # fp16 storage is float_to_half_bits((float)value): 0.1 -> 0x2e66, -65504 -> 0xfbff, 1e-8 -> 0
    assert a.half_bits().tolist() == [0x2E66, 0xFBFF, 0x0000]
    assert out["b"].dtype is mt.int64 and out["b"].tolist() == [[1, 2], [3, 4]]
    assert out["c"].dtype is mt.float32 and out["c"].dim() == 0 and out["c"].item() == 2.5  # unknown -> float32
    assert out["d"] == (1, [2, OrderedDict([("k", 3)])])


@pytest.mark.parametrize("dt", ["float16", "float32", "float64", "int32", "int64", "bool"])
def test_save_load_roundtrip_host(dt, tmp_path):
    rng = np.random.default_rng(3)
    if dt == "bool":
        a = rng.random((3, 4)) < 0.5
    elif dt.startswith("int"):
        a = rng.integers(-100, 100, (3, 4)).astype(dt)
    else:
        a = rng.standard_normal((3, 4)).astype(np.float32 if dt == "float16" else dt)
    t = mt.tensor(a, dtype=getattr(mt, dt))
    p = tmp_path / "t.pt"
    mt.save([t, {"t": t}], str(p))
    back = mt.load(str(p))
    for x in (back[0], back[1]["t"]):
        assert x.dtype is t.dtype and list(x.shape) == [3, 4]
        if dt == "float16":
            assert np.array_equal(x.half_bits(), t.half_bits())
        else:
            assert np.array_equal(x.numpy(), t.numpy())


def test_load_refuses_pickled_code():
    class Payload:
        def __reduce__(self):
            return (print, ("side effect",))

    data = pickle.dumps({"x": Payload()}, protocol=2)
    with pytest.raises(pickle.UnpicklingError, match="refuses"):
        mt.load(io.BytesIO(data))
    # built-in values that protocol 2 writes through constructors still load
    plain = {"s": {1, 2}, "f": frozenset([3]), "c": 1 + 2j, "b": b"\x00\xff", "ba": bytearray(b"xy")}
    assert mt.load(io.BytesIO(pickle.dumps(plain, protocol=2))) == plain
    # an explicit pickle module is the caller's choice, as in the reference
    assert mt.load(io.BytesIO(pickle.dumps({"k": 1}, protocol=2)), pickle_module=pickle) == {"k": 1}


def test_mha_default_initialisation():
    """_initial_weight(row, col, width) = ((row*width + col) % (2*span+1) - span) / span^2 with
    span = width (mtorch/__init__.py:4383-4385); values worked out by hand for embed_dim 4."""
    m = mt.nn.MultiheadAttention(4, 2)
    w = m.in_proj_weight.numpy()
    assert w.shape == (12, 4)
    # span 4, modulus 9: row 0 -> -4,-3,-2,-1; row 1 -> 0,1,2,3; row 2 -> 4,-4,-3,-2 (index 8, 0, 1, 2)
    assert w[0].tolist() == [-0.25, -0.1875, -0.125, -0.0625]
    assert w[1].tolist() == [0.0, 0.0625, 0.125, 0.1875]
    assert w[2].tolist() == [0.25, -0.25, -0.1875, -0.125]
    assert m.in_proj_bias.numpy().tolist() == [0.0] * 12
    assert m.out_proj.weight.numpy()[0].tolist() == [-0.25, -0.1875, -0.125, -0.0625]
    m = mt.nn.MultiheadAttention(4, 2, kdim=3, vdim=5, add_bias_kv=True)
    assert m.in_proj_weight is None
    assert [list(m.q_proj_weight.shape), list(m.k_proj_weight.shape), list(m.v_proj_weight.shape)] == [[4, 4], [4, 3], [4, 5]]
    # kdim 3: span 3, modulus 7: row 1 -> indices 3, 4, 5 -> 0, 1/9, 2/9
    assert np.allclose(m.k_proj_weight.numpy()[1], [0.0, 1 / 9, 2 / 9])
    assert list(m.bias_k.shape) == [1, 1, 4] and m.bias_k.numpy().ravel().tolist() == w[0].tolist()
    assert m.bias_v.numpy().ravel().tolist() == w[1].tolist()
    names = [n for n, _ in m.named_parameters()]
    assert names == ["q_proj_weight", "k_proj_weight", "v_proj_weight", "in_proj_bias", "bias_k", "bias_v",
                     "out_proj.weight", "out_proj.bias"]
    with pytest.raises(ValueError, match="divisible"):
        mt.nn.MultiheadAttention(6, 4)


def test_einsum_and_masked_fill_argument_checks():
    x = mt.zeros((3, 3))
    with pytest.raises(ValueError, match="operand count"):
        mt.einsum("ij,jk->ik", x)
    with pytest.raises(ValueError, match="invalid character"):
        mt.einsum("i1,jk->ik", x, x)
    with pytest.raises(NotImplementedError):
        mt.einsum("ii->i", x)
    with pytest.raises(TypeError):
        mt.einsum(3, x)
    with pytest.raises(RuntimeError, match="not implemented for device 'cpu'"):
        mt.einsum("ij,jk->ik", x, x)  # host tensors are staging only; the operators run on the GPU
    with pytest.raises(ValueError, match="bool"):
        x.masked_fill(mt.zeros((3, 3)), 1.0)
    with pytest.raises(ValueError, match="broadcastable"):
        x.masked_fill(mt.ones((2, 3, 3), dtype=mt.bool), 1.0)


def test_copy_into_expanded_host_destination_last_write_wins():
    """Tensor::copy_from writes every index in row-major order (tensor.cpp:8335-8338): along a
    zero-stride (expanded) destination dim the last index's value stays.  Host tensors follow
    the same rule as device ones."""
    base = mt.from_numpy(np.zeros((3, 1, 5), np.float32))
    src = np.arange(60, dtype=np.float32).reshape(3, 4, 5)
    base.expand(3, 4, 5).copy_(mt.from_numpy(src))
    assert np.array_equal(base.numpy(), src[:, 3:4, :])
    col = mt.from_numpy(np.zeros((4, 1), np.float32))
    col.expand(4, 6)[:, :] = mt.from_numpy(np.arange(24, dtype=np.float32).reshape(4, 6))
    assert np.array_equal(col.numpy()[:, 0], np.arange(24, dtype=np.float32).reshape(4, 6)[:, 5])
