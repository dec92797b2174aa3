"""mtorch.save / mtorch.load in the reference's file format (mtorch/__init__.py:6101-6160).

A file is a pickle (protocol 2 by default) of plain Python values: each Tensor becomes
``{"__mtorch_tensor__": True, "data": t.tolist(), "dtype": "<name>", "requires_grad": b}``, an
OrderedDict becomes ``{"__mtorch_ordered_dict__": True, "items": [(key, value), ...]}``, a tuple
``{"__mtorch_tuple__": True, "items": [...]}``; dicts and lists are walked, other values kept.
Files written by the reference load here and the other way round.  Device tensors are read back
to the host for ``tolist`` and re-uploaded on load when ``map_location`` names a GPU.

One deliberate difference: unless the caller passes its own ``pickle_module``, ``load`` uses an
unpickler that resolves only the constructors of built-in values (set, complex, bytes).  The
reference's files hold only built-in containers and scalars, so they load unchanged, while a file
that would import or call anything else is refused.
"""

from __future__ import annotations

import pickle
from collections import OrderedDict

from . import _tensor as T

_DTYPES = {"float16": T.float16, "half": T.float16, "float32": T.float32, "float": T.float32,
           "float64": T.float64, "double": T.float64, "int32": T.int32, "int64": T.int64, "long": T.int64,
           "bool": T.bool_}


def _dtype_from_name(name) -> T.dtype:
    """The reference looks its stored dtype string up among its module globals, defaulting to
    float32 (mtorch/__init__.py:6121-6123); a "mtorch." or "torch." prefix is accepted too."""
    key = str(name).rsplit(".", 1)[-1]
    return _DTYPES.get(key, T.float32)


def _serialize(value):
    if isinstance(value, T.Tensor):
        return {"__mtorch_tensor__": True, "data": value.tolist(), "dtype": value.dtype.name,
                "requires_grad": bool(value.requires_grad)}
    if isinstance(value, OrderedDict):
        return {"__mtorch_ordered_dict__": True, "items": [(k, _serialize(v)) for k, v in value.items()]}
    if isinstance(value, dict):
        return {k: _serialize(v) for k, v in value.items()}
    if isinstance(value, tuple):
        return {"__mtorch_tuple__": True, "items": [_serialize(v) for v in value]}
    if isinstance(value, list):
        return [_serialize(v) for v in value]
    return value


def _deserialize(value, map_location):
    if isinstance(value, dict) and value.get("__mtorch_tensor__"):
        return T.tensor(value["data"], dtype=_dtype_from_name(value["dtype"]),
                        requires_grad=bool(value["requires_grad"]), device=map_location or "cpu")
    if isinstance(value, dict) and value.get("__mtorch_ordered_dict__"):
        return OrderedDict((k, _deserialize(v, map_location)) for k, v in value["items"])
    if isinstance(value, dict) and value.get("__mtorch_tuple__"):
        return tuple(_deserialize(v, map_location) for v in value["items"])
    if isinstance(value, dict):
        return {k: _deserialize(v, map_location) for k, v in value.items()}
    if isinstance(value, list):
        return [_deserialize(v, map_location) for v in value]
    return value


def _latin1_bytes(text, encoding="latin1"):
    """What protocol-2 pickles call (as _codecs.encode) to rebuild a bytes value."""
    if encoding not in ("latin1", "latin-1"):
        raise pickle.UnpicklingError(f"mtorch_amd.load: unexpected bytes encoding {encoding!r}")
    return text.encode("latin1")


# Constructors that protocol-2 pickles of built-in values name (sets, complex numbers, bytes).
_PLAIN_GLOBALS = {("builtins", "set"): set, ("builtins", "frozenset"): frozenset,
                  ("builtins", "complex"): complex, ("builtins", "bytearray"): bytearray,
                  ("_codecs", "encode"): _latin1_bytes}


class _PlainUnpickler(pickle.Unpickler):
    """Unpickler for payloads of built-in containers and scalars only."""

    def find_class(self, module, name):
        key = ("builtins" if module == "__builtin__" else module, name)  # protocol 2 writes Python 2 names
        if key in _PLAIN_GLOBALS:
            return _PLAIN_GLOBALS[key]
        raise pickle.UnpicklingError(
            f"mtorch_amd.load refuses to resolve global {module}.{name}: the file holds more than tensors and "
            "built-in containers (pass pickle_module=pickle to load it with the standard unpickler)")


class _PlainPickleModule:
    @staticmethod
    def load(f, **kwargs):
        return _PlainUnpickler(f, **kwargs).load()


def save(obj, f, pickle_module=pickle, pickle_protocol=2, **pickle_save_args):
    """mtorch.save (mtorch/__init__.py:6135-6142)."""
    payload = _serialize(obj)
    if hasattr(f, "write"):
        pickle_module.dump(payload, f, protocol=pickle_protocol, **pickle_save_args)
        return None
    with open(f, "wb") as handle:
        pickle_module.dump(payload, handle, protocol=pickle_protocol, **pickle_save_args)
    return None


def load(f, map_location=None, pickle_module=None, **pickle_load_args):
    """mtorch.load (mtorch/__init__.py:6145-6151); ``map_location`` is a device (or its name)."""
    pm = _PlainPickleModule if pickle_module is None else pickle_module
    if hasattr(f, "read"):
        payload = pm.load(f, **pickle_load_args)
    else:
        with open(f, "rb") as handle:
            payload = pm.load(handle, **pickle_load_args)
    return _deserialize(payload, map_location)
