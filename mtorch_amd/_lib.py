"""ctypes binding of libmthip (include/mthip.h).

The device path has no fallback: if the library is missing every device operation raises
``RuntimeError`` naming the file, instead of silently computing somewhere else.
"""

from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libmthip.so")

# dtype codes (mtorch ScalarType order, tensor.h:13-20)
F16, F32, F64, I32, I64, BOOL = 0, 1, 2, 3, 4, 5

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_dbl = ctypes.c_double
_size = ctypes.c_size_t
_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes)
_SIGNATURES = {
    "mthip_last_error": (ctypes.c_char_p, []),
    "mthip_version": (ctypes.c_char_p, []),
    "mthip_device_count": (_int, [ctypes.POINTER(_int)]),
    "mthip_device_info": (_int, [_int, ctypes.c_char_p, _size, ctypes.POINTER(_int), ctypes.POINTER(_size)]),
    "mthip_malloc": (_int, [_int, _size, ctypes.POINTER(_c_void_p)]),
    "mthip_free": (_int, [_int, _c_void_p]),
    "mthip_empty_cache": (_int, [_int]),
    "mthip_memory_stats": (_int, [_int, ctypes.POINTER(_size), ctypes.POINTER(_size)]),
    "mthip_memcpy_h2d": (_int, [_int, _c_void_p, _c_void_p, _size]),
    "mthip_memcpy_d2h": (_int, [_int, _c_void_p, _c_void_p, _size]),
    "mthip_memcpy_d2d": (_int, [_int, _c_void_p, _c_void_p, _size]),
    "mthip_synchronize": (_int, [_int]),
    "mthip_stream": (_c_void_p, [_int]),
    "mthip_graph_begin": (_int, [_int]),
    "mthip_graph_end": (_int, [_int, ctypes.POINTER(_c_void_p)]),
    "mthip_graph_launch": (_int, [_int, _c_void_p]),
    "mthip_graph_destroy": (_int, [_int, _c_void_p]),
    "mthip_event_create": (_int, [ctypes.POINTER(_c_void_p)]),
    "mthip_event_record": (_int, [_int, _c_void_p]),
    "mthip_event_elapsed_ms": (_int, [_c_void_p, _c_void_p, ctypes.POINTER(ctypes.c_float)]),
    "mthip_event_destroy": (_int, [_c_void_p]),
    "mthip_cast": (_int, [_int, _int, _c_void_p, _int, _c_void_p, _i64]),
    "mthip_copy_strided": (_int, [_int, _int, _c_void_p, _int, _i64p, _i64p, _c_void_p]),
    "mthip_copy_strided_to": (_int, [_int, _int, _c_void_p, _i64p, _int, _i64p, _c_void_p, _i64p]),
    "mthip_fill": (_int, [_int, _int, _c_void_p, _i64, _dbl]),
    "mthip_fill_strided": (_int, [_int, _int, _c_void_p, _int, _i64p, _i64p, _dbl]),
    "mthip_masked_fill": (_int, [_int, _int, _c_void_p, _i64p, _c_void_p, _i64p, _dbl, _c_void_p, _int, _i64p]),
    "mthip_logical_not": (_int, [_int, _c_void_p, _c_void_p, _i64]),
    "mthip_cat": (_int, [_int, _int, _int, ctypes.POINTER(_c_void_p), _i64p, _int, _i64p, _int, _c_void_p]),
    "mthip_upsample_nearest2d": (_int, [_int, _int, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64]),
    "mthip_timestep_embedding_f16": (_int, [_int, _c_void_p, _c_void_p, _c_void_p, _i64, _i64]),
    "mthip_binary": (_int, [_int, _int, _int, _c_void_p, _i64p, _c_void_p, _i64p, _c_void_p, _int, _i64p]),
    "mthip_binary_scalar": (_int, [_int, _int, _int, _c_void_p, _dbl, _int, _c_void_p, _i64]),
    "mthip_unary": (_int, [_int, _int, _int, _c_void_p, _c_void_p, _i64]),
    "mthip_geglu": (_int, [_int, _int, _c_void_p, _c_void_p, _i64, _i64]),
    "mthip_linear": (_int, [_int, _int, _c_void_p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p, _i64,
                            _i64, _i64, _i64, _int, _c_void_p, _i64]),
    "mthip_linear_geglu": (_int, [_int, _int, _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64,
                                  _i64]),
    "mthip_gemm": (_int, [_int, _int, _i64, _i64, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _i64, _i64,
                          _int, _c_void_p, _i64, _i64, _dbl, _dbl, _c_void_p, _i64, _i64, _i64]),
    "mthip_conv2d": (_int, [_int, _int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64,
                            _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _c_void_p]),
    "mthip_conv2d_packed_bytes": (_i64, [_int, _i64, _i64, _i64, _i64]),
    "mthip_conv2d_pack_weight": (_int, [_int, _int, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64]),
    "mthip_conv2d_prepacked": (_int, [_int, _int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64,
                                      _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _c_void_p]),
    "mthip_upsample2x_to_nhwc": (_int, [_int, _int, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64]),
    "mthip_conv2d_nhwc": (_int, [_int, _int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64,
                                 _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _c_void_p,
                                 _c_void_p, _i64]),
    "mthip_sdpa": (_int, [_int, _int, _c_void_p, _i64p, _c_void_p, _i64p, _c_void_p, _i64p, _c_void_p, _i64p,
                          _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _int, _c_void_p, _i64p, _int, _int,
                          _dbl]),
    "mthip_group_norm": (_int, [_int, _int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64,
                                _i64, _dbl, _int, _int]),
    "mthip_group_norm_noalloc": (_int, [_int, _int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64,
                                        _i64, _dbl, _int, _int]),
    "mthip_group_norm_nhwc": (_int, [_int, _int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64,
                                     _i64, _dbl, _int, _int]),
    "mthip_group_norm_nhwc_cat": (_int, [_int, _int, _c_void_p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p,
                                          _c_void_p, _i64, _i64, _i64, _dbl, _int, _int]),
    "mthip_layer_norm": (_int, [_int, _int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _dbl, _int]),
    "mthip_softmax_lastdim": (_int, [_int, _int, _c_void_p, _c_void_p, _i64, _i64, _int]),
    "mthip_generator_create": (_c_void_p, [ctypes.c_uint64]),
    "mthip_generator_destroy": (None, [_c_void_p]),
    "mthip_generator_seed": (_int, [_c_void_p, ctypes.c_uint64]),
    "mthip_generator_get_state": (_int, [_c_void_p, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(_int),
                                         ctypes.POINTER(_dbl)]),
    "mthip_generator_set_state": (_int, [_c_void_p, ctypes.c_uint64, _int, _dbl]),
    "mthip_rng_normal": (_int, [_c_void_p, _int, _c_void_p, _i64, _dbl, _dbl]),
    "mthip_rng_uniform": (_int, [_c_void_p, _int, _c_void_p, _i64, _dbl, _dbl]),
}

_lib = None


def lib():
    """Returns the loaded library, loading it on first use."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"mtorch_amd: the device library {LIB_PATH} is not built "
                "(run `make -C mtorch_amd/csrc` or __graft_entry__.build())"
            )
        handle = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def check(rc: int) -> None:
    """Raises RuntimeError carrying the library's message for a non-zero status."""
    if rc != 0:
        msg = _lib.mthip_last_error().decode("utf-8", "replace") if _lib is not None else ""
        raise RuntimeError(msg or f"mthip call failed with status {rc}")


def int64_array(values):
    values = list(values)
    return (ctypes.c_int64 * max(len(values), 1))(*values)


def declared_symbols():
    """Entry points this binding expects the library to export (all of include/mthip.h)."""
    return list(_SIGNATURES)
