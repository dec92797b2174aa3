"""mtorch.cuda surface backed by libmthip.

The reference stubs is_available()/device_count() to False/0 (mtorch/__init__.py:2320-2321);
here they report the MI355X devices the HIP runtime sees.  Graph capture records the device
stream into a replayable HIP graph (for launch-bound inner loops such as a denoising step).
"""

from __future__ import annotations

import ctypes

from . import _lib


def device_count() -> int:
    try:
        lib = _lib.lib()
    except RuntimeError:
        return 0
    n = ctypes.c_int(0)
    _lib.check(lib.mthip_device_count(ctypes.byref(n)))
    return n.value


def is_available() -> bool:
    return device_count() > 0


def current_device() -> int:
    return 0


def synchronize(device=None) -> None:
    _lib.check(_lib.lib().mthip_synchronize(_index(device)))


def _index(device):
    if device is None:
        return 0
    if isinstance(device, int):
        return device
    idx = getattr(device, "index", None)
    if idx is not None:
        return idx
    text = str(device)
    return int(text.split(":")[1]) if ":" in text else 0


def get_device_name(device=None) -> str:
    buf = ctypes.create_string_buffer(256)
    cu = ctypes.c_int()
    mem = ctypes.c_size_t()
    _lib.check(_lib.lib().mthip_device_info(_index(device), buf, 256, ctypes.byref(cu), ctypes.byref(mem)))
    return buf.value.decode()


def get_device_properties(device=None):
    buf = ctypes.create_string_buffer(256)
    cu = ctypes.c_int()
    mem = ctypes.c_size_t()
    _lib.check(_lib.lib().mthip_device_info(_index(device), buf, 256, ctypes.byref(cu), ctypes.byref(mem)))
    return {"name": buf.value.decode(), "multi_processor_count": cu.value, "total_memory": mem.value}


def memory_allocated(device=None) -> int:
    a, r = ctypes.c_size_t(), ctypes.c_size_t()
    _lib.check(_lib.lib().mthip_memory_stats(_index(device), ctypes.byref(a), ctypes.byref(r)))
    return a.value


def memory_reserved(device=None) -> int:
    a, r = ctypes.c_size_t(), ctypes.c_size_t()
    _lib.check(_lib.lib().mthip_memory_stats(_index(device), ctypes.byref(a), ctypes.byref(r)))
    return r.value


def empty_cache(device=None) -> None:
    _lib.check(_lib.lib().mthip_empty_cache(_index(device)))


class Event:
    """Timing event on the device stream."""

    def __init__(self, enable_timing=True):
        h = ctypes.c_void_p()
        _lib.check(_lib.lib().mthip_event_create(ctypes.byref(h)))
        self._h = h.value

    def record(self, device=None):
        _lib.check(_lib.lib().mthip_event_record(_index(device), self._h))

    def elapsed_time(self, end: "Event") -> float:
        ms = ctypes.c_float()
        _lib.check(_lib.lib().mthip_event_elapsed_ms(self._h, end._h, ctypes.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            if getattr(self, "_h", None) and _lib._lib is not None:
                _lib._lib.mthip_event_destroy(self._h)
                self._h = None
        except Exception:
            pass


class CUDAGraph:
    """Captures the device stream between capture_begin/capture_end; replay() relaunches it.

    Tensors allocated during capture keep their device memory for the graph's lifetime, so
    outputs produced inside the capture are refreshed in place by every replay."""

    def __init__(self, device=None):
        self._dev = _index(device)
        self._g = None

    def capture_begin(self):
        _lib.check(_lib.lib().mthip_graph_begin(self._dev))

    def capture_end(self):
        g = ctypes.c_void_p()
        _lib.check(_lib.lib().mthip_graph_end(self._dev, ctypes.byref(g)))
        self._g = g.value

    def replay(self):
        _lib.check(_lib.lib().mthip_graph_launch(self._dev, self._g))

    def reset(self):
        if self._g:
            _lib.check(_lib.lib().mthip_graph_destroy(self._dev, self._g))
            self._g = None

    def __del__(self):
        try:
            if getattr(self, "_g", None) and _lib._lib is not None:
                _lib._lib.mthip_graph_destroy(self._dev, self._g)
                self._g = None
        except Exception:
            pass


class graph:
    """Context manager form: `with mtorch_amd.cuda.graph(g): ...`."""

    def __init__(self, cuda_graph: CUDAGraph):
        self.g = cuda_graph

    def __enter__(self):
        self.g.capture_begin()
        return self.g

    def __exit__(self, exc_type, exc, tb):
        self.g.capture_end()
        return False
