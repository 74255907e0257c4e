"""Device memory, streams, events and graphs over the C ABI.

``DeviceBuffer`` owns one ``doe_malloc`` allocation and moves numpy arrays in
and out of it; ``Stream``/``Event``/``Graph`` wrap the HIP objects the C ABI
hands out.  Nothing here imports torch.
"""
from __future__ import annotations

import ctypes as C
import json

import numpy as np

from . import _lib

_initialised_device: int | None = None


def init(device: int = 0) -> None:
    """Initialises the library on ``device`` (idempotent)."""
    global _initialised_device
    if _initialised_device == device:
        return
    _lib.call("doe_init", device)
    _initialised_device = device


def device_info() -> dict:
    buf = C.create_string_buffer(1024)
    _lib.call("doe_device_info", buf, len(buf))
    return json.loads(buf.value.decode())


def synchronize() -> None:
    _lib.call("doe_device_synchronize")


class DeviceBuffer:
    """One device allocation of ``nbytes`` bytes with an optional dtype/shape view."""

    def __init__(self, nbytes: int, dtype=np.uint8, shape: tuple | None = None):
        self.nbytes = int(nbytes)
        self.dtype = np.dtype(dtype)
        self.shape = shape if shape is not None else (self.nbytes // self.dtype.itemsize,)
        ptr = C.c_void_p()
        _lib.call("doe_malloc", C.byref(ptr), self.nbytes)
        self._ptr = ptr.value

    @classmethod
    def empty(cls, shape, dtype) -> "DeviceBuffer":
        shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        nbytes = int(np.prod(shape, dtype=np.int64)) * np.dtype(dtype).itemsize
        return cls(nbytes, dtype, shape)

    @classmethod
    def from_array(cls, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes, arr.dtype, arr.shape)
        buf.upload(arr)
        return buf

    @property
    def ptr(self) -> int:
        if self._ptr is None and self.nbytes:
            raise RuntimeError("buffer was freed")
        return self._ptr or 0

    def upload(self, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        if arr.nbytes != self.nbytes:
            raise ValueError(f"upload of {arr.nbytes} bytes into a {self.nbytes}-byte buffer")
        _lib.call("doe_memcpy_h2d", C.c_void_p(self.ptr), arr.ctypes.data_as(C.c_void_p), self.nbytes)

    def download(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        _lib.call("doe_memcpy_d2h", out.ctypes.data_as(C.c_void_p), C.c_void_p(self.ptr), self.nbytes)
        return out

    def copy_from(self, other: "DeviceBuffer", stream: "Stream | None" = None) -> None:
        if other.nbytes != self.nbytes:
            raise ValueError("size mismatch")
        _lib.call("doe_memcpy_d2d", C.c_void_p(self.ptr), C.c_void_p(other.ptr), self.nbytes,
                  _stream_ptr(stream))

    def view(self, offset: int, nbytes: int, dtype=np.uint8, shape=None) -> DeviceView:
        return DeviceView(self, offset, nbytes, dtype, shape)

    def fill_zero(self, stream: "Stream | None" = None) -> None:
        _lib.call("doe_memset", C.c_void_p(self.ptr), 0, self.nbytes, _stream_ptr(stream))

    def free(self) -> None:
        if self._ptr is not None:
            _lib.call("doe_free", C.c_void_p(self._ptr))
            self._ptr = None

    def __del__(self):
        try:
            if getattr(self, "_ptr", None) is not None:
                _lib.load().doe_free(C.c_void_p(self._ptr))
                self._ptr = None
        except Exception:
            pass


class DeviceView:
    """A non-owning window [offset, offset + nbytes) into a DeviceBuffer,
    usable wherever an op takes a buffer (binding at a byte offset)."""

    def __init__(self, base: "DeviceBuffer", offset: int, nbytes: int, dtype=np.uint8, shape=None):
        if offset < 0 or nbytes < 0 or offset + nbytes > base.nbytes:
            raise ValueError(f"view [{offset}, {offset + nbytes}) outside a {base.nbytes}-byte buffer")
        self.base = base
        self.offset = int(offset)
        self.nbytes = int(nbytes)
        self.dtype = np.dtype(dtype)
        self.shape = shape if shape is not None else (self.nbytes // self.dtype.itemsize,)

    @property
    def ptr(self) -> int:
        return self.base.ptr + self.offset

    def download(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        _lib.call("doe_memcpy_d2h", out.ctypes.data_as(C.c_void_p), C.c_void_p(self.ptr), self.nbytes)
        return out

    def upload(self, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        if arr.nbytes != self.nbytes:
            raise ValueError(f"upload of {arr.nbytes} bytes into a {self.nbytes}-byte view")
        _lib.call("doe_memcpy_h2d", C.c_void_p(self.ptr), arr.ctypes.data_as(C.c_void_p), self.nbytes)


class Stream:
    """A created HIP stream (default priority)."""

    def __init__(self):
        h = C.c_void_p()
        _lib.call("doe_stream_create", C.byref(h))
        self.handle = h.value

    def synchronize(self) -> None:
        _lib.call("doe_stream_synchronize", C.c_void_p(self.handle))

    def destroy(self) -> None:
        if self.handle:
            _lib.call("doe_stream_destroy", C.c_void_p(self.handle))
            self.handle = None


def _stream_ptr(stream) -> C.c_void_p:
    if stream is None:
        return C.c_void_p(None)
    if isinstance(stream, Stream):
        return C.c_void_p(stream.handle)
    return C.c_void_p(int(stream))


class Event:
    def __init__(self):
        h = C.c_void_p()
        _lib.call("doe_event_create", C.byref(h))
        self.handle = h.value

    def record(self, stream=None) -> None:
        _lib.call("doe_event_record", C.c_void_p(self.handle), _stream_ptr(stream))

    def synchronize(self) -> None:
        _lib.call("doe_event_synchronize", C.c_void_p(self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        _lib.call("doe_event_elapsed_ms", C.byref(ms), C.c_void_p(self.handle), C.c_void_p(end.handle))
        return float(ms.value)

    def destroy(self) -> None:
        if self.handle:
            _lib.call("doe_event_destroy", C.c_void_p(self.handle))
            self.handle = None


class Graph:
    """A HIP graph captured from the calls made inside ``capture()``."""

    def __init__(self, handle: int):
        self.handle = handle

    @staticmethod
    def capture(stream: Stream, body) -> "Graph":
        _lib.call("doe_graph_capture_begin", C.c_void_p(stream.handle))
        try:
            body()
        finally:
            g = C.c_void_p()
            _lib.call("doe_graph_capture_end", C.c_void_p(stream.handle), C.byref(g))
        return Graph(g.value)

    def launch(self, stream: Stream) -> None:
        _lib.call("doe_graph_launch", C.c_void_p(self.handle), C.c_void_p(stream.handle))

    def destroy(self) -> None:
        if self.handle:
            _lib.call("doe_graph_destroy", C.c_void_p(self.handle))
            self.handle = None
