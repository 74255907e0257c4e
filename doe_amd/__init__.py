"""doe_amd -- MI355X (gfx950) quantized-decode hot path behind a C ABI.

The kernels live in ``libdoe_mi355x.so`` (built from ``doe_amd/csrc`` by
``doe_amd.build``); this package is the ctypes host layer over it.
"""
from . import q4k
from ._lib import DoeError, DoeLibraryMissing, LIB_PATH
from .device import DeviceBuffer, Event, Graph, Stream, device_info, init, synchronize
from . import ops

__all__ = [
    "DoeError",
    "DoeLibraryMissing",
    "LIB_PATH",
    "DeviceBuffer",
    "Event",
    "Graph",
    "Stream",
    "device_info",
    "init",
    "synchronize",
    "ops",
    "q4k",
]
