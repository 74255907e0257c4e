"""Per-kernel operator interface of the hot path (host side).

Each function is one dispatch of one kernel, named after the Doppler op it
replaces (runtime/zig/src/doe_wgsl/emit_csl_exec_v1.zig:114-182 ``opToSpec``)
and taking the reference's binding roles as ``DeviceBuffer`` arguments plus its
shape parameters.  Shapes and byte lengths are validated here with the
reference's error behaviour (``ValueError`` on a byte-length mismatch, as in
bench/tools/doppler_rdrr_q4k.py:128-156); the kernel itself runs in
``libdoe_mi355x.so``.  Calls are asynchronous on ``stream`` (None = default).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from . import q4k as _q4k
from .device import DeviceBuffer, _stream_ptr


def _p(buf: DeviceBuffer) -> C.c_void_p:
    return C.c_void_p(buf.ptr)


def _need(buf: DeviceBuffer, nbytes: int, role: str) -> None:
    if buf.nbytes < nbytes:
        raise ValueError(f"{role} has {buf.nbytes} bytes, expected at least {nbytes}")


def _q4k_weight_check(weight: DeviceBuffer, n: int, k: int) -> None:
    expected = n * _q4k.row_bytes(k)
    if weight.nbytes != expected:
        raise ValueError(f"Q4_K_M rowwise byte length {weight.nbytes} != expected {expected}")


def dequant_q4k(weight: DeviceBuffer, output: DeviceBuffer, n: int, k: int, stream=None) -> None:
    """``dequant`` op: output f32[n][k] = row-wise Q4_K_M dequant of ``weight``."""
    _q4k_weight_check(weight, n, k)
    _need(output, n * k * 4, "output")
    _lib.call("doe_q4k_dequant", _p(weight), _p(output), n, k, _stream_ptr(stream))


def matmul_q4k(weight: DeviceBuffer, activation: DeviceBuffer, output: DeviceBuffer, n: int,
               k: int, stream=None) -> None:
    """``matmul_q4k`` op (pattern ``fused_gemv_dequant``), decode M = 1.

    output f32[n] = dequant(weight)[n][k] @ activation f32[k].
    """
    _q4k_weight_check(weight, n, k)
    _need(activation, k * 4, "activation")
    _need(output, n * 4, "output")
    _lib.call("doe_q4k_gemv", _p(weight), _p(activation), _p(output), n, k, _stream_ptr(stream))


OPS = {
    "dequant": dequant_q4k,
    "matmul_q4k": matmul_q4k,
}
