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


def attention(q: DeviceBuffer, k_cache: DeviceBuffer, v_cache: DeviceBuffer, output: DeviceBuffer, *,
              batch: int, num_heads: int, num_kv_heads: int, head_dim: int, kv_len: int,
              kv_stride: int, scale: float, q_f16: bool = False, out_f16: bool = False,
              softcap: float = 0.0, sliding_window: int = 0, kv_layout: int = 0,
              kv_len_buffer: DeviceBuffer | None = None, stream=None) -> None:
    """``attention`` op (pattern ``attention_decode``): one query token per
    sequence against an f16 KV cache (GQA, kv head = h / (Hq / Hkv)).

    ``kv_len_buffer`` (a device int32) replaces ``kv_len`` when given, as the
    reference's ``kv_len_source = 1`` does."""
    if num_kv_heads <= 0 or num_heads % num_kv_heads:
        raise ValueError(f"num_heads {num_heads} is not a multiple of num_kv_heads {num_kv_heads}")
    if kv_len_buffer is None and not 0 <= kv_len <= kv_stride:
        raise ValueError(f"kv_len {kv_len} outside [0, kv_stride={kv_stride}]")
    _need(q, batch * num_heads * head_dim * (2 if q_f16 else 4), "q")
    cache_bytes = batch * num_kv_heads * kv_stride * head_dim * 2
    _need(k_cache, cache_bytes, "k_cache")
    _need(v_cache, cache_bytes, "v_cache")
    _need(output, batch * num_heads * head_dim * (2 if out_f16 else 4), "output")
    kvp = C.c_void_p(kv_len_buffer.ptr) if kv_len_buffer is not None else C.c_void_p(None)
    _lib.call("doe_attn_decode", _p(q), int(q_f16), _p(k_cache), _p(v_cache), _p(output), int(out_f16),
              batch, num_heads, num_kv_heads, head_dim, kv_len, kvp, kv_stride, kv_layout, scale, softcap,
              sliding_window, _stream_ptr(stream))


def tune(key: str, value: int) -> None:
    """Overrides a launch-shape choice (``doe_tune_set``); 0 restores automatic."""
    _lib.call("doe_tune_set", key.encode(), int(value))


OPS = {
    "attention": attention,
    "dequant": dequant_q4k,
    "matmul_q4k": matmul_q4k,
}
