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
from . import q8_0 as _q8_0
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


def matmul_q4k_gemm(a_bf16: DeviceBuffer, weight: DeviceBuffer, output: DeviceBuffer, m: int, n: int, k: int,
                    stream=None) -> None:
    """``matmul_q4k`` at M > 1 (prefill): output f32[m][n] = a bf16[m][k] @
    dequant(weight)[n][k]^T on the matrix cores."""
    _q4k_weight_check(weight, n, k)
    _need(a_bf16, m * k * 2, "a")
    _need(output, m * n * 4, "output")
    _lib.call("doe_q4k_gemm", _p(a_bf16), _p(weight), _p(output), m, n, k, _stream_ptr(stream))


def matmul_q4k_gemm_f32(a: DeviceBuffer, weight: DeviceBuffer, output: DeviceBuffer, m: int, n: int, k: int,
                        stream=None) -> None:
    """``matmul_q4k`` at M > 1 with f32 activations a [m][k] (rounded to f16
    per row by the GEMM's pre-pass): output f32 [m][n]."""
    _q4k_weight_check(weight, n, k)
    _need(a, m * k * 4, "a")
    _need(output, m * n * 4, "output")
    _lib.call("doe_q4k_gemm_f32", _p(a), _p(weight), _p(output), m, n, k, _stream_ptr(stream))


def qkv_rope_kv_rows(qkv: DeviceBuffer, tokens: int, row_stride: int, num_heads: int, num_kv_heads: int,
                     head_dim: int, freq_cis: DeviceBuffer, start_pos: int, key_cache: DeviceBuffer | None,
                     val_cache: DeviceBuffer | None, max_seq_len: int, stream=None) -> None:
    """Prompt rope_q / rope_k + cache write over `tokens` fused q/k/v rows."""
    if tokens:
        _need(qkv, ((tokens - 1) * row_stride + (num_heads + 2 * num_kv_heads) * head_dim) * 4, "qkv")
    _need(freq_cis, max_seq_len * head_dim * 4, "freq_cis")
    kc = vc = C.c_void_p(None)
    if num_kv_heads:
        _need(key_cache, num_kv_heads * max_seq_len * head_dim * 2, "key_cache")
        _need(val_cache, num_kv_heads * max_seq_len * head_dim * 2, "val_cache")
        kc, vc = _p(key_cache), _p(val_cache)
    _lib.call("doe_qkv_rope_kv_rows", _p(qkv), tokens, row_stride, num_heads, num_kv_heads, head_dim, _p(freq_cis),
              start_pos, kc, vc, max_seq_len, _stream_ptr(stream))


def geglu_pairs(gate_up: DeviceBuffer, output: DeviceBuffer, n: int, stream=None) -> None:
    """``gelu_gated`` over interleaved (gate, up) pairs: output[i] =
    gelu(gate_up[2i]) * gate_up[2i + 1]."""
    _need(gate_up, 2 * n * 4, "gate_up")
    _need(output, n * 4, "output")
    _lib.call("doe_geglu_pairs", _p(gate_up), _p(output), n, _stream_ptr(stream))


def qkv_rope_half_kv_rows(qkv: DeviceBuffer, tokens: int, row_stride: int, num_heads: int, num_kv_heads: int,
                          head_dim: int, freq_cis: DeviceBuffer, start_pos: int, key_cache: DeviceBuffer | None,
                          val_cache: DeviceBuffer | None, max_seq_len: int, stream=None) -> None:
    """Prompt rope_q / rope_k (rotate-half pairs, as ``rope``) + cache write
    over `tokens` rows of [q heads | k heads | v heads]."""
    if tokens:
        _need(qkv, ((tokens - 1) * row_stride + (num_heads + 2 * num_kv_heads) * head_dim) * 4, "qkv")
    _need(freq_cis, max_seq_len * head_dim * 4, "freq_cis")
    kc = vc = C.c_void_p(None)
    if num_kv_heads:
        _need(key_cache, num_kv_heads * max_seq_len * head_dim * 2, "key_cache")
        _need(val_cache, num_kv_heads * max_seq_len * head_dim * 2, "val_cache")
        kc, vc = _p(key_cache), _p(val_cache)
    _lib.call("doe_qkv_rope_half_kv_rows", _p(qkv), tokens, row_stride, num_heads, num_kv_heads, head_dim,
              _p(freq_cis), start_pos, kc, vc, max_seq_len, _stream_ptr(stream))


def geglu_halves(gate_up: DeviceBuffer, output: DeviceBuffer, rows: int, n: int, stream=None) -> None:
    """``gelu_gated`` over rows of [gate (n) | up (n)]: output[t][i] =
    gelu(gate_up[t][i]) * gate_up[t][n + i]."""
    _need(gate_up, rows * 2 * n * 4, "gate_up")
    _need(output, rows * n * 4, "output")
    _lib.call("doe_geglu_halves", _p(gate_up), _p(output), rows, n, _stream_ptr(stream))


def matmul_q8_0_gemm_f32(a: DeviceBuffer, weight: DeviceBuffer, output: DeviceBuffer, m: int, n: int, k: int,
                         stream=None) -> None:
    """``matmul`` with quantFormat ``q8_0`` at M > 1: output f32 [m][n] =
    a f32 [m][k] @ dequant(weight)[n][k]^T (weights rounded to f16 once)."""
    _need(weight, n * _q8_0.row_bytes(k), "weight")
    _need(a, m * k * 4, "a")
    _need(output, m * n * 4, "output")
    _lib.call("doe_q8_0_gemm_f32", _p(a), _p(weight), _p(output), m, n, k, _stream_ptr(stream))


GEGLU_PAIRS, GEGLU_HALVES = 1, 2


def matmul_gemm_f32_fused(a: DeviceBuffer, weight: DeviceBuffer, output: DeviceBuffer, m: int, n: int, k: int,
                          weight_format: str = "q4k", *, norm_weight: DeviceBuffer | None = None,
                          norm_eps: float = 1e-6, norm_weight_offset: bool = False,
                          residual: DeviceBuffer | None = None, activation: int = 0, stream=None) -> None:
    """A prompt projection with its neighbouring steps folded in: optional
    RMSNorm of a's rows (``input_norm`` / ``post_attn_norm``), then ``matmul``
    over Q4_K or Q8_0 rows, then an optional residual add (``attn_residual``
    / ``ffn_residual``; residual may be output) or GeGLU over the gate/up
    columns (GEGLU_PAIRS: (2j, 2j + 1), GEGLU_HALVES: (j, j + n/2); output
    [m][n/2]).  Equals the unfused ops bit for bit."""
    if weight_format == "q4k":
        _q4k_weight_check(weight, n, k)
        fmt = 0
    elif weight_format == "q8_0":
        _need(weight, n * _q8_0.row_bytes(k), "weight")
        fmt = 1
    else:
        raise ValueError(f"weight_format {weight_format!r} is not q4k or q8_0")
    _need(a, m * k * 4, "a")
    _need(output, m * (n // 2 if activation else n) * 4, "output")
    if norm_weight is not None:
        _need(norm_weight, k * 4, "norm_weight")
    if residual is not None:
        _need(residual, m * n * 4, "residual")
    _lib.call("doe_quant_gemm_f32_fused", _p(a), _p(weight), _p(output), m, n, k, fmt,
              C.c_void_p(norm_weight.ptr) if norm_weight is not None else C.c_void_p(None), norm_eps,
              int(norm_weight_offset), C.c_void_p(residual.ptr) if residual is not None else C.c_void_p(None),
              activation, _stream_ptr(stream))


def matmul_q8_0(weight: DeviceBuffer, activation: DeviceBuffer, output: DeviceBuffer, n: int, k: int,
                residual: DeviceBuffer | None = None, stream=None, *, norm_weight: DeviceBuffer | None = None,
                norm_eps: float = 1e-6, norm_weight_offset: bool = False) -> None:
    """``matmul`` with quantFormat ``q8_0`` at M = 1: output f32[n] =
    dequant(weight)[n][k] @ activation f32[k] (+ residual f32[n]); weight
    row-wise Q8_0 (34-byte blocks: f16 scale, 32 int8 quants).  With
    ``norm_weight`` the activation is RMS-normalised first (the
    ``input_norm`` / ``post_attn_norm`` step folded in)."""
    expected = n * _q8_0.row_bytes(k)
    if weight.nbytes != expected:
        raise ValueError(f"Q8_0 rowwise byte length {weight.nbytes} != expected {expected}")
    _need(activation, k * 4, "activation")
    _need(output, n * 4, "output")
    if residual is not None:
        _need(residual, n * 4, "residual")
    res = None if residual is None else _p(residual)
    if norm_weight is not None:
        _need(norm_weight, k * 4, "norm_weight")
        _lib.call("doe_q8_0_gemv_norm", _p(weight), _p(activation), _p(output), n, k, _p(norm_weight), norm_eps,
                  int(norm_weight_offset), res, _stream_ptr(stream))
        return
    _lib.call("doe_q8_0_gemv", _p(weight), _p(activation), _p(output), n, k, res, _stream_ptr(stream))


def matmul_q8_0_attn_out(weight: DeviceBuffer, partials: DeviceBuffer, splits: int, num_heads: int,
                         head_dim: int, output: DeviceBuffer, n: int, residual: DeviceBuffer | None = None,
                         stream=None) -> None:
    """Q8_0 ``o_proj`` (+ ``attn_residual``) over the combine of the attention
    partials of ``attention_partials`` (the caller's buffer)."""
    k = num_heads * head_dim
    expected = n * _q8_0.row_bytes(k)
    if weight.nbytes != expected:
        raise ValueError(f"Q8_0 rowwise byte length {weight.nbytes} != expected {expected}")
    _need(partials, num_heads * splits * (head_dim + 2) * 4, "partials")
    _need(output, n * 4, "output")
    if residual is not None:
        _need(residual, n * 4, "residual")
    res = None if residual is None else _p(residual)
    _lib.call("doe_q8_0_gemv_attn_out", _p(weight), _p(partials), splits, num_heads, head_dim, _p(output), n, res,
              _stream_ptr(stream))


def matmul_int4g32(weight_u4: DeviceBuffer, scales_f16: DeviceBuffer, x: DeviceBuffer, output: DeviceBuffer,
                   m: int, n: int, k: int, stream=None) -> None:
    """Fused int4 group-32 dequant GEMV (``complex_fused_gemv_dequant``) over a
    batch of m <= 8 activation rows: output f32[m][n] = x f32[m][k] @
    ((q - 8) * scale)[n][k]^T."""
    _need(weight_u4, n * k // 2, "weight")
    _need(scales_f16, n * (k // 32) * 2, "scales")
    _need(x, m * k * 4, "x")
    _need(output, m * n * 4, "output")
    _lib.call("doe_int4g32_gemv", _p(weight_u4), _p(scales_f16), _p(x), _p(output), m, n, k, _stream_ptr(stream))


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


class AttentionUniforms(C.Structure):
    """The reference attention kernel's Uniforms block
    (attention_head256_f16kv.wgsl:14-30), field for field."""
    _fields_ = [("num_heads", C.c_uint32), ("num_kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("seq_len", C.c_uint32), ("query_len", C.c_uint32), ("scale", C.c_float),
                ("is_causal", C.c_uint32), ("start_pos", C.c_uint32), ("attn_softcap", C.c_float),
                ("sliding_window", C.c_uint32), ("kv_len_source", C.c_uint32), ("kv_start", C.c_uint32),
                ("page_size", C.c_uint32), ("kv_layout", C.c_uint32), ("pad", C.c_uint32)]


def attention_dispatch(q: DeviceBuffer, k: DeviceBuffer, v: DeviceBuffer, output: DeviceBuffer, *,
                       kv_capacity: int, kv_len_buffer: DeviceBuffer | None = None,
                       page_table: DeviceBuffer | None = None, stream=None, **uniforms) -> None:
    """``attention`` as the reference dispatches it: the Uniforms fields as
    keywords (query_len defaults to 1), K/V f16 [kv_capacity][num_kv_heads]
    [head_dim], f32 q and output [query_len][num_heads][head_dim]."""
    u = AttentionUniforms(**{"query_len": 1, **uniforms})
    hd, hq, hkv, ql = u.head_dim, u.num_heads, u.num_kv_heads, u.query_len
    _need(q, ql * hq * hd * 4, "q")
    _need(output, ql * hq * hd * 4, "output")
    _need(k, kv_capacity * hkv * hd * 2, "k")
    _need(v, kv_capacity * hkv * hd * 2, "v")
    pt_len = 0
    if page_table is not None:
        pt_len = page_table.nbytes // 4
    _lib.call("doe_attention_dispatch", C.byref(u), C.c_void_p(q.ptr), C.c_void_p(k.ptr), C.c_void_p(v.ptr),
              C.c_void_p(output.ptr), C.c_void_p(kv_len_buffer.ptr if kv_len_buffer is not None else None),
              C.c_void_p(page_table.ptr if page_table is not None else None), pt_len, kv_capacity,
              _stream_ptr(stream))


def attention_prefill_f16kv(q: DeviceBuffer, k_cache: DeviceBuffer, v_cache: DeviceBuffer, output: DeviceBuffer, *,
                            num_heads: int, num_kv_heads: int, head_dim: int, query_len: int, kv_len: int,
                            kv_stride: int, start_pos: int, scale: float, softcap: float = 0.0,
                            sliding_window: int = 0, kv_layout: int = 0, q_row_stride: int | None = None,
                            out_row_stride: int | None = None, stream=None) -> None:
    """Causal multi-query ``attention`` of a prompt (queries at start_pos +
    i) over an f16 cache in the decoder's layout; f32 q / output rows."""
    hd = num_heads * head_dim
    qs = hd if q_row_stride is None else q_row_stride
    os_ = hd if out_row_stride is None else out_row_stride
    if query_len:
        _need(q, ((query_len - 1) * qs + hd) * 4, "q")
        _need(output, ((query_len - 1) * os_ + hd) * 4, "output")
    _need(k_cache, num_kv_heads * kv_stride * head_dim * 2, "k_cache")
    _need(v_cache, num_kv_heads * kv_stride * head_dim * 2, "v_cache")
    _lib.call("doe_attn_prefill_f16kv", _p(q), qs, _p(k_cache), _p(v_cache), _p(output), os_, num_heads, num_kv_heads,
              head_dim, query_len, kv_len, kv_stride, kv_layout, start_pos, scale, softcap, sliding_window,
              _stream_ptr(stream))


def attention_prefill(q: DeviceBuffer, k: DeviceBuffer, v: DeviceBuffer, output: DeviceBuffer, *, num_heads: int,
                      num_kv_heads: int, head_dim: int, q_len: int, kv_len: int, kv_stride: int | None = None,
                      start_pos: int = 0, scale: float, causal: bool = True, out_bf16: bool = False,
                      stream=None) -> None:
    """``attention`` op, prefill form (tiled, ``is_causal``): bf16 q
    [q_len][Hq][D] against bf16 K/V [Hkv][kv_stride][D]; f32 (or bf16) output
    [q_len][Hq][D]."""
    kv_stride = kv_len if kv_stride is None else kv_stride
    if num_kv_heads <= 0 or num_heads % num_kv_heads:
        raise ValueError(f"num_heads {num_heads} is not a multiple of num_kv_heads {num_kv_heads}")
    _need(q, q_len * num_heads * head_dim * 2, "q")
    _need(k, num_kv_heads * kv_stride * head_dim * 2, "k")
    _need(v, num_kv_heads * kv_stride * head_dim * 2, "v")
    _need(output, q_len * num_heads * head_dim * (2 if out_bf16 else 4), "output")
    _lib.call("doe_attn_prefill", _p(q), _p(k), _p(v), _p(output), int(out_bf16), num_heads, num_kv_heads,
              head_dim, q_len, kv_len, kv_stride, start_pos, scale, int(causal), _stream_ptr(stream))


def attention_partials(q: DeviceBuffer, k_cache: DeviceBuffer, v_cache: DeviceBuffer, partials: DeviceBuffer, *,
                       batch: int, num_heads: int, num_kv_heads: int, head_dim: int, kv_len: int, kv_stride: int,
                       scale: float, max_splits: int = 8, q_f16: bool = False, softcap: float = 0.0,
                       sliding_window: int = 0, kv_layout: int = 0, kv_len_buffer: DeviceBuffer | None = None,
                       stream=None) -> int:
    """The split half of the ``attention`` op: (o, m, l) partials into
    ``partials`` for a consumer-side combine; returns the split count."""
    if num_kv_heads <= 0 or num_heads % num_kv_heads:
        raise ValueError(f"num_heads {num_heads} is not a multiple of num_kv_heads {num_kv_heads}")
    splits = C.c_int32()
    kvl = C.c_void_p(kv_len_buffer.ptr) if kv_len_buffer is not None else C.c_void_p(None)
    _lib.call("doe_attn_decode_partials", _p(q), int(q_f16), _p(k_cache), _p(v_cache), batch, num_heads,
              num_kv_heads, head_dim, kv_len, kvl, kv_stride, kv_layout, scale, softcap, sliding_window, _p(partials),
              partials.nbytes // 4, max_splits, C.byref(splits), _stream_ptr(stream))
    return int(splits.value)


def matmul_q4k_attn_out(weight: DeviceBuffer, partials: DeviceBuffer, splits: int, num_heads: int, head_dim: int,
                        output: DeviceBuffer, n: int, residual: DeviceBuffer | None = None, stream=None) -> None:
    """``o_proj`` (+ ``attn_residual``) over the combine of attention partials."""
    k = num_heads * head_dim
    _q4k_weight_check(weight, n, k)
    _need(partials, num_heads * splits * (head_dim + 2) * 4, "partials")
    _need(output, n * 4, "output")
    res = C.c_void_p(residual.ptr) if residual is not None else C.c_void_p(None)
    _lib.call("doe_q4k_gemv_attn_out", _p(weight), _p(partials), splits, num_heads, head_dim, _p(output), n, res,
              _stream_ptr(stream))


class Q4kGemvArgs(C.Structure):
    """``doe_q4k_gemv_args`` (include/doe_mi355x.h), field for field."""
    _fields_ = [
        ("weight_q4k", C.c_void_p), ("activation", C.c_void_p), ("activation_parts", C.c_void_p),
        ("activation_nparts", C.c_int64), ("activation_sum", C.c_void_p), ("output", C.c_void_p),
        ("n", C.c_int64), ("k", C.c_int64), ("norm_weight", C.c_void_p), ("norm_eps", C.c_float),
        ("norm_weight_offset", C.c_int32), ("residual", C.c_void_p), ("gated", C.c_int32), ("rope_kv", C.c_int32),
        ("num_heads", C.c_int64), ("num_kv_heads", C.c_int64), ("head_dim", C.c_int64), ("freq_cis", C.c_void_p),
        ("position_dev", C.c_void_p), ("key_cache", C.c_void_p), ("val_cache", C.c_void_p),
        ("max_seq_len", C.c_int64), ("attn_partials", C.c_void_p), ("attn_splits", C.c_int64),
        ("attn_num_heads", C.c_int64), ("attn_head_dim", C.c_int64), ("output_parts", C.c_void_p),
        ("max_output_parts", C.c_int64), ("output_nparts", C.c_void_p), ("residual_parts", C.c_void_p),
        ("residual_nparts", C.c_int64),
    ]


MAX_GEMV_PARTS = 4  # activation / output parts of doe_q4k_gemv_ex


def q4k_gemv_ex(weight: DeviceBuffer, n: int, k: int, *, activation: DeviceBuffer | None = None,
                activation_parts: DeviceBuffer | None = None, activation_nparts: int = 0,
                activation_sum: DeviceBuffer | None = None, output: DeviceBuffer | None = None,
                norm_weight: DeviceBuffer | None = None, norm_eps: float = 1e-6, norm_weight_offset: bool = True,
                residual: DeviceBuffer | None = None, gated: bool = False, rope: dict | None = None,
                attn_partials: DeviceBuffer | None = None, attn_splits: int = 0, attn_num_heads: int = 0,
                attn_head_dim: int = 0, output_parts: DeviceBuffer | None = None, max_output_parts: int = 0,
                residual_parts: DeviceBuffer | None = None, residual_nparts: int = 0, stream=None) -> int:
    """``doe_q4k_gemv_ex``: the Q4_K decode GEMV with every fused form, plus
    activation parts (activation + parts[0] + ... in order, the sum kept in
    ``activation_sum``) and output parts (the K ranges' row sums, one part
    each, for the next GEMV's activation parts) and residual parts (residual
    + parts[0] + ... in order: the sum an earlier GEMV's activation parts
    formed, not stored).  ``rope``: the keyword
    arguments of ``qkv_rope_kv``'s epilogue (num_heads, num_kv_heads,
    head_dim, freq_cis, position_buffer, key_cache, val_cache, max_seq_len).
    Returns the number of output parts written (1 without them)."""
    _q4k_weight_check(weight, n, k)
    a = Q4kGemvArgs()
    a.weight_q4k, a.n, a.k = weight.ptr, n, k
    if attn_partials is not None:
        _need(attn_partials, attn_num_heads * attn_splits * (attn_head_dim + 2) * 4, "attn_partials")
        a.attn_partials, a.attn_splits = attn_partials.ptr, attn_splits
        a.attn_num_heads, a.attn_head_dim = attn_num_heads, attn_head_dim
    else:
        _need(activation, k * 4, "activation")
        a.activation = activation.ptr
    if activation_nparts:
        _need(activation_parts, activation_nparts * k * 4, "activation_parts")
        a.activation_parts, a.activation_nparts = activation_parts.ptr, activation_nparts
        if activation_sum is not None:
            _need(activation_sum, k * 4, "activation_sum")
            a.activation_sum = activation_sum.ptr
    if norm_weight is not None:
        _need(norm_weight, k * 4, "norm_weight")
        a.norm_weight = norm_weight.ptr
    a.norm_eps, a.norm_weight_offset = norm_eps, int(norm_weight_offset)
    if residual is not None:
        _need(residual, n * 4, "residual")
        a.residual = residual.ptr
    if residual_nparts:
        _need(residual_parts, residual_nparts * n * 4, "residual_parts")
        a.residual_parts, a.residual_nparts = residual_parts.ptr, residual_nparts
    a.gated = int(gated)
    if rope is not None:
        hd, nh, nkv, ms = rope["head_dim"], rope["num_heads"], rope["num_kv_heads"], rope["max_seq_len"]
        _need(rope["freq_cis"], ms * hd * 4, "freq_cis")
        _need(rope["position_buffer"], 4, "position_buffer")
        a.rope_kv, a.num_heads, a.num_kv_heads, a.head_dim, a.max_seq_len = 1, nh, nkv, hd, ms
        a.freq_cis, a.position_dev = rope["freq_cis"].ptr, rope["position_buffer"].ptr
        if nkv:
            _need(rope["key_cache"], nkv * ms * hd * 2, "key_cache")
            _need(rope["val_cache"], nkv * ms * hd * 2, "val_cache")
            a.key_cache, a.val_cache = rope["key_cache"].ptr, rope["val_cache"].ptr
    nparts = C.c_int32(1)
    if output_parts is not None:
        _need(output_parts, max_output_parts * n * 4, "output_parts")
        a.output_parts, a.max_output_parts = output_parts.ptr, max_output_parts
        a.output_nparts = C.cast(C.pointer(nparts), C.c_void_p)
    else:
        _need(output, (n // 2 if gated else n) * 4, "output")
        a.output = output.ptr
    _lib.call("doe_q4k_gemv_ex", C.byref(a), _stream_ptr(stream))
    return int(nparts.value)


def _weight_check(weight: DeviceBuffer, n: int, k: int, weight_format: str) -> None:
    if weight_format == "q8_0":
        if weight.nbytes != n * _q8_0.row_bytes(k):
            raise ValueError(f"Q8_0 rowwise byte length {weight.nbytes} != expected {n * _q8_0.row_bytes(k)}")
    elif weight_format == "q4k":
        _q4k_weight_check(weight, n, k)
    else:
        raise ValueError(f"weight_format {weight_format!r} is not q4k or q8_0")


def matmul_q4k_fused(weight: DeviceBuffer, activation: DeviceBuffer, output: DeviceBuffer, n: int, k: int, *,
                     norm_weight: DeviceBuffer | None = None, norm_eps: float = 1e-6,
                     norm_weight_offset: bool = True, residual: DeviceBuffer | None = None,
                     gated: bool = False, stream=None, weight_format: str = "q4k") -> None:
    """``matmul_q4k`` with its step-list neighbours folded in: an ``rmsnorm``
    prologue (``norm_weight``), an ``attn_residual``/``ffn_residual``
    epilogue (``residual``) or a ``gelu_gated`` epilogue over interleaved
    (gate, up) rows (``gated``: output has n/2 values).  ``weight_format``
    "q8_0": the same over Q8_0 rows (``doe_q8_0_gemv_fused``)."""
    _weight_check(weight, n, k, weight_format)
    _need(activation, k * 4, "activation")
    _need(output, (n // 2 if gated else n) * 4, "output")
    if norm_weight is not None:
        _need(norm_weight, k * 4, "norm_weight")
    if residual is not None:
        _need(residual, n * 4, "residual")
    nw = C.c_void_p(norm_weight.ptr) if norm_weight is not None else C.c_void_p(None)
    rs = C.c_void_p(residual.ptr) if residual is not None else C.c_void_p(None)
    fn = "doe_q8_0_gemv_fused" if weight_format == "q8_0" else "doe_q4k_gemv_fused"
    _lib.call(fn, _p(weight), _p(activation), _p(output), n, k, nw, norm_eps,
              int(norm_weight_offset), rs, int(gated), _stream_ptr(stream))


def qkv_rope_kv(weight: DeviceBuffer, activation: DeviceBuffer, output: DeviceBuffer, *, hidden: int,
                num_heads: int, num_kv_heads: int, head_dim: int, freq_cis: DeviceBuffer,
                position_buffer: DeviceBuffer, key_cache: DeviceBuffer, val_cache: DeviceBuffer,
                max_seq_len: int, norm_weight: DeviceBuffer | None = None, norm_eps: float = 1e-6,
                norm_weight_offset: bool = True, stream=None, weight_format: str = "q4k") -> None:
    """input_norm + q/k/v_proj + rope_q/rope_k + cache write in one dispatch.

    Q and K weight rows must be interleaved rotation pairs per head (see
    ``interleave_rope_rows``); output holds [q; k; v] in that order.
    ``weight_format`` "q4k" or "q8_0" names the rows' block format."""
    n = (num_heads + 2 * num_kv_heads) * head_dim
    _weight_check(weight, n, hidden, weight_format)
    _need(activation, hidden * 4, "activation")
    _need(output, n * 4, "output")
    cache = num_kv_heads * max_seq_len * head_dim * 2
    if num_kv_heads:  # 0: q rows only, no cache (a shared-KV layer)
        _need(key_cache, cache, "key_cache")
        _need(val_cache, cache, "val_cache")
    _need(freq_cis, max_seq_len * head_dim * 4, "freq_cis")
    _need(position_buffer, 4, "position_buffer")
    nw = C.c_void_p(norm_weight.ptr) if norm_weight is not None else C.c_void_p(None)
    kc = _p(key_cache) if num_kv_heads else C.c_void_p(None)
    vc = _p(val_cache) if num_kv_heads else C.c_void_p(None)
    fn = "doe_q8_0_gemv_qkv_rope_kv" if weight_format == "q8_0" else "doe_q4k_gemv_qkv_rope_kv"
    _lib.call(fn, _p(weight), _p(activation), _p(output), hidden, nw, norm_eps,
              int(norm_weight_offset), num_heads, num_kv_heads, head_dim, _p(freq_cis), _p(position_buffer),
              kc, vc, max_seq_len, _stream_ptr(stream))


def interleave_rope_rows(rows: np.ndarray, head_dim: int) -> np.ndarray:
    """Reorders the rows of each head so that rows (2i, 2i+1) are the
    rotate-half pair (i, i + head_dim/2).  Works on any per-row array
    (Q4_K row bytes included)."""
    r = np.asarray(rows)
    heads = r.shape[0] // head_dim
    half = head_dim // 2
    v = r.reshape(heads, 2, half, *r.shape[1:])
    return np.ascontiguousarray(np.swapaxes(v, 1, 2).reshape(r.shape))


def deinterleave_rope_rows(rows: np.ndarray, head_dim: int) -> np.ndarray:
    """Inverse of ``interleave_rope_rows``."""
    r = np.asarray(rows)
    heads = r.shape[0] // head_dim
    half = head_dim // 2
    v = r.reshape(heads, half, 2, *r.shape[1:])
    return np.ascontiguousarray(np.swapaxes(v, 1, 2).reshape(r.shape))


def rmsnorm(input: DeviceBuffer, weight: DeviceBuffer, output: DeviceBuffer, rows: int, size: int,
            eps: float = 1e-6, weight_offset: bool = False, stream=None) -> None:
    """``rmsnorm`` op: per row x * 1/sqrt(mean(x^2) + eps) * (w or 1 + w)."""
    _need(input, rows * size * 4, "input")
    _need(weight, size * 4, "weight")
    _need(output, rows * size * 4, "output")
    _lib.call("doe_rmsnorm", _p(input), _p(weight), _p(output), rows, size, eps, int(weight_offset),
              _stream_ptr(stream))


def rope(qk: DeviceBuffer, freq_cis: DeviceBuffer, seq_len: int, num_heads: int, head_dim: int,
         position_offset: int = 0, position_buffer: DeviceBuffer | None = None, stream=None) -> None:
    """``rope`` op: rotate-half RoPE in place on qk[seq][heads][head_dim]."""
    _need(qk, seq_len * num_heads * head_dim * 4, "qk")
    pb = C.c_void_p(position_buffer.ptr) if position_buffer is not None else C.c_void_p(None)
    _lib.call("doe_rope", _p(qk), _p(freq_cis), seq_len, num_heads, head_dim, position_offset, pb,
              _stream_ptr(stream))


def rope_partial(qk: DeviceBuffer, freq_cis: DeviceBuffer, seq_len: int, num_heads: int, head_dim: int,
                 rotary_dim: int, position_offset: int = 0, stream=None) -> None:
    """``rope`` over each head's first ``rotary_dim`` dims (rotate-half pairs
    within them; freq_cis [pos][rotary_dim/2][2])."""
    _need(qk, seq_len * num_heads * head_dim * 4, "qk")
    _need(freq_cis, (position_offset + seq_len) * rotary_dim * 4, "freq_cis")
    _lib.call("doe_rope_partial", _p(qk), _p(freq_cis), seq_len, num_heads, head_dim, rotary_dim, position_offset,
              C.c_void_p(None), _stream_ptr(stream))


def gelu_gated(gate: DeviceBuffer, up: DeviceBuffer, output: DeviceBuffer, n: int, stream=None) -> None:
    """``gelu_gated`` op: gelu_tanh(gate) * up."""
    for buf, role in ((gate, "gate"), (up, "up"), (output, "output")):
        _need(buf, n * 4, role)
    _lib.call("doe_geglu", _p(gate), _p(up), _p(output), n, _stream_ptr(stream))


def copy_rows(dst: DeviceBuffer, dst_pitch: int, src: DeviceBuffer, src_pitch: int, row_bytes: int, rows: int,
              stream=None) -> None:
    """``rows`` rows of ``row_bytes`` from ``src`` (rows ``src_pitch`` bytes
    apart) into ``dst`` (rows ``dst_pitch`` apart), on the device."""
    if rows and row_bytes:
        if row_bytes > min(dst_pitch, src_pitch):
            raise ValueError(f"row of {row_bytes} bytes wider than a pitch ({dst_pitch}, {src_pitch})")
        _need(dst, (rows - 1) * dst_pitch + row_bytes, "dst")
        _need(src, (rows - 1) * src_pitch + row_bytes, "src")
    _lib.call("doe_memcpy2d_d2d", _p(dst), dst_pitch, _p(src), src_pitch, row_bytes, rows, _stream_ptr(stream))


def residual(input: DeviceBuffer, residual_in: DeviceBuffer, output: DeviceBuffer, n: int, stream=None) -> None:
    """``residual`` op: input + residual."""
    for buf, role in ((input, "input"), (residual_in, "residual"), (output, "output")):
        _need(buf, n * 4, role)
    _lib.call("doe_residual_add", _p(input), _p(residual_in), _p(output), n, _stream_ptr(stream))


GATED_KINDS = {"gelu": 0, "silu": 1, "sigmoid": 2}


def gated(gate: DeviceBuffer, input: DeviceBuffer, output: DeviceBuffer, n: int, kind: str, stream=None) -> None:
    """``gelu_gated`` / ``silu_gated`` / ``sigmoid_gated`` (the graph's
    ``o_gate``): output = act(gate) * input, the reference's clamps."""
    if kind not in GATED_KINDS:
        raise ValueError(f"kind {kind!r} is not one of {sorted(GATED_KINDS)}")
    for buf, role in ((gate, "gate"), (input, "input"), (output, "output")):
        _need(buf, n * 4, role)
    _lib.call("doe_gated", _p(gate), _p(input), _p(output), n, GATED_KINDS[kind], _stream_ptr(stream))


def l2_normalize(input: DeviceBuffer, output: DeviceBuffer, rows: int, hidden: int, eps: float = 1e-6,
                 stream=None) -> None:
    """``l2_normalize``: each row / sqrt(sum of squares + eps)."""
    _need(input, rows * hidden * 4, "input")
    _need(output, rows * hidden * 4, "output")
    _lib.call("doe_l2_normalize", _p(input), _p(output), rows, hidden, eps, _stream_ptr(stream))


def conv1d_depthwise(input: DeviceBuffer, weight: DeviceBuffer, bias: DeviceBuffer | None, output: DeviceBuffer,
                     tokens: int, channels: int, kernel_size: int, stream=None) -> None:
    """``conv1d_depthwise``: causal depthwise conv over [tokens][channels]."""
    _need(input, tokens * channels * 4, "input")
    _need(output, tokens * channels * 4, "output")
    _need(weight, channels * kernel_size * 4, "weight")
    if bias is not None:
        _need(bias, channels * 4, "bias")
    b = _p(bias) if bias is not None else C.c_void_p(None)
    _lib.call("doe_conv1d_depthwise", _p(input), _p(weight), b, _p(output), tokens, channels, kernel_size,
              _stream_ptr(stream))


def linear_attention(q: DeviceBuffer, k: DeviceBuffer, v: DeviceBuffer, gate: DeviceBuffer, state: DeviceBuffer,
                     output: DeviceBuffer, tokens: int, heads: int, key_dim: int, value_dim: int,
                     a_log: DeviceBuffer | None = None, stream=None) -> None:
    """``linear_attention`` (gated DeltaNet): `tokens` tokens in order
    through the per-head state [heads][value_dim][key_dim] (in place)."""
    for buf, role, n in ((q, "q", value_dim), (gate, "gate", value_dim), (output, "output", value_dim),
                         (k, "k", key_dim), (v, "v", key_dim)):
        _need(buf, tokens * heads * n * 4, role)
    _need(state, heads * value_dim * key_dim * 4, "state")
    al = _p(a_log) if a_log is not None else C.c_void_p(None)
    if a_log is not None:
        _need(a_log, heads * 4, "a_log")
    _lib.call("doe_linear_attention", _p(q), _p(k), _p(v), _p(gate), _p(state), _p(output), tokens, heads, key_dim,
              value_dim, al, _stream_ptr(stream))


def ple_modulate(projected: DeviceBuffer, gathered: DeviceBuffer, output: DeviceBuffer, n: int, scale: float,
                 stream=None) -> None:
    """``ple_modulate`` step: output = (projected + gathered) * scale."""
    for b, role in ((projected, "projected"), (gathered, "gathered"), (output, "output")):
        _need(b, n * 4, role)
    _lib.call("doe_ple_modulate", _p(projected), _p(gathered), _p(output), n, scale, _stream_ptr(stream))


def sample(logits: DeviceBuffer, n: int, token: DeviceBuffer, workspace: DeviceBuffer, stream=None) -> None:
    """``sample`` op (greedy): token = argmax(logits), lowest index on ties."""
    _need(logits, n * 4, "logits")
    _need(token, 4, "token")
    _need(workspace, 8192, "workspace")
    _lib.call("doe_argmax", _p(logits), n, _p(token), _p(workspace), _stream_ptr(stream))


def kv_write(key_proj: DeviceBuffer, val_proj: DeviceBuffer, key_cache: DeviceBuffer, val_cache: DeviceBuffer,
             num_kv_heads: int, max_seq_len: int, head_dim: int, position: int = 0,
             position_buffer: DeviceBuffer | None = None, kv_layout: int = 0, stream=None) -> None:
    """``kv_write`` op: cache[h][pos][:] = f16(proj[h][:]) for K and V."""
    if position_buffer is None and not 0 <= position < max_seq_len:
        raise ValueError(f"position {position} exceeds max_seq_len {max_seq_len}")
    _need(key_proj, num_kv_heads * head_dim * 4, "key_proj")
    _need(val_proj, num_kv_heads * head_dim * 4, "val_proj")
    _need(key_cache, num_kv_heads * max_seq_len * head_dim * 2, "key_cache")
    _need(val_cache, num_kv_heads * max_seq_len * head_dim * 2, "val_cache")
    pb = C.c_void_p(position_buffer.ptr) if position_buffer is not None else C.c_void_p(None)
    _lib.call("doe_kv_write", _p(key_proj), _p(val_proj), _p(key_cache), _p(val_cache), num_kv_heads,
              max_seq_len, head_dim, position, pb, kv_layout, _stream_ptr(stream))


def embed(table: DeviceBuffer, ids: DeviceBuffer, output: DeviceBuffer, n_ids: int, vocab: int, hidden: int,
          scale: float = 1.0, stream=None) -> None:
    """``embed`` op (pattern ``gather``): output[t] = scale * table[ids[t]]."""
    _need(table, vocab * hidden * 2, "table")
    _need(ids, n_ids * 4, "ids")
    _need(output, n_ids * hidden * 4, "output")
    _lib.call("doe_embed_gather", _p(table), _p(ids), _p(output), n_ids, vocab, hidden, scale,
              _stream_ptr(stream))


def gather_f32(table: DeviceBuffer, ids: DeviceBuffer, output: DeviceBuffer, n_ids: int, vocab: int,
               hidden: int, *, strict: bool = True, bad_ids: DeviceBuffer | None = None, stream=None) -> None:
    """The interpreter's ``gather``: output[t] = table[ids[t]], u32 ids, f32
    table.  ``strict`` mirrors the reference's rejection of an id outside the
    table: the call waits for the stream and raises ValueError naming the
    count (the rows are zero-filled).  ``strict=False`` does not wait; pass
    ``bad_ids`` (one device int32) to collect the count."""
    _need(table, vocab * hidden * 4, "table")
    _need(ids, n_ids * 4, "ids")
    _need(output, n_ids * hidden * 4, "output")
    if strict and bad_ids is None:
        bad_ids = DeviceBuffer.empty((1,), np.int32)
    if bad_ids is not None:
        _need(bad_ids, 4, "bad_ids")
    _lib.call("doe_gather_f32", _p(ids), _p(table), _p(output), n_ids, vocab, hidden,
              C.c_void_p(bad_ids.ptr) if bad_ids is not None else C.c_void_p(None), _stream_ptr(stream))
    if strict:
        if stream is not None:
            _lib.call("doe_stream_synchronize", _stream_ptr(stream))
        bad = int(bad_ids.download()[0])
        if bad:
            raise ValueError(f"gather rejects {bad} token index(es) outside the {vocab}-row table")


def lm_head(weight_f16: DeviceBuffer, activation: DeviceBuffer, output: DeviceBuffer, n: int, k: int,
            alpha: float = 1.0, stream=None) -> None:
    """f16-weight GEMV (lm_head_gemv): output[n] = alpha * weight[n][k] @ activation[k]."""
    _need(weight_f16, n * k * 2, "weight")
    _need(activation, k * 4, "activation")
    _need(output, n * 4, "output")
    _lib.call("doe_f16_gemv", _p(weight_f16), _p(activation), _p(output), n, k, alpha, _stream_ptr(stream))


def lm_head_gemv(activation: DeviceBuffer, weight_f16: DeviceBuffer, output: DeviceBuffer, m: int, n: int,
                 k: int, alpha: float = 1.0, transpose_b: int = 1, stream=None) -> None:
    """lm_head_gemv with its uniforms (M, N, K, alpha, transpose_b):
    output[r][j] = alpha * sum_k activation[r][k] * B(j, k), B(j, k) =
    weight[j][k] (transpose_b 1) or weight[k][j] (transpose_b 0)."""
    _need(weight_f16, n * k * 2, "weight")
    _need(activation, m * k * 4, "activation")
    _need(output, m * n * 4, "output")
    _lib.call("doe_lm_head_gemv", _p(activation), _p(weight_f16), _p(output), m, n, k, alpha, int(transpose_b),
              _stream_ptr(stream))


def lm_head_sample(weight_f16: DeviceBuffer, activation: DeviceBuffer, n: int, k: int, partials: DeviceBuffer, *,
                   logits: DeviceBuffer | None = None, norm_weight: DeviceBuffer | None = None,
                   norm_eps: float = 1e-6, norm_weight_offset: bool = True, alpha: float = 1.0,
                   stream=None) -> int:
    """Final norm + lm_head + greedy-sample partials in one dispatch; returns
    the number of argmax partial keys written to ``partials`` (u64, >= 1024)."""
    _need(weight_f16, n * k * 2, "weight")
    _need(activation, k * 4, "activation")
    _need(partials, 1024 * 8, "partials")
    if logits is not None:
        _need(logits, n * 4, "logits")
    cnt = C.c_int32()
    _lib.call("doe_f16_gemv_argmax", _p(weight_f16), _p(activation),
              C.c_void_p(logits.ptr) if logits is not None else C.c_void_p(None), n, k, alpha,
              C.c_void_p(norm_weight.ptr) if norm_weight is not None else C.c_void_p(None), norm_eps,
              int(norm_weight_offset), _p(partials), partials.nbytes // 8, C.byref(cnt), _stream_ptr(stream))
    return int(cnt.value)


def tune(key: str, value: int) -> None:
    """Overrides a launch-shape choice (``doe_tune_set``); 0 restores automatic."""
    _lib.call("doe_tune_set", key.encode(), int(value))


OPS = {
    "attention": attention,
    "attention_prefill": attention_prefill,
    "dequant": dequant_q4k,
    "embed": embed,
    "gelu_gated": gelu_gated,
    "kv_write": kv_write,
    "lm_head": lm_head,
    "matmul_q4k": matmul_q4k,
    "matmul_q4k_gemm": matmul_q4k_gemm,
    "matmul_int4g32": matmul_int4g32,
    "residual": residual,
    "rmsnorm": rmsnorm,
    "rope": rope,
    "sample": sample,
}
