"""ctypes wrapper of the CPU oracle ``oracle/liboracle.so``.

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
bench.py's cpu_baseline leg, to check results.  The product package
``doe_amd`` never imports it.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = C.CDLL(str(LIB_PATH))
        L = _lib
        vp, i64, f32, i32 = C.c_void_p, C.c_int64, C.c_float, C.c_int
        sig = {
            "ora_f16_to_f32": ([C.c_uint16], f32),
            "ora_f32_to_f16": ([f32], C.c_uint16),
            "ora_bf16_to_f32": ([C.c_uint16], f32),
            "ora_f32_to_bf16": ([f32], C.c_uint16),
            "ora_q4k_unpack_scale_min": ([vp, vp, vp, vp, vp], None),
            "ora_q4k_dequant_block": ([vp, vp], None),
            "ora_q4k_dequant_rowwise": ([vp, i64, i64, vp], i32),
            "ora_q4k_gemv": ([vp, vp, vp, i64, i64], i32),
            "ora_q4k_gemv_rows": ([vp, vp, vp, i64, i64, i64, i64], i32),
            "ora_q4k_gemm_sampled": ([vp, vp, i64, i64, i64, vp, vp, i64, vp], i32),
            "ora_q4k_gemm": ([vp, vp, vp, i64, i64, i64], i32),
            "ora_f32_gemv": ([vp, vp, vp, i64, i64], i32),
            "ora_f16_gemv": ([vp, vp, vp, i64, i64, f32], i32),
            "ora_lm_head_gemv": ([vp, vp, vp, i64, i64, i64, f32, i32], i32),
            "ora_int4g32_gemv": ([vp, vp, vp, vp, i64, i64, i64], i32),
            "ora_q8_0_element_count": ([i64], i64),
            "ora_q8_0_dequant": ([vp, vp, i64, i64], i32),
            "ora_q8_0_gemv": ([vp, vp, vp, vp, i64, i64], i32),
            "ora_rmsnorm": ([vp, vp, vp, i64, i64, f32, i32], i32),
            "ora_rope_table": ([vp, i64, i64, C.c_double], i32),
            "ora_rope": ([vp, vp, i64, i64, i64, i64], i32),
            "ora_rope_pairs": ([vp, vp, vp, i64, i64, i32], i32),
            "ora_geglu": ([vp, vp, vp, i64], i32),
            "ora_residual": ([vp, vp, vp, i64], i32),
            "ora_argmax": ([vp, i64], i64),
            "ora_embed_gather": ([vp, vp, vp, i64, i64, i64, f32], i32),
            "ora_gather_f32": ([vp, vp, vp, i64, i64, i64], i32),
            "ora_kv_write": ([vp, vp, vp, vp, i64, i64, i64, i64, i32], i32),
            "ora_attn_decode": ([vp, vp, vp, vp, i64, i64, i64, i64, i64, f32, f32, i64, i32], i32),
            "ora_attn_prefill": ([vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, f32, i32, i64, i64], i32),
            "ora_gated": ([vp, vp, vp, i64, i32], i32),
            "ora_l2_normalize": ([vp, vp, i64, i64, f32], i32),
            "ora_conv1d_depthwise": ([vp, vp, vp, vp, i64, i64, i64], i32),
            "ora_linear_attention": ([vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, vp], i32),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
    return _lib


def _ptr(a: np.ndarray) -> C.c_void_p:
    return a.ctypes.data_as(C.c_void_p)


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def _ok(rc: int, name: str) -> None:
    if rc != 0:
        raise ValueError(f"{name} rejected its arguments (status {rc})")


def q4k_unpack_scale_min(block: np.ndarray):
    b = _c(block, np.uint8)
    sc = np.zeros(8, np.uint8)
    mn = np.zeros(8, np.uint8)
    d = C.c_float()
    dmin = C.c_float()
    lib().ora_q4k_unpack_scale_min(_ptr(b), _ptr(sc), _ptr(mn), C.byref(d), C.byref(dmin))
    return sc, mn, d.value, dmin.value


def q4k_dequant_block(block: np.ndarray) -> np.ndarray:
    b = _c(block, np.uint8)
    out = np.zeros(256, np.float32)
    lib().ora_q4k_dequant_block(_ptr(b), _ptr(out))
    return out


def q4k_dequant_rowwise(w: np.ndarray, rows: int, cols: int) -> np.ndarray:
    w = _c(w, np.uint8)
    out = np.zeros((rows, cols), np.float32)
    _ok(lib().ora_q4k_dequant_rowwise(_ptr(w), rows, cols, _ptr(out)), "q4k_dequant_rowwise")
    return out


def q4k_gemv(w: np.ndarray, x: np.ndarray, n: int, k: int, rows: tuple[int, int] | None = None) -> np.ndarray:
    w = _c(w, np.uint8)
    x = _c(x, np.float32)
    y = np.zeros(n, np.float32)
    if rows is None:
        _ok(lib().ora_q4k_gemv(_ptr(w), _ptr(x), _ptr(y), n, k), "q4k_gemv")
    else:
        _ok(lib().ora_q4k_gemv_rows(_ptr(w), _ptr(x), _ptr(y), n, k, rows[0], rows[1]), "q4k_gemv_rows")
    return y


def q4k_gemv_threads(w: np.ndarray, x: np.ndarray, n: int, k: int, threads: int) -> np.ndarray:
    """The same GEMV with its rows split over `threads` host threads (each
    row computed exactly as in q4k_gemv, so the result is the same bits);
    the calls release the GIL.  For the all-core CPU baseline."""
    from concurrent.futures import ThreadPoolExecutor

    w = _c(w, np.uint8)
    x = _c(x, np.float32)
    y = np.zeros(n, np.float32)
    threads = max(1, min(int(threads), n)) if n else 1
    cuts = [n * i // threads for i in range(threads + 1)]

    def part(i):
        return lib().ora_q4k_gemv_rows(_ptr(w), _ptr(x), _ptr(y), n, k, cuts[i], cuts[i + 1])

    with ThreadPoolExecutor(threads) as ex:
        for rc in ex.map(part, range(threads)):
            _ok(rc, "q4k_gemv_rows")
    return y


def q4k_gemm_sampled(a_bf16: np.ndarray, b: np.ndarray, m: int, n: int, k: int, mi, ni) -> np.ndarray:
    a = _c(a_bf16, np.uint16)
    b = _c(b, np.uint8)
    mi = _c(mi, np.int64)
    ni = _c(ni, np.int64)
    out = np.zeros(len(mi), np.float32)
    _ok(lib().ora_q4k_gemm_sampled(_ptr(a), _ptr(b), m, n, k, _ptr(mi), _ptr(ni), len(mi), _ptr(out)),
        "q4k_gemm_sampled")
    return out


def q4k_gemm(a_bf16: np.ndarray, b: np.ndarray, m: int, n: int, k: int) -> np.ndarray:
    a = _c(a_bf16, np.uint16)
    b = _c(b, np.uint8)
    c = np.zeros((m, n), np.float32)
    _ok(lib().ora_q4k_gemm(_ptr(a), _ptr(b), _ptr(c), m, n, k), "q4k_gemm")
    return c


def f32_gemv(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = _c(w, np.float32)
    x = _c(x, np.float32)
    m, k = w.shape
    y = np.zeros(m, np.float32)
    _ok(lib().ora_f32_gemv(_ptr(w), _ptr(x), _ptr(y), m, k), "f32_gemv")
    return y


def f16_gemv(b_f16: np.ndarray, a: np.ndarray, alpha: float = 1.0) -> np.ndarray:
    b = _c(b_f16, np.float16).view(np.uint16)
    a = _c(a, np.float32)
    n, k = b.shape
    c = np.zeros(n, np.float32)
    _ok(lib().ora_f16_gemv(_ptr(b), _ptr(a), _ptr(c), n, k, alpha), "f16_gemv")
    return c


def lm_head_gemv(a: np.ndarray, b_f16: np.ndarray, alpha: float = 1.0, transpose_b: int = 1) -> np.ndarray:
    """a [m][k] f32; b f16 [n][k] (transpose_b 1) or [k][n] (0); returns c [m][n]."""
    a = np.atleast_2d(_c(a, np.float32))
    b = _c(b_f16, np.float16).view(np.uint16)
    m, k = a.shape
    n = b.shape[0] if transpose_b else b.shape[1]
    assert b.shape == ((n, k) if transpose_b else (k, n))
    c = np.zeros((m, n), np.float32)
    _ok(lib().ora_lm_head_gemv(_ptr(a), _ptr(b), _ptr(c), m, n, k, alpha, transpose_b), "lm_head_gemv")
    return c


def int4g32_gemv(q_u32: np.ndarray, scales_f16: np.ndarray, x: np.ndarray, m: int, n: int, k: int) -> np.ndarray:
    q = _c(q_u32, np.uint32)
    s = _c(scales_f16, np.float16).view(np.uint16)
    x = _c(x, np.float32)
    y = np.zeros((m, n), np.float32)
    _ok(lib().ora_int4g32_gemv(_ptr(q), _ptr(s), _ptr(x), _ptr(y), m, n, k), "int4g32_gemv")
    return y


def q8_0_element_count(nbytes: int) -> int | None:
    v = lib().ora_q8_0_element_count(nbytes)
    return None if v < 0 else int(v)


def q8_0_dequant(w: np.ndarray, n: int, k: int) -> np.ndarray:
    w = _c(w, np.uint8)
    if w.size != n * ((k + 31) // 32) * 34:
        raise ValueError("Q8_0 byte count does not match n x k")
    out = np.zeros((n, k), np.float32)
    _ok(lib().ora_q8_0_dequant(_ptr(w), _ptr(out), n, k), "q8_0_dequant")
    return out


def q8_0_gemv(w: np.ndarray, x: np.ndarray, n: int, k: int, residual: np.ndarray | None = None) -> np.ndarray:
    w = _c(w, np.uint8)
    if w.size != n * ((k + 31) // 32) * 34:
        raise ValueError("Q8_0 byte count does not match n x k")
    x = _c(x, np.float32)
    r = None if residual is None else _c(residual, np.float32)
    y = np.zeros(n, np.float32)
    _ok(lib().ora_q8_0_gemv(_ptr(w), _ptr(x), None if r is None else _ptr(r), _ptr(y), n, k), "q8_0_gemv")
    return y


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float, weight_offset: bool = False) -> np.ndarray:
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    h = w.shape[0]
    rows = x.size // h
    out = np.zeros_like(x)
    _ok(lib().ora_rmsnorm(_ptr(x), _ptr(w), _ptr(out), rows, h, eps, int(weight_offset)), "rmsnorm")
    return out


def rope_table(max_pos: int, head_dim: int, base: float = 10000.0) -> np.ndarray:
    t = np.zeros(max_pos * head_dim, np.float32)
    _ok(lib().ora_rope_table(_ptr(t), max_pos, head_dim, base), "rope_table")
    return t


def rope(qk: np.ndarray, freq_cis: np.ndarray, seq_len: int, num_heads: int, head_dim: int,
         position_offset: int) -> np.ndarray:
    out = _c(qk, np.float32).copy()
    f = _c(freq_cis, np.float32)
    _ok(lib().ora_rope(_ptr(out), _ptr(f), seq_len, num_heads, head_dim, position_offset), "rope")
    return out


def rope_partial(qk: np.ndarray, freq_cis: np.ndarray, seq_len: int, num_heads: int, head_dim: int,
                 rotary_dim: int, position_offset: int) -> np.ndarray:
    """ora_rope on each head's first rotary_dim dims (rotate-half pairs (i,
    i + rotary_dim/2); freq_cis [pos][rotary_dim/2][2]), the other dims
    unchanged: the rope_partial kernel of qwen-3-6-27b-smoke.json."""
    x = _c(qk, np.float32).reshape(seq_len, num_heads, head_dim).copy()
    r = rope(np.ascontiguousarray(x[..., :rotary_dim]), freq_cis, seq_len, num_heads, rotary_dim, position_offset)
    x[..., :rotary_dim] = r.reshape(seq_len, num_heads, rotary_dim)
    return x.reshape(-1)


def rope_pairs(x: np.ndarray, cos_t: np.ndarray, sin_t: np.ndarray, head_dim: int, num_pairs: int,
               interleaved: bool) -> np.ndarray:
    out = _c(x, np.float32).copy()
    c = _c(cos_t, np.float32)
    s = _c(sin_t, np.float32)
    _ok(lib().ora_rope_pairs(_ptr(out), _ptr(c), _ptr(s), head_dim, num_pairs, int(interleaved)), "rope_pairs")
    return out


def geglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g = _c(gate, np.float32)
    u = _c(up, np.float32)
    out = np.zeros_like(g)
    _ok(lib().ora_geglu(_ptr(g), _ptr(u), _ptr(out), g.size), "geglu")
    return out


GATED_KINDS = {"gelu": 0, "silu": 1, "sigmoid": 2}


def gated(gate: np.ndarray, inp: np.ndarray, kind: str) -> np.ndarray:
    """act(gate) * input, act gelu / silu / sigmoid with the interpreter's clamps."""
    g = _c(gate, np.float32)
    x = _c(inp, np.float32)
    out = np.zeros_like(g)
    _ok(lib().ora_gated(_ptr(g), _ptr(x), _ptr(out), g.size, GATED_KINDS[kind]), "gated")
    return out


def l2_normalize(x: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    x = _c(x, np.float32)
    hidden = x.shape[-1]
    out = np.zeros_like(x)
    _ok(lib().ora_l2_normalize(_ptr(x), _ptr(out), x.size // hidden, hidden, eps), "l2_normalize")
    return out


def conv1d_depthwise(x: np.ndarray, w: np.ndarray, bias: np.ndarray | None) -> np.ndarray:
    """x [tokens][channels], w [channels][kernel_size], causal."""
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    tokens, channels = x.shape
    out = np.zeros_like(x)
    b = _c(bias, np.float32) if bias is not None else None
    _ok(lib().ora_conv1d_depthwise(_ptr(x), _ptr(w), _ptr(b) if b is not None else None, _ptr(out), tokens,
                                    channels, w.shape[1]), "conv1d_depthwise")
    return out


def linear_attention(q, k, v, gate, state, a_log=None):
    """q, gate [tokens][heads][value_dim]; k, v [tokens][heads][key_dim];
    state [heads][value_dim][key_dim] (a copy is updated and returned)."""
    q, k, v, g = (_c(a, np.float32) for a in (q, k, v, gate))
    s = np.array(state, np.float32, copy=True)
    tokens, heads, vd = q.shape
    kd = k.shape[-1]
    out = np.zeros_like(q)
    al = _c(a_log, np.float32) if a_log is not None else None
    _ok(lib().ora_linear_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(s), _ptr(out), tokens, heads, kd, vd,
                                    _ptr(al) if al is not None else None), "linear_attention")
    return s, out


def residual(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = _c(a, np.float32)
    b = _c(b, np.float32)
    out = np.zeros_like(a)
    _ok(lib().ora_residual(_ptr(a), _ptr(b), _ptr(out), a.size), "residual")
    return out


def argmax(logits: np.ndarray) -> int:
    x = _c(logits, np.float32)
    return int(lib().ora_argmax(_ptr(x), x.size))


def gather_f32(table: np.ndarray, ids: np.ndarray) -> np.ndarray:
    """The interpreter's gather: f32 table [vocab][hidden], u32 ids; raises
    ValueError for an id outside the table (nothing is clamped)."""
    t = _c(table, np.float32)
    i = _c(ids, np.uint32)
    vocab, hidden = t.shape
    out = np.zeros((i.size, hidden), np.float32)
    _ok(lib().ora_gather_f32(_ptr(i), _ptr(t), _ptr(out), i.size, vocab, hidden), "gather_f32")
    return out


def embed_gather(table_f16: np.ndarray, ids: np.ndarray, scale: float = 1.0) -> np.ndarray:
    t = _c(table_f16, np.float16).view(np.uint16)
    ids = _c(ids, np.int32)
    vocab, hidden = t.shape
    out = np.zeros((ids.size, hidden), np.float32)
    _ok(lib().ora_embed_gather(_ptr(t), _ptr(ids), _ptr(out), ids.size, vocab, hidden, scale), "embed_gather")
    return out


def kv_write(k_proj, v_proj, k_cache: np.ndarray, v_cache: np.ndarray, num_kv_heads: int, max_seq: int,
             head_dim: int, pos: int, kv_layout: int = 0) -> None:
    kp = _c(k_proj, np.float32)
    vp = _c(v_proj, np.float32)
    assert k_cache.dtype == np.float16 and k_cache.flags.c_contiguous
    assert v_cache.dtype == np.float16 and v_cache.flags.c_contiguous
    _ok(lib().ora_kv_write(_ptr(kp), _ptr(vp), _ptr(k_cache), _ptr(v_cache), num_kv_heads, max_seq, head_dim,
                           pos, kv_layout), "kv_write")


def attn_decode(q: np.ndarray, k_f16: np.ndarray, v_f16: np.ndarray, num_heads: int, num_kv_heads: int,
                head_dim: int, kv_len: int, kv_stride: int, scale: float, softcap: float = 0.0,
                sliding_window: int = 0, kv_layout: int = 0) -> np.ndarray:
    q = _c(q, np.float32)
    k = _c(k_f16, np.float16).view(np.uint16)
    v = _c(v_f16, np.float16).view(np.uint16)
    o = np.zeros((num_heads, head_dim), np.float32)
    _ok(lib().ora_attn_decode(_ptr(q), _ptr(k), _ptr(v), _ptr(o), num_heads, num_kv_heads, head_dim, kv_len,
                              kv_stride, scale, softcap, sliding_window, kv_layout), "attn_decode")
    return o


def attn_prefill(q: np.ndarray, k: np.ndarray, v: np.ndarray, num_heads: int, num_kv_heads: int, head_dim: int,
                 q_len: int, kv_len: int, start_pos: int, scale: float, causal: bool = True,
                 rows: tuple[int, int] | None = None) -> np.ndarray:
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    v = _c(v, np.float32)
    o = np.zeros((q_len, num_heads, head_dim), np.float32)
    r0, r1 = rows if rows is not None else (0, q_len)
    _ok(lib().ora_attn_prefill(_ptr(q), _ptr(k), _ptr(v), _ptr(o), num_heads, num_kv_heads, head_dim, q_len,
                               kv_len, start_pos, scale, int(causal), r0, r1), "attn_prefill")
    return o
