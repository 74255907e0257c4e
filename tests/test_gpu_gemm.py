"""GPU parity of the Q4_K dequant-fused prefill GEMM against the CPU oracle
(f32 left-fold over dequantised rows, bf16 activations upcast exactly),
through the C ABI.  Contract: rel-L2 <= 1e-3 (f32 accumulate)."""
import ctypes as C

import numpy as np
import pytest

from doe_amd import DeviceBuffer, _lib, ops, q4k

pytestmark = pytest.mark.gpu

TOL = 1e-3
# the f32-accurate prompt GEMM (f32 activations): f16 hi + lo operands, the
# dropped lo x lo term ~2^-22 of each product; measured ~1e-6 against float64
EXACT_TOL = 1e-5


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def to_bf16(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bits, round to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    r[nan] = 0x7FC0
    return r


def up(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


@pytest.mark.parametrize("m,n,k", [(1, 1, 256), (37, 200, 300), (128, 128, 512), (130, 257, 2304),
                                   (256, 384, 5376), (5, 1000, 64)])
def test_gemm_matches_oracle(dev, ora, m, n, k):
    rng = np.random.default_rng(m * 7 + n + k)
    a = to_bf16(rng.standard_normal((m, k), dtype=np.float32))
    b = q4k.random_q4k(rng, n, k)
    out = DeviceBuffer.empty((m, n), np.float32)
    ops.matmul_q4k_gemm(up(a), up(b), out, m, n, k)
    got = out.download()
    want = ora.q4k_gemm(a, b, m, n, k)
    err = rel_l2(got, want)
    print(f"[gemm {m}x{n}x{k}] rel_l2 {err:.2e}", flush=True)
    assert err <= TOL


@pytest.mark.parametrize("m,n,k", [(128, 2304, 9216), (128, 4096, 2304), (17, 300, 2048), (128, 18432, 2304),
                                   (3, 64, 1024)])
def test_gemm_f32_prompt_shapes(dev, ora, m, n, k):
    # the decoder's batched prompt: f32 activations, few 128 x 128 tiles, so K
    # runs split over the grid (partial tiles summed in split order); float64
    # reference over the dequantised weights.  The f32-accurate kernel (hi +
    # lo operands) sits at f32-GEMV accuracy; the f16-operand form (tuned) at
    # one f16 rounding per operand, inside the 1e-3 contract.
    rng = np.random.default_rng(m + n + k)
    a = rng.standard_normal((m, k), dtype=np.float32)
    b = q4k.random_q4k(rng, n, k)
    want = a.astype(np.float64) @ ora.q4k_dequant_rowwise(b, n, k).astype(np.float64).T
    ops.tune("quant_gemm.f16_operands", 1)
    try:
        out16 = DeviceBuffer.empty((m, n), np.float32)
        ops.matmul_q4k_gemm_f32(up(a), up(b), out16, m, n, k)
        err16 = rel_l2(out16.download(), want)
    finally:
        ops.tune("quant_gemm.f16_operands", 0)
    out = DeviceBuffer.empty((m, n), np.float32)
    ops.matmul_q4k_gemm_f32(up(a), up(b), out, m, n, k)
    got = out.download()
    err = rel_l2(got, want)
    print(f"[gemm f32 {m}x{n}x{k}] rel_l2 {err:.2e} (f16 operands {err16:.2e})", flush=True)
    assert err <= EXACT_TOL
    assert err16 <= TOL
    # the same call twice gives the same bits (fixed split order, no atomics)
    out2 = DeviceBuffer.empty((m, n), np.float32)
    ops.matmul_q4k_gemm_f32(up(a), up(b), out2, m, n, k)
    assert np.array_equal(out2.download(), got)


@pytest.mark.parametrize("m,n,k", [(5, 77, 129), (128, 2304, 9216), (17, 300, 2048), (64, 1000, 64),
                                   (130, 257, 2304), (1, 3, 32)])
def test_q8_0_gemm_f32(dev, ora, m, n, k):
    # Q8_0 rows (34-byte blocks, 2-byte aligned; a K that is no multiple of 32
    # zero-pads the last block) through the 128 x 128 kernel with its K split;
    # float64 reference over the oracle's dequantised rows
    from doe_amd import q8_0

    rng = np.random.default_rng(m * 3 + n + k)
    a = rng.standard_normal((m, k), dtype=np.float32)
    b = q8_0.random_q8_0(rng, n, k)
    want = a.astype(np.float64) @ ora.q8_0_dequant(b, n, k).astype(np.float64).T
    ops.tune("quant_gemm.f16_operands", 1)
    try:
        out16 = DeviceBuffer.empty((m, n), np.float32)
        ops.matmul_q8_0_gemm_f32(up(a), up(b), out16, m, n, k)
        err16 = rel_l2(out16.download(), want)
    finally:
        ops.tune("quant_gemm.f16_operands", 0)
    out = DeviceBuffer.empty((m, n), np.float32)
    ops.matmul_q8_0_gemm_f32(up(a), up(b), out, m, n, k)
    got = out.download()
    err = rel_l2(got, want)
    print(f"[q8_0 gemm {m}x{n}x{k}] rel_l2 {err:.2e} (f16 operands {err16:.2e})", flush=True)
    assert err <= EXACT_TOL
    assert err16 <= TOL
    # rows of the GEMM are the M = 1 GEMV's rows (the same blocks, f32 left-fold there)
    y0 = ora.q8_0_gemv(b, a[0], n, k)
    assert rel_l2(got[0], y0) <= EXACT_TOL


def test_gemm_prefill_config_sampled(dev, ora):
    # the 31B-class prefill shape: M=2048 tokens, K=5376, N=21504; the oracle
    # evaluates 2048 sampled entries (every row once, at a random column)
    m, n, k = 2048, 21504, 5376
    rng = np.random.default_rng(3)
    a = to_bf16(rng.standard_normal((m, k), dtype=np.float32))
    b = q4k.random_q4k(rng, n, k)
    out = DeviceBuffer.empty((m, n), np.float32)
    ops.matmul_q4k_gemm(up(a), up(b), out, m, n, k)
    got = out.download()
    mi = np.arange(m, dtype=np.int64)
    ni = rng.integers(0, n, m).astype(np.int64)
    order = np.argsort(ni, kind="stable")  # the oracle caches one dequantised row
    mi, ni = mi[order], ni[order]
    want = ora.q4k_gemm_sampled(a, b, m, n, k, mi, ni)
    err = rel_l2(got[mi, ni], want)
    print(f"[gemm config] sampled rel_l2 {err:.2e}", flush=True)
    assert err <= TOL
    assert np.isfinite(got).all()


def test_gemm_large_tiles_ragged(dev, ora):
    # enough tiles for the 256 x 256 path, with M, N and K all off the tile
    # grid (K tail inside the last Q4_K block): sampled entries, including the
    # last row and column
    m, n, k = 2000, 33000, 1000
    rng = np.random.default_rng(5)
    a = to_bf16(rng.standard_normal((m, k), dtype=np.float32))
    b = q4k.random_q4k(rng, n, k)
    out = DeviceBuffer.empty((m, n), np.float32)
    ops.matmul_q4k_gemm(up(a), up(b), out, m, n, k)
    got = out.download()
    mi = np.concatenate([rng.integers(0, m, 1500), [m - 1, m - 1, 0, 1999]]).astype(np.int64)
    ni = np.concatenate([rng.integers(0, n, 1500), [n - 1, 0, n - 1, 32767]]).astype(np.int64)
    order = np.argsort(ni, kind="stable")
    mi, ni = mi[order], ni[order]
    want = ora.q4k_gemm_sampled(a, b, m, n, k, mi, ni)
    err = rel_l2(got[mi, ni], want)
    print(f"[gemm ragged] sampled rel_l2 {err:.2e}", flush=True)
    assert err <= TOL
    assert np.isfinite(got).all()


def test_gemm_row_scaling_extremes(dev, ora):
    # rows of very different magnitude (2^-60 .. 2^60, a zero row, a row with
    # one non-zero): each row keeps the contract on its own
    rng = np.random.default_rng(4)
    m, n, k = 8, 96, 768
    base = rng.standard_normal((m, k), dtype=np.float32)
    scales = np.array([1.0, 2.0 ** 60, 2.0 ** -60, 1e-20, 3e4, 0.0, 1.0, 1.0], np.float32)
    x = base * scales[:, None]
    x[6] = 0.0
    x[6, 17] = 5.0
    x[7, ::2] *= 1e-6  # mixed magnitudes inside one row
    a = to_bf16(x)
    b = q4k.random_q4k(rng, n, k)
    out = DeviceBuffer.empty((m, n), np.float32)
    ops.matmul_q4k_gemm(up(a), up(b), out, m, n, k)
    got = out.download()
    want = ora.q4k_gemm(a, b, m, n, k)
    for r in range(m):
        if r == 5:
            assert np.array_equal(got[r], np.zeros(n, np.float32))
        else:
            assert rel_l2(got[r], want[r]) <= TOL, r


def test_gemm_zero_k_and_empty(dev):
    out = up(np.full((3, 4), 7.0, np.float32))
    dummy = DeviceBuffer(256)
    _lib.call("doe_q4k_gemm", C.c_void_p(dummy.ptr), C.c_void_p(dummy.ptr), C.c_void_p(out.ptr), 3, 4, 0,
              C.c_void_p(None))
    assert np.array_equal(out.download(), np.zeros((3, 4), np.float32))
    # m == 0 / n == 0: nothing launched, nothing written
    _lib.call("doe_q4k_gemm", C.c_void_p(dummy.ptr), C.c_void_p(dummy.ptr), C.c_void_p(out.ptr), 0, 4, 256,
              C.c_void_p(None))
    _lib.call("doe_q4k_gemm", C.c_void_p(dummy.ptr), C.c_void_p(dummy.ptr), C.c_void_p(out.ptr), 3, 0, 256,
              C.c_void_p(None))
    assert np.array_equal(out.download(), np.zeros((3, 4), np.float32))


def test_gemm_rejects_misaligned_weight(dev):
    buf = DeviceBuffer(144 * 4 + 16)
    out = DeviceBuffer.empty((1, 1), np.float32)
    a = DeviceBuffer(256 * 2)
    with pytest.raises(_lib.DoeError):
        _lib.call("doe_q4k_gemm", C.c_void_p(a.ptr), C.c_void_p(buf.ptr + 8), C.c_void_p(out.ptr), 1, 1, 256,
                  C.c_void_p(None))


@pytest.mark.parametrize("fmt", ["q4k", "q8_0"])
@pytest.mark.parametrize("m,n,k", [(128, 4096, 2304), (5, 78, 300), (130, 512, 2304), (1, 2, 256)])
def test_fused_gemm_equals_the_op_sequence(dev, fmt, m, n, k):
    # input_norm + q/k/v_proj, o_proj + attn_residual (in place) and
    # post_attn_norm + gate/up_proj + GeGLU: bit for bit the unfused ops
    from doe_amd import q8_0

    rng = np.random.default_rng(m + n + k + (fmt == "q8_0"))
    a = (rng.standard_normal((m, k)) * 3).astype(np.float32)
    nw = (0.1 * rng.standard_normal(k)).astype(np.float32)
    w = q4k.random_q4k(rng, n, k) if fmt == "q4k" else q8_0.random_q8_0(rng, n, k)
    res = rng.standard_normal((m, n)).astype(np.float32)
    gemm = ops.matmul_q4k_gemm_f32 if fmt == "q4k" else ops.matmul_q8_0_gemm_f32
    da, dw, dnw = up(a), up(w), up(nw)
    for offset in (False, True):
        xn = DeviceBuffer.empty((m, k), np.float32)
        ops.rmsnorm(da, dnw, xn, m, k, 1e-6, weight_offset=offset)
        want = DeviceBuffer.empty((m, n), np.float32)
        gemm(xn, dw, want, m, n, k)
        got = DeviceBuffer.empty((m, n), np.float32)
        ops.matmul_gemm_f32_fused(da, dw, got, m, n, k, fmt, norm_weight=dnw, norm_eps=1e-6,
                                  norm_weight_offset=offset)
        assert np.array_equal(got.download(), want.download()), ("norm", offset)
        # GeGLU over the gate/up columns in either layout
        for act in (ops.GEGLU_PAIRS, ops.GEGLU_HALVES):
            h_want = DeviceBuffer.empty((m, n // 2), np.float32)
            if act == ops.GEGLU_PAIRS:
                ops.geglu_pairs(want, h_want, m * (n // 2))
            else:
                ops.geglu_halves(want, h_want, m, n // 2)
            h_got = DeviceBuffer.empty((m, n // 2), np.float32)
            ops.matmul_gemm_f32_fused(da, dw, h_got, m, n, k, fmt, norm_weight=dnw, norm_eps=1e-6,
                                      norm_weight_offset=offset, activation=act)
            assert np.array_equal(h_got.download(), h_want.download()), ("geglu", act, offset)
    # residual, in place: x = a W^T + x
    t = DeviceBuffer.empty((m, n), np.float32)
    gemm(da, dw, t, m, n, k)
    x_want = up(res)
    ops.residual(t, x_want, x_want, m * n)
    x_got = up(res)
    ops.matmul_gemm_f32_fused(da, dw, x_got, m, n, k, fmt, residual=x_got)
    assert np.array_equal(x_got.download(), x_want.download())


@pytest.mark.parametrize("f16_operands", [0, 1])
def test_fused_gemm_large_tiles(dev, f16_operands):
    # many tiles (no K split): the f32-accurate kernel, or with f16 operands
    # the 256 x 256 tile kernel, writes its tiles to the workspace and the
    # second pass adds the residual
    ops.tune("quant_gemm.f16_operands", f16_operands)
    try:
        _fused_large_tiles()
    finally:
        ops.tune("quant_gemm.f16_operands", 0)


def _fused_large_tiles():
    m, n, k = 1024, 16384, 256
    rng = np.random.default_rng(9)
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = q4k.random_q4k(rng, n, k)
    res = rng.standard_normal((m, n)).astype(np.float32)
    da, dw = up(a), up(w)
    t = DeviceBuffer.empty((m, n), np.float32)
    ops.matmul_q4k_gemm_f32(da, dw, t, m, n, k)
    x_want = up(res)
    ops.residual(t, x_want, x_want, m * n)
    x_got = up(res)
    ops.matmul_gemm_f32_fused(da, dw, x_got, m, n, k, "q4k", residual=x_got)
    assert np.array_equal(x_got.download(), x_want.download())


def test_fused_gemm_rejects(dev):
    a = DeviceBuffer.empty((4, 256), np.float32)
    w = up(q4k.random_q4k(np.random.default_rng(1), 8, 256))
    out = DeviceBuffer.empty((4, 8), np.float32)
    with pytest.raises(_lib.DoeError, match="not with a residual"):
        ops.matmul_gemm_f32_fused(a, w, out, 4, 8, 256, residual=out, activation=ops.GEGLU_PAIRS)
    w7 = up(q4k.random_q4k(np.random.default_rng(2), 7, 256))
    with pytest.raises(_lib.DoeError, match="even column count"):
        ops.matmul_gemm_f32_fused(a, w7, out, 4, 7, 256, activation=ops.GEGLU_PAIRS)
    with pytest.raises(_lib.DoeError, match="alias the output"):
        ops.matmul_gemm_f32_fused(a, w, a, 4, 8, 256, norm_weight=up(np.ones(256, np.float32)))
    with pytest.raises(ValueError):
        ops.matmul_gemm_f32_fused(a, w, out, 4, 8, 256, "q6_k")
