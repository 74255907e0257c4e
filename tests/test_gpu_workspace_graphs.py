"""HIP graphs captured over calls that use a library-owned workspace stay
valid after later, larger calls grow those workspaces: an outgrown workspace
stays allocated until doe_shutdown, because captured graphs (and queued
kernels) keep its address.  Covers the decode attention's split partials,
the int4 GEMV's K-range partials and completion counts, and the Q4_K GEMM's
f16 copy of A and split partials; every replay equals the eager result bit
for bit (all three reduce in a fixed order)."""
import numpy as np
import pytest

from doe_amd import DeviceBuffer, Graph, Stream, _lib, ops, q4k

pytestmark = pytest.mark.gpu


def zeros(shape, dtype, s):
    b = DeviceBuffer.empty(shape, dtype)
    b.fill_zero(s)
    return b


def test_graphs_survive_workspace_growth(dev):
    rng = np.random.default_rng(5)
    up = DeviceBuffer.from_array
    s = Stream()
    # attention over 1024 positions with split partials
    hq, hkv, d, t = 8, 4, 128, 1024
    q = up(rng.standard_normal((1, hq, d)).astype(np.float32))
    kc = up(rng.standard_normal((1, hkv, t, d)).astype(np.float16))
    vc = up(rng.standard_normal((1, hkv, t, d)).astype(np.float16))
    o = DeviceBuffer.empty((1, hq, d), np.float32)

    def call_attn():
        ops.attention(q, kc, vc, o, batch=1, num_heads=hq, num_kv_heads=hkv, head_dim=d, kv_len=t,
                      kv_stride=t, scale=0.088, stream=s)

    # int4 GEMV with K split over four ranges
    m, n, k = 4, 1000, 4096
    nib = rng.integers(0, 2 ** 32, (n, k // 8), dtype=np.uint64).astype(np.uint32)
    w4 = up(nib)
    s4 = up(np.abs(rng.normal(0.0, 0.02, (n, k // 32))).astype(np.float16))
    x4 = up(rng.standard_normal((m, k)).astype(np.float32))
    y4 = DeviceBuffer.empty((m, n), np.float32)

    def call_int4():
        ops.matmul_int4g32(w4, s4, x4, y4, m, n, k, stream=s)

    # Q4_K GEMM of a short prompt (K split over the grid)
    gm, gn, gk = 64, 512, 2304
    ga = up(rng.standard_normal((gm, gk)).astype(np.float32))
    gw = up(q4k.random_q4k(rng, gn, gk))
    gc = DeviceBuffer.empty((gm, gn), np.float32)

    def call_gemm():
        ops.matmul_q4k_gemm_f32(ga, gw, gc, gm, gn, gk, stream=s)

    calls = (call_attn, call_int4, call_gemm)
    outs = (o, y4, gc)
    for f in calls:  # first calls outside capture
        f()
    s.synchronize()
    want = [b.download() for b in outs]
    g = Graph.capture(s, lambda: [f() for f in calls])

    # larger calls than any before them grow every workspace
    bq = zeros((2, 64, 128), np.float32, s)
    bk = zeros((2, 8, 32768, 128), np.float16, s)
    bv = zeros((2, 8, 32768, 128), np.float16, s)
    bo = DeviceBuffer.empty((2, 64, 128), np.float32)
    _lib.call("doe_tune_set", b"attn_decode.splits", 512)
    try:
        ops.attention(bq, bk, bv, bo, batch=2, num_heads=64, num_kv_heads=8, head_dim=128, kv_len=32768,
                      kv_stride=32768, scale=0.088, stream=s)
    finally:
        _lib.call("doe_tune_set", b"attn_decode.splits", 0)
    bn, bkk = 25600, 65536
    bw4 = zeros((bn, bkk // 8), np.uint32, s)
    bs4 = zeros((bn, bkk // 32), np.float16, s)
    bx4 = zeros((8, bkk), np.float32, s)
    by4 = DeviceBuffer.empty((8, bn), np.float32)
    ops.matmul_int4g32(bw4, bs4, bx4, by4, 8, bn, bkk, stream=s)
    bgm, bgn, bgk = 4096, 512, 8192
    bga = zeros((bgm, bgk), np.float32, s)
    bgw = up(q4k.random_q4k(rng, bgn, bgk))
    bgc = DeviceBuffer.empty((bgm, bgn), np.float32)
    ops.matmul_q4k_gemm_f32(bga, bgw, bgc, bgm, bgn, bgk, stream=s)
    s.synchronize()
    for b in (bq, bk, bv, bo, bw4, bs4, bx4, by4, bga, bgw, bgc):
        b.free()

    for rep in range(3):
        for b in outs:
            b.fill_zero(s)
        g.launch(s)
        s.synchronize()
        for name, b, ref in zip(("attention", "int4", "gemm"), outs, want):
            assert np.array_equal(b.download(), ref), (name, rep)
    g.destroy()
    s.destroy()
