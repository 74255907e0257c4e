"""GPU parity of the symmetric int4 group-32 GEMV (batch 1..8, f16 scales)
against the CPU oracle's f32 left-fold (complex_fused_gemv_dequant.wgsl
semantics), through the C ABI.  Contract: rel-L2 <= 1e-3; measured ~1e-6."""
import ctypes as C

import numpy as np
import pytest

from doe_amd import DeviceBuffer, _lib, ops

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def random_int4(rng, n, k):
    """Nibbles q+8 for q uniform in -8..7, eight per u32 (element k at bits
    4*(k%8)), and f16 scales |N(0, 0.02)| per 32 elements."""
    nib = rng.integers(0, 16, (n, k), dtype=np.uint32)
    words = np.zeros((n, k // 8), np.uint32)
    for j in range(8):
        words |= nib[:, j::8] << (4 * j)
    scales = np.abs(rng.normal(0.0, 0.02, (n, k // 32))).astype(np.float16)
    return words, scales


def up(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


@pytest.mark.parametrize("m,n,k", [(8, 9216, 5120), (1, 64, 256), (3, 1000, 512), (8, 100, 25600),
                                   (5, 5120, 2048), (8, 17, 256)])
def test_int4_gemv_matches_oracle(dev, ora, m, n, k):
    rng = np.random.default_rng(m + n + k)
    w, s = random_int4(rng, n, k)
    x = rng.standard_normal((m, k), dtype=np.float32)
    out = DeviceBuffer.empty((m, n), np.float32)
    ops.matmul_int4g32(up(w), up(s), up(x), out, m, n, k)
    got = out.download()
    want = ora.int4g32_gemv(w, s, x, m, n, k)
    err = rel_l2(got, want)
    print(f"[int4 {m}x{n}x{k}] rel_l2 {err:.2e}", flush=True)
    assert err <= 1e-5


def test_int4_known_answer_and_extremes(dev, ora):
    # all nibbles 15 (q = 7) with scale 0.5 and x = 1: every output is
    # 7 * 0.5 * k; all nibbles 0 (q = -8) gives -4 k; then per-row x scales of
    # 2^60 and 2^-60 keep the contract
    n, k = 32, 512
    w = np.full((n, k // 8), 0xFFFFFFFF, np.uint32)
    w[16:] = 0
    s = np.full((n, k // 32), 0.5, np.float16)
    x = np.ones((2, k), np.float32)
    out = DeviceBuffer.empty((2, n), np.float32)
    ops.matmul_int4g32(up(w), up(s), up(x), out, 2, n, k)
    got = out.download()
    assert np.array_equal(got[:, :16], np.full((2, 16), 3.5 * k, np.float32))
    assert np.array_equal(got[:, 16:], np.full((2, 16), -4.0 * k, np.float32))
    rng = np.random.default_rng(5)
    w, s = random_int4(rng, 256, 1024)
    x = rng.standard_normal((4, 1024), dtype=np.float32)
    x[1] *= 2.0 ** 60
    x[2] *= 2.0 ** -60
    x[3, ::3] = 0.0
    out = DeviceBuffer.empty((4, 256), np.float32)
    ops.matmul_int4g32(up(w), up(s), up(x), out, 4, 256, 1024)
    got = out.download()
    want = ora.int4g32_gemv(w, s, x, 4, 256, 1024)
    for b in range(4):
        assert rel_l2(got[b], want[b]) <= 1e-5, b


def test_int4_rejects_bad_shapes(dev):
    buf = DeviceBuffer(1 << 16)
    for m, k in ((9, 256), (0, 256), (1, 100)):
        with pytest.raises(_lib.DoeError):
            _lib.call("doe_int4g32_gemv", C.c_void_p(buf.ptr), C.c_void_p(buf.ptr), C.c_void_p(buf.ptr),
                      C.c_void_p(buf.ptr), m, 4, k, C.c_void_p(None))
    # x read by every workgroup while others write y: the two must not alias
    w = DeviceBuffer(1 << 16)
    with pytest.raises(_lib.DoeError):
        _lib.call("doe_int4g32_gemv", C.c_void_p(w.ptr), C.c_void_p(w.ptr), C.c_void_p(buf.ptr),
                  C.c_void_p(buf.ptr), 1, 4, 256, C.c_void_p(None))


@pytest.mark.parametrize("m,n,k", [(8, 9216, 5120), (8, 5120, 25600), (3, 777, 1536)])
def test_int4_gemv_is_deterministic(dev, m, n, k):
    # K ranges are summed in a fixed order (no atomics): repeated calls agree
    # bit for bit, also after a call of another shape reused the workspace
    rng = np.random.default_rng(n ^ k)
    w, s = random_int4(rng, n, k)
    x = rng.standard_normal((m, k), dtype=np.float32)
    dw, ds, dx = up(w), up(s), up(x)
    out = DeviceBuffer.empty((m, n), np.float32)
    ops.matmul_int4g32(dw, ds, dx, out, m, n, k)
    first = out.download()
    w2, s2 = random_int4(rng, 64, 2048)
    other = DeviceBuffer.empty((8, 64), np.float32)
    ops.matmul_int4g32(up(w2), up(s2), up(rng.standard_normal((8, 2048), dtype=np.float32)), other, 8, 64, 2048)
    for _ in range(3):
        ops.matmul_int4g32(dw, ds, dx, out, m, n, k)
        assert np.array_equal(out.download(), first)


@pytest.mark.parametrize("m,n,k", [(8, 25600, 5120), (8, 5120, 25600)])
def test_int4_ffn_shapes_streaming(dev, ora, m, n, k):
    # the config-4 FFN projections: enough (row block, K range) items that the
    # automatic choice is the streaming kernel (workgroups walk row blocks)
    rng = np.random.default_rng(n + k)
    w, s = random_int4(rng, n, k)
    x = rng.standard_normal((m, k), dtype=np.float32)
    out = DeviceBuffer.empty((m, n), np.float32)
    ops.matmul_int4g32(up(w), up(s), up(x), out, m, n, k)
    err = rel_l2(out.download(), ora.int4g32_gemv(w, s, x, m, n, k))
    print(f"[int4 ffn {m}x{n}x{k}] rel_l2 {err:.2e}", flush=True)
    assert err <= 1e-5


@pytest.mark.parametrize("kernel", [1, 2])
@pytest.mark.parametrize("m,n,k", [(8, 3000, 2048), (3, 1000, 7168), (1, 64 * 97 + 5, 1024)])
def test_int4_both_kernels_match_oracle(dev, ora, kernel, m, n, k):
    # one-shot (1) and streaming (2) workgroups forced on the same shapes,
    # ragged row counts and batches below 8 included
    rng = np.random.default_rng(m * n + k)
    w, s = random_int4(rng, n, k)
    x = rng.standard_normal((m, k), dtype=np.float32)
    out = DeviceBuffer.empty((m, n), np.float32)
    _lib.call("doe_tune_set", b"int4_gemv.kernel", kernel)
    try:
        ops.matmul_int4g32(up(w), up(s), up(x), out, m, n, k)
        got = out.download()
    finally:
        _lib.call("doe_tune_set", b"int4_gemv.kernel", 0)
    err = rel_l2(got, ora.int4g32_gemv(w, s, x, m, n, k))
    assert err <= 1e-5, (kernel, err)


@pytest.mark.parametrize("depth", [2, 3])
@pytest.mark.parametrize("m,n,k", [(8, 3000, 2048), (2, 64 * 9 + 7, 1024), (8, 25600, 5120)])
def test_int4_streaming_prefetch_depths(dev, ora, depth, m, n, k):
    # the streaming kernel with one and with two row blocks of weights in
    # flight per wave (int4_gemv.depth), forced on ragged and config-4 shapes:
    # both give the oracle's result and the same bits
    rng = np.random.default_rng(7 * n + k + depth)
    w, s = random_int4(rng, n, k)
    x = rng.standard_normal((m, k), dtype=np.float32)
    dw, ds, dx = up(w), up(s), up(x)
    out = DeviceBuffer.empty((m, n), np.float32)
    got = {}
    _lib.call("doe_tune_set", b"int4_gemv.kernel", 2)
    try:
        for d in (depth, 5 - depth):
            _lib.call("doe_tune_set", b"int4_gemv.depth", d)
            ops.matmul_int4g32(dw, ds, dx, out, m, n, k)
            got[d] = out.download()
    finally:
        _lib.call("doe_tune_set", b"int4_gemv.kernel", 0)
        _lib.call("doe_tune_set", b"int4_gemv.depth", 0)
    assert rel_l2(got[depth], ora.int4g32_gemv(w, s, x, m, n, k)) <= 1e-5
    assert np.array_equal(got[2], got[3])


def test_int4_one_shot_counts_across_shapes_and_graphs(dev, ora):
    # the one-shot kernel's per-row-block counts only grow (the range that
    # brings a count to a multiple of the range count adds the ranges): calls
    # of other range counts and row-block counts in between, a region that
    # grows, and replays of a captured graph with eager calls between them all
    # leave every later call exact and bit-identical
    from doe_amd import Graph, Stream

    rng = np.random.default_rng(21)
    shapes = [(8, 9216, 5120), (4, 512, 2048), (8, 20000, 5120), (2, 64, 8192), (8, 9216, 3072)]
    data = []
    for m, n, k in shapes:
        w, s = random_int4(rng, n, k)
        x = rng.standard_normal((m, k), dtype=np.float32)
        data.append((m, n, k, up(w), up(s), up(x), DeviceBuffer.empty((m, n), np.float32), w, s, x))
    ops.tune("int4_gemv.kernel", 1)  # one-shot workgroups on every shape
    try:
        first = []
        for m, n, k, dw, ds, dx, out, w, s, x in data:
            ops.matmul_int4g32(dw, ds, dx, out, m, n, k)
            got = out.download()
            assert rel_l2(got, ora.int4g32_gemv(w, s, x, m, n, k)) <= 1e-5, (m, n, k)
            first.append(got)
        for rnd in range(3):
            for i in ([0, 2, 1, 4, 3] if rnd % 2 else [4, 1, 3, 0, 2]):
                m, n, k, dw, ds, dx, out, *_ = data[i]
                ops.matmul_int4g32(dw, ds, dx, out, m, n, k)
                assert np.array_equal(out.download(), first[i]), (rnd, i)
        st = Stream()
        m, n, k, dw, ds, dx, out, *_ = data[0]
        g = Graph.capture(st, lambda: [ops.matmul_int4g32(dw, ds, dx, out, m, n, k, stream=st) for _ in range(3)])
        for rep in range(4):
            out.upload(np.zeros((m, n), np.float32))
            g.launch(st)
            st.synchronize()
            assert np.array_equal(out.download(), first[0]), rep
            m1, n1, k1, dw1, ds1, dx1, out1, *_ = data[1 + rep % 4]
            ops.matmul_int4g32(dw1, ds1, dx1, out1, m1, n1, k1)
            assert np.array_equal(out1.download(), first[1 + rep % 4]), rep
        g.destroy()
        st.destroy()
    finally:
        ops.tune("int4_gemv.kernel", 0)
