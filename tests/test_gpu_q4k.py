"""GPU parity of the Q4_K dequant (bit-exact) and decode GEMV (rel-L2 <= 1e-3)
kernels against the CPU oracle, through the C ABI."""
import numpy as np
import pytest

from doe_amd import DeviceBuffer, DoeError, Graph, Stream, ops, q4k

pytestmark = pytest.mark.gpu

GEMV_REL_L2 = 1e-3  # north-star tolerance for GEMV outputs (fp32 accumulate)


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def _extreme_q4k(rng, n, k):
    """Random blocks whose d/dmin run over the whole f16 range incl. subnormals."""
    w = q4k.random_q4k(rng, n, k).reshape(-1, 144).copy()
    vals = np.array([2.0 ** -24, 1023 * 2.0 ** -24, 2.0 ** -14, 0.0123, 0.5, 3.0, 1000.0, 65504.0],
                    np.float16)
    d = vals[rng.integers(0, len(vals), w.shape[0])]
    dmin = vals[rng.integers(0, len(vals), w.shape[0])]
    w[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    w[:, 2:4] = dmin.view(np.uint8).reshape(-1, 2)
    return w.reshape(n, -1)


@pytest.mark.parametrize("n,k", [(1, 256), (7, 300), (33, 2304), (64, 9216), (5, 5376)])
def test_dequant_bit_exact(dev, ora, n, k):
    rng = np.random.default_rng(100 + n)
    w = _extreme_q4k(rng, n, k)
    dw = DeviceBuffer.from_array(w)
    out = DeviceBuffer.empty((n, k), np.float32)
    ops.dequant_q4k(dw, out, n, k)
    got = out.download()
    want = ora.q4k_dequant_rowwise(w, n, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_reference_tail_fixture(dev, known_answers):
    e = known_answers["q4k_rowwise_tail"]
    blocks = [q4k.pack_blocks(np.array([1.0]), np.array([0.0]), np.ones((1, 8)), np.zeros((1, 8)),
                              np.full((1, 256), f))[0] for f in e["block_quant_fill"]]
    raw = np.concatenate(blocks)
    rows, cols = e["shape"]
    out = DeviceBuffer.empty((rows, cols), np.float32)
    ops.dequant_q4k(DeviceBuffer.from_array(raw), out, rows, cols)
    want = np.concatenate([np.full(c, v, np.float32) for v, c in e["expected_runs"]])
    assert np.array_equal(out.download().reshape(-1), want)


def _gemv(w, x, n, k, stream=None):
    dw = DeviceBuffer.from_array(w)
    dx = DeviceBuffer.from_array(x.astype(np.float32))
    dy = DeviceBuffer.empty((n,), np.float32)
    ops.matmul_q4k(dw, dx, dy, n, k, stream)
    if stream is not None:
        stream.synchronize()
    return dy.download()


# config-0 shape, every 2B-class projection shape, 31B prefill K, tails
GEMV_SHAPES = [(9216, 2304), (2048, 2304), (1024, 2304), (2304, 2048), (2304, 9216),
               (21504 // 16, 5376), (1, 256), (3, 300), (37, 64 * 3 + 5), (1000, 1024),
               (100, 16384), (50, 12300)]


@pytest.mark.parametrize("n,k", GEMV_SHAPES)
def test_gemv_matches_oracle(dev, ora, n, k, gemv_kernel):
    if gemv_kernel == 1 and k > 12288:
        pytest.skip("past k ~ 12K the activation no longer fits the dot-product kernel's LDS; "
                    "the matrix-core kernel runs instead")
    rng = np.random.default_rng(n * 7 + k)
    w = q4k.random_q4k(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    got = _gemv(w, x, n, k)
    want = ora.q4k_gemv(w, x, n, k)
    err = rel_l2(got, want)
    print(f"[gemv {n}x{k}] rel_l2={err:.3e}", flush=True)
    assert err <= GEMV_REL_L2
    # The hi/lo activation split keeps the GEMV near f32 quality.
    assert err < 1e-5


def test_gemv_reference_block_one_hot(dev, known_answers, gemv_kernel):
    # The reference's known-answer block (test_doppler_rdrr_q4k.py:63-85)
    # through the GEMV: a one-hot activation picks out one dequantized value.
    e = known_answers["q4k_scale_min_block"]
    blk = q4k.pack_blocks(np.array([e["d"]]), np.array([e["dmin"]]), np.array([e["scale_bits"]]),
                          np.array([e["min_bits"]]), np.array([[i % 16 for i in range(256)]]))
    for idx, want in e["expected_values"].items():
        x = np.zeros(256, np.float32)
        x[int(idx)] = 1.0
        assert _gemv(blk, x, 1, 256)[0] == np.float32(want)


@pytest.mark.parametrize("scale", [1e-30, 1e-8, 1e6, 1e30])
def test_gemv_activation_range(dev, ora, scale, gemv_kernel):
    rng = np.random.default_rng(7)
    n, k = 256, 2304
    w = q4k.random_q4k(rng, n, k)
    x = (rng.standard_normal(k) * scale).astype(np.float32)
    assert rel_l2(_gemv(w, x, n, k), ora.q4k_gemv(w, x, n, k)) < 1e-5


def test_gemv_extreme_scales(dev, ora, gemv_kernel):
    rng = np.random.default_rng(8)
    n, k = 128, 1024
    w = _extreme_q4k(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    assert rel_l2(_gemv(w, x, n, k), ora.q4k_gemv(w, x, n, k)) < 1e-5


def test_gemv_zero_k_and_zero_n(dev):
    dy = DeviceBuffer.from_array(np.full(4, 7.0, np.float32))
    ops.matmul_q4k(DeviceBuffer(0), DeviceBuffer(0), dy, 4, 0)
    assert dy.download().tolist() == [0.0] * 4
    ops.matmul_q4k(DeviceBuffer(0), DeviceBuffer(16), DeviceBuffer(0), 0, 4)


def test_gemv_stream_and_graph_replays(dev, ora, gemv_kernel):
    rng = np.random.default_rng(9)
    n, k = 2048, 2304
    w = q4k.random_q4k(rng, n, k)
    dw = DeviceBuffer.from_array(w)
    dx = DeviceBuffer.empty((k,), np.float32)
    dy = DeviceBuffer.empty((n,), np.float32)
    s = Stream()
    g = Graph.capture(s, lambda: ops.matmul_q4k(dw, dx, dy, n, k, s))
    for rep in range(4):
        x = rng.standard_normal(k).astype(np.float32)
        dx.upload(x)
        g.launch(s)
        s.synchronize()
        assert rel_l2(dy.download(), ora.q4k_gemv(w, x, n, k)) < 1e-5, rep
    g.destroy()
    s.destroy()


def test_gemv_rejects_misaligned_weight(dev):
    dw = DeviceBuffer(144 * 2 + 16)
    dx = DeviceBuffer.empty((256,), np.float32)
    dy = DeviceBuffer.empty((2,), np.float32)
    import ctypes as C
    from doe_amd import _lib
    with pytest.raises(DoeError) as ei:
        _lib.call("doe_q4k_gemv", C.c_void_p(dw.ptr + 8), C.c_void_p(dx.ptr), C.c_void_p(dy.ptr), 2, 256,
                  C.c_void_p(None))
    assert ei.value.status == -1
    with pytest.raises(DoeError) as ei:
        _lib.call("doe_q4k_gemv", C.c_void_p(dw.ptr), C.c_void_p(dx.ptr), C.c_void_p(dy.ptr), 2, 70000,
                  C.c_void_p(None))
    assert ei.value.status == -4


def test_gemv_unaligned_activation(dev, ora, gemv_kernel):
    # an activation pointer that is 4-byte but not 16-byte aligned takes the
    # per-element load path
    import ctypes as C

    from doe_amd import _lib
    rng = np.random.default_rng(21)
    n, k = 100, 2304
    w = q4k.random_q4k(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    dx = DeviceBuffer.from_array(np.concatenate([np.zeros(1, np.float32), x]))
    dw = DeviceBuffer.from_array(w)
    dy = DeviceBuffer.empty((n,), np.float32)
    _lib.call("doe_q4k_gemv", C.c_void_p(dw.ptr), C.c_void_p(dx.ptr + 4), C.c_void_p(dy.ptr), n, k,
              C.c_void_p(None))
    assert rel_l2(dy.download(), ora.q4k_gemv(w, x, n, k)) < 1e-5


@pytest.mark.parametrize("n,k", [(2304, 9216), (37, 5376), (1000, 4352)])
def test_gemv_inplace_residual_k_split(dev, ora, n, k):
    # y <- y + W x with the output buffer as the residual: past 16 blocks and
    # below one 16-row group per CU the K range is split over workgroups whose
    # partial sums are added atomically; the unsplit kernel agrees
    rng = np.random.default_rng(k + n)
    w = q4k.random_q4k(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    r = rng.standard_normal(n).astype(np.float32)
    want = ora.q4k_gemv(w, x, n, k) + r.astype(np.float64)
    dw, dx = DeviceBuffer.from_array(w), DeviceBuffer.from_array(x)
    got = {}
    for split in (0, 1):
        ops.tune("q4k_gemv.ksplit", split)
        try:
            dy = DeviceBuffer.from_array(r)
            ops.matmul_q4k_fused(dw, dx, dy, n, k, residual=dy)
            got[split] = dy.download()
        finally:
            ops.tune("q4k_gemv.ksplit", 0)
        assert rel_l2(got[split], want) < 1e-5, split
    assert rel_l2(got[0], got[1]) < 1e-6


@pytest.mark.parametrize("k", [21504, 25600, 65536])
def test_gemv_large_k_splits(dev, ora, k):
    # past 64 Q4_K blocks per row the K ranges add into y: plain (y cleared),
    # residual into a separate output (y starts as the residual) and in place
    rng = np.random.default_rng(k)
    n = 333
    w = q4k.random_q4k(rng, n, k)
    x = rng.standard_normal(k, dtype=np.float32)
    r = rng.standard_normal(n, dtype=np.float32)
    want = ora.q4k_gemv(w, x, n, k)
    dw, dx = DeviceBuffer.from_array(w), DeviceBuffer.from_array(x)
    y = DeviceBuffer.from_array(np.full(n, 7.0, np.float32))  # stale contents are overwritten
    ops.matmul_q4k(dw, dx, y, n, k)
    assert rel_l2(y.download(), want) <= 1e-5
    res = DeviceBuffer.from_array(r)
    out = DeviceBuffer.from_array(np.full(n, -3.0, np.float32))
    ops.matmul_q4k_fused(dw, dx, out, n, k, residual=res)
    assert rel_l2(out.download(), want + r) <= 1e-5
    ops.matmul_q4k_fused(dw, dx, res, n, k, residual=res)  # in place
    assert rel_l2(res.download(), want + r) <= 1e-5
    # captured: the clear / residual copy replay with the GEMV
    s = Stream()
    g = Graph.capture(s, lambda: ops.matmul_q4k(dw, dx, y, n, k, s))
    for i in range(3):
        y.upload(np.full(n, float(i + 1), np.float32))
        g.launch(s)
        s.synchronize()
        assert rel_l2(y.download(), want) <= 1e-5, i
    g.destroy()
    s.destroy()
    with pytest.raises(DoeError, match="plain and residual"):
        ops.matmul_q4k_fused(dw, dx, out, n, k, norm_weight=DeviceBuffer.from_array(np.ones(k, np.float32)))


@pytest.fixture
def stream_groups(request, dev):
    """Forces the streaming GEMV kernel to walk `param` row groups per
    workgroup (q4k_gemv.stream) and restores the automatic choice."""
    ops.tune("q4k_gemv.stream", request.param)
    yield request.param
    ops.tune("q4k_gemv.stream", 0)


@pytest.mark.parametrize("stream_groups", [1, 2, 3, 7, 16], indirect=True)
@pytest.mark.parametrize("n,k", [(9216, 2304), (1000, 2304), (77, 300), (4096, 4096), (18432, 2304), (33, 256)])
def test_gemv_streaming_kernel(dev, ora, n, k, stream_groups):
    # the persistent streaming form: each workgroup walks `stream_groups` row
    # groups (the last one partial where n % 16 != 0), one wave per block
    print(f"[gemv stream {stream_groups}] {n}x{k}", flush=True)
    rng = np.random.default_rng(n + k + stream_groups)
    w = q4k.random_q4k(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    err = rel_l2(_gemv(w, x, n, k), ora.q4k_gemv(w, x, n, k))
    assert err < 1e-5, err


@pytest.mark.parametrize("n,k", [(40000, 2304), (65536, 2304), (70001, 512)])
def test_gemv_streaming_automatic(dev, ora, n, k):
    # the automatic choice streams from 8 row groups per CU (one persistent
    # workgroup per CU, up to 16 groups each; past that, several rounds)
    print(f"[gemv stream auto] {n}x{k}", flush=True)
    rng = np.random.default_rng(n + k)
    w = q4k.random_q4k(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    err = rel_l2(_gemv(w, x, n, k), ora.q4k_gemv(w, x, n, k))
    assert err < 1e-5, err


@pytest.mark.parametrize("stream_groups", [2, 5], indirect=True)
def test_gemv_streaming_fused_forms(dev, ora, stream_groups):
    # RMSNorm prologue, residual epilogue, gated epilogue and the RoPE + KV
    # cache epilogue through the streaming kernel
    rng = np.random.default_rng(40 + stream_groups)
    up = DeviceBuffer.from_array
    k = 2304
    x = (rng.standard_normal(k) * 3).astype(np.float32)
    nw = (0.1 * rng.standard_normal(k)).astype(np.float32)
    xn = ora.rmsnorm(x, nw, 1e-6, True)
    n = 3000
    w = q4k.random_q4k(rng, n, k)
    out = DeviceBuffer.empty((n,), np.float32)
    ops.matmul_q4k_fused(up(w), up(x), out, n, k, norm_weight=up(nw), norm_eps=1e-6, norm_weight_offset=True)
    assert rel_l2(out.download(), ora.q4k_gemv(w, xn, n, k)) < 1e-5
    res = rng.standard_normal(n).astype(np.float32)
    out2 = DeviceBuffer.empty((n,), np.float32)
    ops.matmul_q4k_fused(up(w), up(x), out2, n, k, residual=up(res))
    assert rel_l2(out2.download(), ora.residual(ora.q4k_gemv(w, x, n, k), res)) < 1e-5
    wg = q4k.random_q4k(rng, 2 * 1500, k)
    out3 = DeviceBuffer.empty((1500,), np.float32)
    ops.matmul_q4k_fused(up(wg), up(x), out3, 3000, k, norm_weight=up(nw), norm_eps=1e-6, gated=True)
    y = ora.q4k_gemv(wg, xn, 3000, k)
    assert rel_l2(out3.download(), ora.geglu(y[0::2], y[1::2])) < 1e-5
    # RoPE + cache write: 8 q / 4 kv heads of 256 at position 5
    hq, hkv, d, maxs, pos = 8, 4, 256, 16, 5
    qd, kd = hq * d, hkv * d
    nq = qd + 2 * kd
    w_plain = q4k.random_q4k(rng, nq, k).reshape(nq, -1)
    w_dev = w_plain.copy()
    w_dev[: qd + kd] = ops.interleave_rope_rows(w_plain[: qd + kd], d)
    table = ora.rope_table(maxs, d, 10000.0)
    kc = up(np.zeros((hkv, maxs, d), np.float16))
    vc = up(np.zeros((hkv, maxs, d), np.float16))
    out4 = DeviceBuffer.empty((nq,), np.float32)
    ops.qkv_rope_kv(up(w_dev), up(x), out4, hidden=k, num_heads=hq, num_kv_heads=hkv, head_dim=d,
                    freq_cis=up(table), position_buffer=up(np.array([pos], np.int32)), key_cache=kc,
                    val_cache=vc, max_seq_len=maxs, norm_weight=up(nw), norm_eps=1e-6, norm_weight_offset=True)
    qkv = ora.q4k_gemv(w_plain, xn, nq, k)
    qk = ora.rope(qkv[: qd + kd], table, 1, hq + hkv, d, pos)
    want = np.concatenate([ops.interleave_rope_rows(qk, d), qkv[qd + kd:]])
    assert rel_l2(out4.download(), want) < 1e-5
    kg = kc.download()
    assert rel_l2(kg[:, pos].astype(np.float32),
                  ops.interleave_rope_rows(qk[qd:], d).reshape(hkv, d).astype(np.float32)) < 1e-3


@pytest.mark.parametrize("stream_groups", [1, 3, 11], indirect=True)
@pytest.mark.parametrize("n,k", [(16384, 5376), (1000, 4352), (77, 5376), (4100, 5632)])
def test_gemv_streaming_two_blocks_per_wave(dev, ora, n, k, stream_groups):
    # rows of 17..22 Q4_K blocks: the streaming kernel with two blocks per
    # wave (the last wave's second block past the row where the count is odd)
    print(f"[gemv stream 2bpw {stream_groups}] {n}x{k}", flush=True)
    rng = np.random.default_rng(n + k + 7 * stream_groups)
    w = q4k.random_q4k(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    err = rel_l2(_gemv(w, x, n, k), ora.q4k_gemv(w, x, n, k))
    assert err < 1e-5, err


@pytest.mark.parametrize("form", ["norm_gated_parts", "rope_parts", "residual"])
def test_gemv_streaming_two_blocks_bit_identical_to_one_shot(dev, form):
    # the two-blocks-per-wave streaming kernel and the one-shot kernel sum
    # every block, wave and row in the same order: the same bits, with the
    # RMSNorm prologue and activation parts, the gated and RoPE / KV-cache
    # epilogues, and the residual
    from doe_amd.model import rope_table

    rng = np.random.default_rng(len(form))
    k = 5376
    up = DeviceBuffer.from_array
    x = up((rng.standard_normal(k) * 2).astype(np.float32))
    parts = up((rng.standard_normal((2, k)) * 0.5).astype(np.float32))
    nw = up((0.1 * rng.standard_normal(k)).astype(np.float32))
    outs = []
    for st in (3, -1):  # streaming (three row groups per workgroup), then never
        ops.tune("q4k_gemv.stream", st)
        try:
            if form == "norm_gated_parts":
                n = 4096
                w = up(q4k.random_q4k(np.random.default_rng(1), n, k))
                y = DeviceBuffer.empty((n // 2,), np.float32)
                ops.q4k_gemv_ex(w, n, k, activation=x, activation_parts=parts, activation_nparts=2, output=y,
                                norm_weight=nw, norm_eps=1e-6, gated=True)
                outs.append([y.download()])
            elif form == "rope_parts":
                hq, hkv, d, ms = 8, 4, 256, 16
                n = (hq + 2 * hkv) * d
                w = up(q4k.random_q4k(np.random.default_rng(2), n, k))
                y = DeviceBuffer.empty((n,), np.float32)
                kc = DeviceBuffer.from_array(np.zeros((hkv, ms, d), np.float16))
                vc = DeviceBuffer.from_array(np.zeros((hkv, ms, d), np.float16))
                r = dict(num_heads=hq, num_kv_heads=hkv, head_dim=d, freq_cis=up(rope_table(ms, d, 10000.0)),
                         position_buffer=up(np.array([7], np.int32)), key_cache=kc, val_cache=vc, max_seq_len=ms)
                ops.q4k_gemv_ex(w, n, k, activation=x, activation_parts=parts, activation_nparts=1, output=y,
                                norm_weight=nw, norm_eps=1e-6, rope=r)
                outs.append([y.download(), kc.download().view(np.uint16), vc.download().view(np.uint16)])
            else:
                n = 3000
                w = up(q4k.random_q4k(np.random.default_rng(3), n, k))
                res = up(np.random.default_rng(4).standard_normal(n).astype(np.float32))
                y = DeviceBuffer.empty((n,), np.float32)
                ops.q4k_gemv_ex(w, n, k, activation=x, output=y, residual=res)
                outs.append([y.download()])
        finally:
            ops.tune("q4k_gemv.stream", 0)
    dev.synchronize()
    for a, b in zip(*outs):
        assert np.array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                              b.view(np.uint32) if b.dtype == np.float32 else b)


def test_gemv_streaming_two_blocks_automatic(dev, ora):
    # the 31B-class gate/up shape (43008 x 5376, 2688 row groups): streamed
    # automatically with two blocks per wave
    n, k = 43008, 5376
    rng = np.random.default_rng(43)
    w = q4k.random_q4k(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    err = rel_l2(_gemv(w, x, n, k), ora.q4k_gemv(w, x, n, k))
    assert err < 1e-5, err
