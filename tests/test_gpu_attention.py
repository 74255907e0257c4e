"""GPU parity of GQA decode attention (f16 KV cache) against the CPU oracle,
through the C ABI.  Tolerance: rel-L2 <= 1e-3 (fp32 accumulate)."""
import math
from pathlib import Path

import numpy as np
import pytest

from doe_amd import DeviceBuffer, DoeError, Graph, Stream, ops

pytestmark = pytest.mark.gpu

ATTN_REL_L2 = 1e-3


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def run_attn(q, k, v, *, hq, hkv, d, kv_len, kv_stride, scale, q_f16, out_f16, softcap=0.0, window=0,
             layout=0, batch=1, kv_len_buffer=None, stream=None):
    dq = DeviceBuffer.from_array(q)
    dk = DeviceBuffer.from_array(k)
    dv = DeviceBuffer.from_array(v)
    out = DeviceBuffer.empty((batch, hq, d), np.float16 if out_f16 else np.float32)
    ops.attention(dq, dk, dv, out, batch=batch, num_heads=hq, num_kv_heads=hkv, head_dim=d, kv_len=kv_len,
                  kv_stride=kv_stride, scale=scale, q_f16=q_f16, out_f16=out_f16, softcap=softcap,
                  sliding_window=window, kv_layout=layout, kv_len_buffer=kv_len_buffer, stream=stream)
    return out.download().astype(np.float32)


def oracle_attn(ora, q, k, v, *, batch, hq, hkv, d, kv_len, kv_stride, scale, softcap=0.0, window=0,
                layout=0):
    outs = []
    for b in range(batch):
        outs.append(ora.attn_decode(q[b].astype(np.float32), k[b], v[b], hq, hkv, d, kv_len, kv_stride, scale,
                                    softcap, window, layout))
    return np.stack(outs)


def test_config1_gqa_decode(dev, ora):
    # 8 query / 4 KV heads, head_dim 256, context 4096, f16 Q/K/V N(0,1),
    # scale 1/16, f16 output; KV cache [kv_head][pos][dim].
    rng = np.random.default_rng(1)
    hq, hkv, d, t = 8, 4, 256, 4096
    q = rng.standard_normal((1, hq, d)).astype(np.float16)
    k = rng.standard_normal((1, hkv, t, d)).astype(np.float16)
    v = rng.standard_normal((1, hkv, t, d)).astype(np.float16)
    got = run_attn(q, k, v, hq=hq, hkv=hkv, d=d, kv_len=t, kv_stride=t, scale=1 / 16, q_f16=True, out_f16=True)
    want = oracle_attn(ora, q, k, v, batch=1, hq=hq, hkv=hkv, d=d, kv_len=t, kv_stride=t, scale=1 / 16)
    err = rel_l2(got, want)
    print(f"[attn cfg1] rel_l2={err:.3e}", flush=True)
    assert err <= ATTN_REL_L2


@pytest.mark.parametrize("d", [64, 128, 160, 256, 512])
@pytest.mark.parametrize("g", [1, 2, 4, 8])
def test_head_dims_and_groups(dev, ora, d, g):
    # (head_dim 512 with more than two query heads per kv head runs as g / 2
    # workgroups per kv head)
    rng = np.random.default_rng(d + g)
    hkv = 2
    hq = hkv * g
    t, stride, batch = 300, 320, 2
    q = rng.standard_normal((batch, hq, d)).astype(np.float32)
    k = rng.standard_normal((batch, hkv, stride, d)).astype(np.float16)
    v = rng.standard_normal((batch, hkv, stride, d)).astype(np.float16)
    scale = 1 / math.sqrt(d)
    got = run_attn(q, k, v, hq=hq, hkv=hkv, d=d, kv_len=t, kv_stride=stride, scale=scale, q_f16=False,
                   out_f16=False, batch=batch)
    want = oracle_attn(ora, q, k, v, batch=batch, hq=hq, hkv=hkv, d=d, kv_len=t, kv_stride=stride, scale=scale)
    assert rel_l2(got, want) <= 1e-5  # f32 query (hi/lo split), f32 output


def test_head512_global_layer_shape(dev, ora):
    # a 512-wide global attention layer: 8 query heads on one kv head, the
    # [pos][kv_head][dim] layout, a score softcap and a sliding window
    rng = np.random.default_rng(512)
    hq, hkv, d, t, stride = 8, 1, 512, 700, 768
    q = rng.standard_normal((1, hq, d)).astype(np.float32)
    k = rng.standard_normal((1, stride, hkv, d)).astype(np.float16)
    v = rng.standard_normal((1, stride, hkv, d)).astype(np.float16)
    for softcap, window in ((0.0, 0), (50.0, 0), (0.0, 256)):
        got = run_attn(q, k, v, hq=hq, hkv=hkv, d=d, kv_len=t, kv_stride=stride, scale=1 / 16, q_f16=False,
                       out_f16=False, softcap=softcap, window=window, layout=1)
        want = oracle_attn(ora, q, k, v, batch=1, hq=hq, hkv=hkv, d=d, kv_len=t, kv_stride=stride, scale=1 / 16,
                           softcap=softcap, window=window, layout=1)
        assert rel_l2(got, want) <= 1e-5, (softcap, window)


@pytest.mark.parametrize("t", [1, 15, 16, 17, 63, 64, 65, 1000])
def test_ragged_lengths(dev, ora, t):
    rng = np.random.default_rng(t)
    hq, hkv, d, stride = 4, 2, 128, 1024
    q = rng.standard_normal((1, hq, d)).astype(np.float32)
    k = rng.standard_normal((1, hkv, stride, d)).astype(np.float16)
    v = rng.standard_normal((1, hkv, stride, d)).astype(np.float16)
    got = run_attn(q, k, v, hq=hq, hkv=hkv, d=d, kv_len=t, kv_stride=stride, scale=0.1, q_f16=False, out_f16=False)
    want = oracle_attn(ora, q, k, v, batch=1, hq=hq, hkv=hkv, d=d, kv_len=t, kv_stride=stride, scale=0.1)
    assert rel_l2(got, want) <= 1e-5
    if t == 1:  # a single key returns its value row
        assert np.allclose(got[0, 0], v[0, 0, 0].astype(np.float32), atol=1e-6)


def test_layout1_window_softcap(dev, ora):
    rng = np.random.default_rng(5)
    hq, hkv, d, t = 8, 4, 256, 777
    q = rng.standard_normal((1, hq, d)).astype(np.float32)
    k0 = rng.standard_normal((1, hkv, t, d)).astype(np.float16)
    v0 = rng.standard_normal((1, hkv, t, d)).astype(np.float16)
    k1 = np.ascontiguousarray(k0.transpose(0, 2, 1, 3))
    v1 = np.ascontiguousarray(v0.transpose(0, 2, 1, 3))
    for window, cap in [(0, 0.0), (100, 0.0), (0, 2.0), (50, 1.5)]:
        want = oracle_attn(ora, q, k0, v0, batch=1, hq=hq, hkv=hkv, d=d, kv_len=t, kv_stride=t, scale=0.0625,
                           softcap=cap, window=window)
        g0 = run_attn(q, k0, v0, hq=hq, hkv=hkv, d=d, kv_len=t, kv_stride=t, scale=0.0625, q_f16=False,
                      out_f16=False, softcap=cap, window=window, layout=0)
        g1 = run_attn(q, k1, v1, hq=hq, hkv=hkv, d=d, kv_len=t, kv_stride=t, scale=0.0625, q_f16=False,
                      out_f16=False, softcap=cap, window=window, layout=1)
        assert rel_l2(g0, want) <= 1e-5, (window, cap)
        assert rel_l2(g1, want) <= 1e-5, (window, cap)


def test_split_count_does_not_change_the_result(dev, ora):
    rng = np.random.default_rng(6)
    hq, hkv, d, t = 8, 4, 256, 4096
    q = rng.standard_normal((1, hq, d)).astype(np.float32)
    k = rng.standard_normal((1, hkv, t, d)).astype(np.float16)
    v = rng.standard_normal((1, hkv, t, d)).astype(np.float16)
    want = oracle_attn(ora, q, k, v, batch=1, hq=hq, hkv=hkv, d=d, kv_len=t, kv_stride=t, scale=1 / 16)
    try:
        for splits in (1, 2, 7, 64, 256):
            ops.tune("attn_decode.splits", splits)
            for rep in range(2):  # the split counters must be back at zero
                got = run_attn(q, k, v, hq=hq, hkv=hkv, d=d, kv_len=t, kv_stride=t, scale=1 / 16, q_f16=False,
                               out_f16=False)
                assert rel_l2(got, want) <= 1e-5, (splits, rep)
    finally:
        ops.tune("attn_decode.splits", 0)


def test_device_kv_len_graph_replays(dev, ora):
    # The decode loop captures attention once and replays it as the cache
    # grows: the length comes from a device int32 (kv_len_source = 1).
    rng = np.random.default_rng(7)
    hq, hkv, d, stride = 8, 4, 256, 2048
    q = rng.standard_normal((1, hq, d)).astype(np.float32)
    k = rng.standard_normal((1, hkv, stride, d)).astype(np.float16)
    v = rng.standard_normal((1, hkv, stride, d)).astype(np.float16)
    dq, dk, dv = DeviceBuffer.from_array(q), DeviceBuffer.from_array(k), DeviceBuffer.from_array(v)
    out = DeviceBuffer.empty((1, hq, d), np.float32)
    klen = DeviceBuffer.from_array(np.array([1], np.int32))
    s = Stream()
    g = Graph.capture(s, lambda: ops.attention(dq, dk, dv, out, batch=1, num_heads=hq, num_kv_heads=hkv,
                                               head_dim=d, kv_len=0, kv_stride=stride, scale=1 / 16,
                                               kv_len_buffer=klen, stream=s))
    for t in (1, 17, 500, 2048, 129):
        klen.upload(np.array([t], np.int32))
        g.launch(s)
        s.synchronize()
        want = oracle_attn(ora, q, k, v, batch=1, hq=hq, hkv=hkv, d=d, kv_len=t, kv_stride=stride, scale=1 / 16)
        assert rel_l2(out.download(), want) <= 1e-5, t
    g.destroy()
    s.destroy()


def test_empty_cache_gives_zeros(dev):
    hq, hkv, d = 2, 1, 64
    q = np.ones((1, hq, d), np.float32)
    k = np.ones((1, hkv, 16, d), np.float16)
    got = run_attn(q, k, k, hq=hq, hkv=hkv, d=d, kv_len=0, kv_stride=16, scale=1.0, q_f16=False, out_f16=False)
    assert not got.any()


def test_rejects_bad_shapes(dev):
    from doe_amd import DoeError
    q = DeviceBuffer.empty((1, 3, 64), np.float32)
    kv = DeviceBuffer.empty((1, 1, 16, 64), np.float16)
    with pytest.raises(DoeError):  # 3 query heads per kv head is not supported
        ops.attention(q, kv, kv, q, batch=1, num_heads=3, num_kv_heads=1, head_dim=64, kv_len=16, kv_stride=16,
                      scale=1.0)
    with pytest.raises(ValueError):
        ops.attention(q, kv, kv, q, batch=1, num_heads=3, num_kv_heads=2, head_dim=64, kv_len=16, kv_stride=16,
                      scale=1.0)
    with pytest.raises(ValueError):
        ops.attention(q, kv, kv, q, batch=1, num_heads=1, num_kv_heads=1, head_dim=64, kv_len=17, kv_stride=16,
                      scale=1.0)


def test_workspace_reuse_after_larger_call(dev, ora):
    # Regression: a large multi-split call followed by a smaller one must still
    # find the split counters at zero.
    rng = np.random.default_rng(8)
    for hq, hkv, d, t, batch in [(8, 4, 256, 4096, 2), (2, 2, 64, 300, 1), (8, 4, 256, 2000, 1)]:
        q = rng.standard_normal((batch, hq, d)).astype(np.float32)
        k = rng.standard_normal((batch, hkv, t, d)).astype(np.float16)
        v = rng.standard_normal((batch, hkv, t, d)).astype(np.float16)
        got = run_attn(q, k, v, hq=hq, hkv=hkv, d=d, kv_len=t, kv_stride=t, scale=0.05, q_f16=False,
                       out_f16=False, batch=batch)
        want = oracle_attn(ora, q, k, v, batch=batch, hq=hq, hkv=hkv, d=d, kv_len=t, kv_stride=t, scale=0.05)
        assert rel_l2(got, want) <= 1e-5, (hq, hkv, d, t, batch)


def test_config4_batch8_long_context(dev, ora):
    # the 27B-class long-context decode: batch 8, 64 query / 8 KV heads,
    # head_dim 128, 32768 cached positions per sequence (1 GiB of f16 K/V),
    # generated on the device; oracle on the first and last sequence
    import ctypes as C

    from doe_amd import _lib
    b, hq, hkv, d, t = 8, 64, 8, 128, 32768
    k = DeviceBuffer.empty((b, hkv, t, d), np.float16)
    v = DeviceBuffer.empty((b, hkv, t, d), np.float16)
    _lib.call("doe_fill_normal_f16", C.c_void_p(k.ptr), k.nbytes // 2, 41, 0.0, 1.0, C.c_void_p(None))
    _lib.call("doe_fill_normal_f16", C.c_void_p(v.ptr), v.nbytes // 2, 42, 0.0, 1.0, C.c_void_p(None))
    rng = np.random.default_rng(43)
    q = rng.standard_normal((b, hq, d)).astype(np.float16)
    out = DeviceBuffer.empty((b, hq, d), np.float16)
    scale = 1 / math.sqrt(d)
    ops.attention(DeviceBuffer.from_array(q), k, v, out, batch=b, num_heads=hq, num_kv_heads=hkv, head_dim=d,
                  kv_len=t, kv_stride=t, scale=scale, q_f16=True, out_f16=True)
    got = out.download().astype(np.float32)
    assert np.isfinite(got).all()
    seq_bytes = hkv * t * d * 2
    for sb in (0, b - 1):
        kk = np.empty((hkv, t, d), np.float16)
        vv = np.empty((hkv, t, d), np.float16)
        _lib.call("doe_memcpy_d2h", kk.ctypes.data_as(C.c_void_p), C.c_void_p(k.ptr + sb * seq_bytes), seq_bytes)
        _lib.call("doe_memcpy_d2h", vv.ctypes.data_as(C.c_void_p), C.c_void_p(v.ptr + sb * seq_bytes), seq_bytes)
        want = ora.attn_decode(q[sb].astype(np.float32), kk, vv, hq, hkv, d, t, t, scale)
        err = rel_l2(got[sb], want)
        print(f"[attn cfg4] seq {sb} rel_l2={err:.3e}", flush=True)
        assert err <= ATTN_REL_L2
    k.free()
    v.free()


@pytest.mark.parametrize("waves", [4, 16])
@pytest.mark.parametrize("d,g", [(64, 8), (128, 4), (256, 2), (256, 1)])
def test_wide_and_narrow_workgroups_agree_with_oracle(dev, ora, waves, d, g):
    # short contexts run as one split on a wide workgroup (16 waves, 8 at
    # head_dim 256); forcing the 4-wave split path must give the same answer
    from doe_amd import _lib
    rng = np.random.default_rng(d * 10 + g + waves)
    hkv, t, stride, batch = 2, 333, 384, 2
    hq = hkv * g
    q = rng.standard_normal((batch, hq, d)).astype(np.float32)
    k = rng.standard_normal((batch, hkv, stride, d)).astype(np.float16)
    v = rng.standard_normal((batch, hkv, stride, d)).astype(np.float16)
    scale = 1 / math.sqrt(d)
    _lib.call("doe_tune_set", b"attn_decode.waves", waves)
    try:
        got = run_attn(q, k, v, hq=hq, hkv=hkv, d=d, kv_len=t, kv_stride=stride, scale=scale, q_f16=False,
                       out_f16=False, batch=batch)
    finally:
        _lib.call("doe_tune_set", b"attn_decode.waves", 0)
    want = oracle_attn(ora, q, k, v, batch=batch, hq=hq, hkv=hkv, d=d, kv_len=t, kv_stride=stride, scale=scale)
    assert rel_l2(got, want) <= 1e-5


def _dispatch(q, kc, vc, *, cap, page_table=None, kv_len_buffer=None, **uni):
    """doe_attention_dispatch on host arrays: q f32 [hq][d], K/V f16 [cap][hkv][d]."""
    out = DeviceBuffer.empty((uni["num_heads"], uni["head_dim"]), np.float32)
    ops.attention_dispatch(DeviceBuffer.from_array(q), DeviceBuffer.from_array(kc), DeviceBuffer.from_array(vc),
                           out, kv_capacity=cap,
                           page_table=None if page_table is None else DeviceBuffer.from_array(page_table),
                           kv_len_buffer=kv_len_buffer, **uni)
    return out.download()


def test_reference_dispatch_cache_addressing(dev, ora):
    # The reference attention's own Uniforms and bindings (decode form).  Its
    # cache addressing is pinned by storage invariants: a paged cache (rows
    # scattered over pages by a random page table), a ring of the last
    # `window` rows and a kv_start offset each hold the same keys as a
    # contiguous cache, so they give the same output; the contiguous form
    # matches doe_attn_decode and the oracle.
    rng = np.random.default_rng(21)
    hq, hkv, d, L, ps = 8, 2, 128, 300, 32
    q = rng.standard_normal((hq, d)).astype(np.float32)
    kc = rng.standard_normal((L, hkv, d)).astype(np.float16)
    vc = rng.standard_normal((L, hkv, d)).astype(np.float16)
    base = dict(num_heads=hq, num_kv_heads=hkv, head_dim=d, seq_len=L, scale=1 / math.sqrt(d), is_causal=1,
                start_pos=L - 1)
    ref = _dispatch(q, kc, vc, cap=L, **base)
    want = oracle_attn(ora, q[None], kc[None], vc[None], batch=1, hq=hq, hkv=hkv, d=d, kv_len=L, kv_stride=L,
                       scale=1 / math.sqrt(d), layout=1)[0]
    assert rel_l2(ref, want) <= 1e-5
    same = run_attn(q[None], kc[None], vc[None], hq=hq, hkv=hkv, d=d, kv_len=L, kv_stride=L, scale=1 / math.sqrt(d),
                    q_f16=False, out_f16=False, layout=1)[0]
    assert rel_l2(ref, same) <= 1e-6
    # paged: logical page p lives in physical page perm[p] of a larger pool
    npg = -(-L // ps)
    perm = rng.permutation(npg + 5)[:npg].astype(np.uint32)
    pool_k = rng.standard_normal(((npg + 5) * ps, hkv, d)).astype(np.float16)
    pool_v = rng.standard_normal(((npg + 5) * ps, hkv, d)).astype(np.float16)
    for pg in range(npg):
        n = min(ps, L - pg * ps)
        pool_k[perm[pg] * ps:perm[pg] * ps + n] = kc[pg * ps:pg * ps + n]
        pool_v[perm[pg] * ps:perm[pg] * ps + n] = vc[pg * ps:pg * ps + n]
    paged = _dispatch(q, pool_k, pool_v, cap=(npg + 5) * ps, page_table=perm, kv_layout=2, page_size=ps, **base)
    assert rel_l2(paged, ref) <= 1e-6
    # kv_start: the same keys stored 40 rows further in
    shift_k = np.concatenate([rng.standard_normal((40, hkv, d)).astype(np.float16), kc])
    shift_v = np.concatenate([rng.standard_normal((40, hkv, d)).astype(np.float16), vc])
    shifted = _dispatch(q, shift_k, shift_v, cap=L + 40, **{**base, "kv_start": 40, "start_pos": L - 1 + 40})
    assert rel_l2(shifted, ref) <= 1e-6
    # ring of the last W rows at (abs % W) == contiguous with a W-key window
    W = 64
    ring_k = np.zeros((W, hkv, d), np.float16)
    ring_v = np.zeros((W, hkv, d), np.float16)
    for pos in range(L - W, L):
        ring_k[pos % W], ring_v[pos % W] = kc[pos], vc[pos]
    ring = _dispatch(q, ring_k, ring_v, cap=W, kv_layout=1, **{**base, "sliding_window": W})
    windowed = _dispatch(q, kc, vc, cap=L, **{**base, "sliding_window": W})
    assert rel_l2(ring, windowed) <= 1e-6
    assert rel_l2(windowed, ref) > 1e-3
    # causal at an earlier query position == a cache holding only keys <= it
    early = _dispatch(q, kc, vc, cap=L, **{**base, "start_pos": 100})
    short = _dispatch(q, kc[:101].copy(), vc[:101].copy(), cap=101, **{**base, "seq_len": 101, "start_pos": 100})
    assert rel_l2(early, short) <= 1e-6
    # the length from the device buffer (kv_len_source 1)
    klen = DeviceBuffer.from_array(np.array([L], np.uint32))
    dev_len = _dispatch(q, kc, vc, cap=L, kv_len_buffer=klen, **{**base, "seq_len": 0, "kv_len_source": 1})
    assert rel_l2(dev_len, ref) <= 1e-6
    # page table entries past the pool are clamped into it: finite output, no fault
    bad = perm.copy()
    bad[0] = 1 << 20
    clamped = _dispatch(q, pool_k, pool_v, cap=(npg + 5) * ps, page_table=bad, kv_layout=2, page_size=ps, **base)
    assert np.isfinite(clamped).all()


def test_reference_dispatch_rejects_unsupported(dev):
    buf = DeviceBuffer(1 << 16)
    kw = dict(num_heads=2, num_kv_heads=1, head_dim=64, seq_len=4, scale=1.0, is_causal=1, start_pos=3)
    # several queries run the multi-query kernel, whose head widths are 64 .. 512
    with pytest.raises(DoeError, match="head_dim"):
        ops.attention_dispatch(buf, buf, buf, buf, kv_capacity=8, **{**kw, "query_len": 4, "head_dim": 96})
    with pytest.raises(DoeError, match="kv_layout"):
        ops.attention_dispatch(buf, buf, buf, buf, kv_capacity=8, kv_layout=3, **kw)
    with pytest.raises(DoeError, match="page"):
        ops.attention_dispatch(buf, buf, buf, buf, kv_capacity=8, kv_layout=2, **kw)
    with pytest.raises(DoeError, match="kv_len_buffer"):
        ops.attention_dispatch(buf, buf, buf, buf, kv_capacity=8, kv_len_source=1, **kw)


@pytest.mark.parametrize("splits", [2, 7, 33, 64, 100])
@pytest.mark.parametrize("d,out_f16", [(256, True), (128, False), (64, True), (512, False), (160, False)])
def test_split_combine_kernels(dev, ora, splits, d, out_f16):
    # the one-wave-per-column combine (up to 64 splits, lanes over splits)
    # and the block-reduction combine (any count; forced, and automatic past
    # 64) against the oracle and each other, with empty splits at the end
    # (kv_len not a multiple of the split size)
    rng = np.random.default_rng(splits + d)
    hq, hkv, t = 4, 2, 16 * splits * 4 + 16 * 3
    kv_len = t - 37
    q = rng.standard_normal((1, hq, d)).astype(np.float16)
    k = rng.standard_normal((1, hkv, t, d)).astype(np.float16)
    v = rng.standard_normal((1, hkv, t, d)).astype(np.float16)
    want = oracle_attn(ora, q, k, v, batch=1, hq=hq, hkv=hkv, d=d, kv_len=kv_len, kv_stride=t, scale=d ** -0.5)
    outs = []
    ops.tune("attn_decode.splits", splits)
    try:
        for combine in (0, 1):
            ops.tune("attn_decode.combine", combine)
            outs.append(run_attn(q, k, v, hq=hq, hkv=hkv, d=d, kv_len=kv_len, kv_stride=t, scale=d ** -0.5,
                                 q_f16=True, out_f16=out_f16))
    finally:
        ops.tune("attn_decode.combine", 0)
        ops.tune("attn_decode.splits", 0)
    for got in outs:
        assert rel_l2(got, want) <= ATTN_REL_L2
    assert rel_l2(outs[0], outs[1]) <= (1e-3 if out_f16 else 1e-6)


def test_head160_sliding_layout1_kv_len_device(dev, ora):
    # head_dim 160 (Gemma 4 31B smoke graph: 32 heads x 160): the
    # [pos][kv_head][dim] layout, a sliding window, a device kv_len and a
    # softcap, f16 query and output
    from doe_amd import DeviceBuffer

    rng = np.random.default_rng(160)
    hq, hkv, d, t, stride = 32, 32, 160, 900, 1024
    q = rng.standard_normal((1, hq, d)).astype(np.float16)
    k = rng.standard_normal((1, stride, hkv, d)).astype(np.float16)
    v = rng.standard_normal((1, stride, hkv, d)).astype(np.float16)
    klen = DeviceBuffer.from_array(np.array([t], np.int32))
    for softcap, window in ((0.0, 512), (30.0, 0)):
        got = run_attn(q, k, v, hq=hq, hkv=hkv, d=d, kv_len=0, kv_stride=stride, scale=d ** -0.5, q_f16=True,
                       out_f16=True, softcap=softcap, window=window, layout=1, kv_len_buffer=klen)
        want = oracle_attn(ora, q, k, v, batch=1, hq=hq, hkv=hkv, d=d, kv_len=t, kv_stride=stride, scale=d ** -0.5,
                           softcap=softcap, window=window, layout=1)
        assert rel_l2(got, want) <= ATTN_REL_L2, (softcap, window)


def test_qwen36_partial_rope_gqa6_attention_on_real_activations(dev, ora):
    # Qwen 3.6 27B layer 3 (tests/golden/qwen36_layer3_attention.npz, the
    # reference's frozen Doppler activations): doe_rope_partial over the first
    # 64 of 256 dims (theta 1e7), doe_kv_write into an f16 cache, then decode
    # attention per prompt position with six query heads on one KV head.
    # Against the oracle on the same steps within 1e-5; against the
    # reference run's output (computed in f16) within 3e-3, where the oracle
    # itself sits (tests/test_oracle_qwen_attention.py).
    from doe_amd.model import rope_table

    from test_oracle_qwen_attention import D, G, ROT, T, THETA, oracle_attention, rel

    with np.load(Path(__file__).parent / "golden" / "qwen36_layer3_attention.npz", allow_pickle=False) as z:
        fx = {k: z[k].astype(np.float32) for k in z.files}
    tab = DeviceBuffer.from_array(rope_table(T, ROT, THETA))
    q = DeviceBuffer.from_array(fx["q"])
    k = DeviceBuffer.from_array(fx["k"])
    v = DeviceBuffer.from_array(fx["v"])
    ops.rope_partial(q, tab, T, G, D, ROT)
    ops.rope_partial(k, tab, T, 1, D, ROT)
    kc = DeviceBuffer.empty((1, T, D), np.float16)
    vc = DeviceBuffer.empty((1, T, D), np.float16)
    out = DeviceBuffer.empty((T, G, D), np.float32)
    for t in range(T):
        ops.kv_write(k.view(t * D * 4, D * 4, np.float32), v.view(t * D * 4, D * 4, np.float32), kc, vc, 1, T, D,
                     position=t)
        ops.attention(q.view(t * G * D * 4, G * D * 4, np.float32), kc, vc,
                      out.view(t * G * D * 4, G * D * 4, np.float32), batch=1, num_heads=G, num_kv_heads=1,
                      head_dim=D, kv_len=t + 1, kv_stride=T, scale=1.0 / 16)
    got = out.download().reshape(T, G, D)
    want = oracle_attention(ora, fx, ROT)
    e_oracle, e_run = rel(got, want), rel(got, fx["out"])
    print(f"[qwen36 layer 3] vs oracle {e_oracle:.1e}, vs reference run {e_run:.1e}", flush=True)
    assert e_oracle <= 1e-5
    assert e_run <= 3e-3
