"""GPU parity of the Q8_0 GEMV (doe_q8_0_gemv) against the CPU oracle's f32
left-fold (ora_q8_0_gemv), through the C ABI.  Contract: rel-L2 <= 1e-3.
Shapes cover one-block rows, ragged tails, odd block counts (rows that start
2 bytes off a dword), the 1-, 2- and 4-row wave groups, more groups than the
persistent grid and the largest k; plus residuals, empty reductions, extreme
quants and the argument checks."""
import ctypes as C

import numpy as np
import pytest

from doe_amd import DeviceBuffer, DoeError, Graph, Stream, _lib, ops, q8_0

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


@pytest.mark.parametrize("n,k", [(1, 32), (3, 40), (5, 1000), (64, 2048), (2304, 2304), (9216, 2304),
                                 (2304, 9216), (5000, 96), (10000, 320), (65539, 256), (64, 32768),
                                 (7, 32767), (130, 7)])
def test_q8_0_gemv_matches_oracle(dev, ora, n, k):
    print(f"q8_0_gemv n={n} k={k}", flush=True)
    rng = np.random.default_rng(n * 7 + k)
    w = q8_0.random_q8_0(rng, n, k)
    x = rng.standard_normal(k, dtype=np.float32)
    out = DeviceBuffer.empty((n,), np.float32)
    ops.matmul_q8_0(DeviceBuffer.from_array(w), DeviceBuffer.from_array(x), out, n, k)
    err = rel_l2(out.download(), ora.q8_0_gemv(w, x, n, k))
    assert err <= 1e-3, err
    assert err <= 1e-5, err  # f32 sums of exact products: ~1e-7 expected


@pytest.mark.parametrize("rows,depth", [(1, 1), (1, 2), (2, 1), (2, 2), (4, 1), (4, 2)])
def test_q8_0_gemv_every_variant(dev, ora, rows, depth):
    # wave groups of 1, 2 or 4 rows, one or two units loaded ahead
    rng = np.random.default_rng(rows * 10 + depth)
    try:
        ops.tune("q8_0_gemv.rows", rows)
        ops.tune("q8_0_gemv.depth", depth)
        for n, k in ((777, 1000), (70, 3000), (9, 33)):
            w = q8_0.random_q8_0(rng, n, k)
            x = rng.standard_normal(k, dtype=np.float32)
            r = rng.standard_normal(n, dtype=np.float32)
            out = DeviceBuffer.empty((n,), np.float32)
            ops.matmul_q8_0(DeviceBuffer.from_array(w), DeviceBuffer.from_array(x), out, n, k,
                            residual=DeviceBuffer.from_array(r))
            assert rel_l2(out.download(), ora.q8_0_gemv(w, x, n, k, residual=r)) <= 1e-5, (n, k)
    finally:
        ops.tune("q8_0_gemv.rows", 0)
        ops.tune("q8_0_gemv.depth", 0)


@pytest.mark.parametrize("n,k,offset", [(4096, 2304, True), (300, 1000, False), (9, 33, True)])
def test_q8_0_gemv_with_rmsnorm(dev, ora, n, k, offset):
    # the input_norm / post_attn_norm step folded in: oracle rmsnorm, then the GEMV
    rng = np.random.default_rng(n + k)
    w = q8_0.random_q8_0(rng, n, k)
    x = (rng.standard_normal(k) * 3).astype(np.float32)
    nw = (rng.standard_normal(k) * 0.1).astype(np.float32)
    r = rng.standard_normal(n, dtype=np.float32)
    want = ora.q8_0_gemv(w, ora.rmsnorm(x, nw, 1e-6, offset), n, k, residual=r)
    out = DeviceBuffer.from_array(r)
    ops.matmul_q8_0(DeviceBuffer.from_array(w), DeviceBuffer.from_array(x), out, n, k, residual=out,
                    norm_weight=DeviceBuffer.from_array(nw), norm_eps=1e-6, norm_weight_offset=offset)
    assert rel_l2(out.download(), want) <= 1e-5


def test_q8_0_gemv_residual_in_place_and_separate(dev, ora):
    rng = np.random.default_rng(11)
    n, k = 3000, 544
    w = q8_0.random_q8_0(rng, n, k)
    x = rng.standard_normal(k, dtype=np.float32)
    r = rng.standard_normal(n, dtype=np.float32)
    want = ora.q8_0_gemv(w, x, n, k, residual=r)
    dw, dx = DeviceBuffer.from_array(w), DeviceBuffer.from_array(x)
    dr = DeviceBuffer.from_array(r)
    out = DeviceBuffer.empty((n,), np.float32)
    ops.matmul_q8_0(dw, dx, out, n, k, residual=dr)
    assert rel_l2(out.download(), want) <= 1e-5
    ops.matmul_q8_0(dw, dx, dr, n, k, residual=dr)  # y += W x in place
    assert rel_l2(dr.download(), want) <= 1e-5


def test_q8_0_gemv_extreme_quants_and_negative_scales(dev, ora):
    rng = np.random.default_rng(12)
    n, k = 256, 1024
    nb = k // 32
    q = rng.choice(np.array([-128, 127, -1, 0]), (n, nb, 32))
    d = rng.choice(np.array([-2.0, 0.5, -6.1e-5, 1024.0]), (n, nb))
    w = q8_0.pack_rows(d, q)
    x = (rng.standard_normal(k) * 100).astype(np.float32)
    out = DeviceBuffer.empty((n,), np.float32)
    ops.matmul_q8_0(DeviceBuffer.from_array(w), DeviceBuffer.from_array(x), out, n, k)
    assert rel_l2(out.download(), ora.q8_0_gemv(w, x, n, k)) <= 1e-5


def test_q8_0_gemv_empty_reduction(dev):
    n = 100
    r = np.arange(n, dtype=np.float32)
    out = DeviceBuffer.from_array(np.full(n, 7.0, np.float32))
    dr = DeviceBuffer.from_array(r)
    # no weights or activation are read at k = 0
    _lib.call("doe_q8_0_gemv", None, None, C.c_void_p(out.ptr), n, 0, None, None)
    assert not out.download().any()
    _lib.call("doe_q8_0_gemv", None, None, C.c_void_p(out.ptr), n, 0, C.c_void_p(dr.ptr), None)
    assert np.array_equal(out.download(), r)


def test_q8_0_gemv_graph_replays(dev, ora):
    rng = np.random.default_rng(13)
    n, k = 1024, 2304
    w = q8_0.random_q8_0(rng, n, k)
    xs = [rng.standard_normal(k, dtype=np.float32) for _ in range(3)]
    dw, dx = DeviceBuffer.from_array(w), DeviceBuffer.from_array(xs[0])
    out = DeviceBuffer.empty((n,), np.float32)
    s = Stream()
    g = Graph.capture(s, lambda: ops.matmul_q8_0(dw, dx, out, n, k, stream=s))
    for x in xs:
        dx.upload(x)
        out.fill_zero(s)
        g.launch(s)
        s.synchronize()
        assert rel_l2(out.download(), ora.q8_0_gemv(w, x, n, k)) <= 1e-5
    g.destroy()
    s.destroy()


def test_q8_0_gemv_rejects(dev):
    n, k = 4, 64
    dw = DeviceBuffer(n * q8_0.row_bytes(k) + 4)
    dx = DeviceBuffer.empty((32800,), np.float32)
    out = DeviceBuffer.empty((n,), np.float32)
    with pytest.raises(DoeError, match="4-byte aligned"):
        _lib.call("doe_q8_0_gemv", C.c_void_p(dw.ptr + 2), C.c_void_p(dx.ptr), C.c_void_p(out.ptr), n, k,
                  None, None)
    big = DeviceBuffer(q8_0.row_bytes(32800))
    with pytest.raises(DoeError, match="k <= 32768"):
        _lib.call("doe_q8_0_gemv", C.c_void_p(big.ptr), C.c_void_p(dx.ptr), C.c_void_p(out.ptr), 1, 32800,
                  None, None)
    with pytest.raises(ValueError, match="byte length"):
        ops.matmul_q8_0(dw, dx, out, n, k)


@pytest.mark.parametrize("heads,kv_heads,d,t,n", [(8, 4, 256, 300, 2304), (4, 1, 128, 37, 640), (2, 2, 64, 1, 100)])
def test_q8_0_gemv_attn_out_matches_oracle(dev, ora, heads, kv_heads, d, t, n):
    # split-attention partials (doe_attn_decode_partials) combined in the
    # Q8_0 GEMV's activation staging, against the oracle attention followed by
    # the oracle Q8_0 GEMV with the residual
    print(f"q8_0 attn_out heads={heads}/{kv_heads} d={d} t={t} n={n}", flush=True)
    rng = np.random.default_rng(heads * 1000 + t)
    q = rng.standard_normal((heads, d)).astype(np.float32)
    kc = rng.standard_normal((kv_heads, t, d)).astype(np.float16)
    vc = rng.standard_normal((kv_heads, t, d)).astype(np.float16)
    w = q8_0.random_q8_0(rng, n, heads * d)
    res = rng.standard_normal(n).astype(np.float32)
    parts = DeviceBuffer.empty((heads * 8 * (d + 2),), np.float32)
    scale = 1.0 / np.sqrt(d)
    splits = ops.attention_partials(DeviceBuffer.from_array(q), DeviceBuffer.from_array(kc),
                                    DeviceBuffer.from_array(vc), parts, batch=1, num_heads=heads,
                                    num_kv_heads=kv_heads, head_dim=d, kv_len=t, kv_stride=t, scale=scale)
    out = DeviceBuffer.from_array(res)
    ops.matmul_q8_0_attn_out(DeviceBuffer.from_array(w), parts, splits, heads, d, out, n, residual=out)
    attn = ora.attn_decode(q, kc, vc, heads, kv_heads, d, t, t, scale).reshape(-1)
    want = ora.q8_0_gemv(w, attn, n, heads * d, residual=res)
    err = rel_l2(out.download(), want)
    print(f"  splits {splits} rel_l2 {err:.2e}", flush=True)
    assert err <= 1e-3, err


def test_q8_0_gemv_rejects_aliased_activation(dev):
    n = k = 64
    dw = DeviceBuffer(n * q8_0.row_bytes(k))
    x = DeviceBuffer.empty((k,), np.float32)
    with pytest.raises(DoeError, match="alias"):
        _lib.call("doe_q8_0_gemv", C.c_void_p(dw.ptr), C.c_void_p(x.ptr), C.c_void_p(x.ptr), n, k, None, None)
    nw = DeviceBuffer.empty((k,), np.float32)
    out = DeviceBuffer.empty((n,), np.float32)
    with pytest.raises(DoeError, match="alias"):
        _lib.call("doe_q8_0_gemv_norm", C.c_void_p(dw.ptr), C.c_void_p(x.ptr), C.c_void_p(nw.ptr), n, k,
                  C.c_void_p(nw.ptr), C.c_float(1e-6), 0, None, None)
    with pytest.raises(DoeError, match="splits"):
        _lib.call("doe_q8_0_gemv_attn_out", C.c_void_p(dw.ptr), C.c_void_p(out.ptr), 9, 1, 64, C.c_void_p(x.ptr),
                  n, None, None)


@pytest.mark.parametrize("ffn,k,offset", [(9216, 2304, True), (300, 1000, False), (7, 33, True)])
def test_q8_0_gemv_gated_matches_oracle(dev, ora, ffn, k, offset):
    # post_attn_norm + gate/up_proj + activation in one dispatch over
    # interleaved (gate, up) rows: against the oracle rmsnorm, GEMV and GeGLU,
    # and bit for bit against the unfused GEMV + doe_geglu_pairs at the same
    # wave grouping
    print(f"q8_0 gated ffn={ffn} k={k}", flush=True)
    n = 2 * ffn
    rng = np.random.default_rng(ffn + k)
    w = q8_0.random_q8_0(rng, n, k)
    x = (rng.standard_normal(k) * 3).astype(np.float32)
    nw = (rng.standard_normal(k) * 0.1).astype(np.float32)
    g = ora.q8_0_gemv(w, ora.rmsnorm(x, nw, 1e-6, offset), n, k)
    want = ora.geglu(g[0::2], g[1::2])
    dw, dx, dn = DeviceBuffer.from_array(w), DeviceBuffer.from_array(x), DeviceBuffer.from_array(nw)
    out = DeviceBuffer.empty((ffn,), np.float32)
    ops.matmul_q4k_fused(dw, dx, out, n, k, norm_weight=dn, norm_eps=1e-6, norm_weight_offset=offset, gated=True,
                         weight_format="q8_0")
    got = out.download()
    assert rel_l2(got, want) <= 1e-5
    try:
        ops.tune("q8_0_gemv.rows", 2)
        gu = DeviceBuffer.empty((n,), np.float32)
        ops.matmul_q8_0(dw, dx, gu, n, k, norm_weight=dn, norm_eps=1e-6, norm_weight_offset=offset)
        h = DeviceBuffer.empty((ffn,), np.float32)
        ops.geglu_pairs(gu, h, ffn)
        fused = DeviceBuffer.empty((ffn,), np.float32)
        ops.matmul_q4k_fused(dw, dx, fused, n, k, norm_weight=dn, norm_eps=1e-6, norm_weight_offset=offset,
                             gated=True, weight_format="q8_0")
        assert np.array_equal(fused.download().view(np.uint32), h.download().view(np.uint32))
    finally:
        ops.tune("q8_0_gemv.rows", 0)


@pytest.mark.parametrize("heads,kv_heads,hd,hidden,pos", [(8, 4, 256, 2304, 37), (4, 2, 64, 320, 0),
                                                          (2, 1, 128, 96, 5), (4, 0, 64, 320, 3)])
def test_q8_0_qkv_rope_kv_matches_oracle(dev, ora, heads, kv_heads, hd, hidden, pos):
    # input_norm + q/k/v_proj + rope_q / rope_k + the cache write in one
    # dispatch, the q/k rows stored as rotation pairs: q and the cached k
    # against the oracle's rotate-half RoPE on plain rows, v as projected;
    # other cache rows untouched; kv_heads 0 projects q alone
    from doe_amd.model import rope_table
    from doe_amd.ops import deinterleave_rope_rows, interleave_rope_rows

    print(f"q8_0 qkv_rope_kv {heads}/{kv_heads}x{hd} hidden={hidden} pos={pos}", flush=True)
    rng = np.random.default_rng(heads * 100 + hd + pos)
    qd, kvd = heads * hd, kv_heads * hd
    n = qd + 2 * kvd
    rb = q8_0.row_bytes(hidden)
    w = q8_0.random_q8_0(rng, n, hidden).reshape(n, rb)
    dev_w = w.copy()
    dev_w[:qd] = interleave_rope_rows(w[:qd], hd)
    if kv_heads:
        dev_w[qd:qd + kvd] = interleave_rope_rows(w[qd:qd + kvd], hd)
    x = (rng.standard_normal(hidden) * 2).astype(np.float32)
    nw = (rng.standard_normal(hidden) * 0.1).astype(np.float32)
    max_seq = 64
    table = rope_table(max_seq, hd, 10000.0)
    qkv = ora.q8_0_gemv(w.reshape(-1), ora.rmsnorm(x, nw, 1e-6, True), n, hidden)
    qk = ora.rope(qkv[:qd + kvd], table, 1, heads + kv_heads, hd, pos)
    out = DeviceBuffer.empty((n,), np.float32)
    posb = DeviceBuffer.from_array(np.array([pos], np.int32))
    fill = np.full((max(kv_heads, 1), max_seq, hd), 7.0, np.float16)
    kc, vc = DeviceBuffer.from_array(fill), DeviceBuffer.from_array(fill)
    ops.qkv_rope_kv(DeviceBuffer.from_array(dev_w.reshape(-1)), DeviceBuffer.from_array(x), out, hidden=hidden,
                    num_heads=heads, num_kv_heads=kv_heads, head_dim=hd, freq_cis=DeviceBuffer.from_array(table),
                    position_buffer=posb, key_cache=kc, val_cache=vc, max_seq_len=max_seq,
                    norm_weight=DeviceBuffer.from_array(nw), norm_eps=1e-6, norm_weight_offset=True,
                    weight_format="q8_0")
    got = out.download()
    assert rel_l2(deinterleave_rope_rows(got[:qd], hd), qk[:qd]) <= 1e-5
    if not kv_heads:
        assert np.array_equal(kc.download(), fill) and np.array_equal(vc.download(), fill)
        return
    k_got = deinterleave_rope_rows(got[qd:qd + kvd], hd)
    assert rel_l2(k_got, qk[qd:]) <= 1e-5
    assert rel_l2(got[qd + kvd:], qkv[qd + kvd:]) <= 1e-5
    kcg, vcg = kc.download(), vc.download()
    kc_plain = np.concatenate([kcg[..., 0::2], kcg[..., 1::2]], axis=-1)  # cached in pair order
    # the cache rows are the f16 of the device's own rotated rows
    assert np.array_equal(kcg[:, pos].reshape(-1), got[qd:qd + kvd].astype(np.float16))
    assert np.array_equal(vcg[:, pos].reshape(-1), got[qd + kvd:].astype(np.float16))
    assert rel_l2(kc_plain[:, pos].reshape(-1).astype(np.float32), qk[qd:]) <= 1e-3
    others = np.ones(max_seq, bool)
    others[pos] = False
    assert np.all(kcg[:, others] == 7.0) and np.all(vcg[:, others] == 7.0)


def test_q8_0_fused_rejects(dev):
    w = DeviceBuffer.from_array(q8_0.random_q8_0(np.random.default_rng(0), 6, 64))
    x = DeviceBuffer.empty((64,), np.float32)
    y = DeviceBuffer.empty((6,), np.float32)
    with pytest.raises(DoeError):  # gated needs an even row count
        _lib.call("doe_q8_0_gemv_fused", C.c_void_p(w.ptr), C.c_void_p(x.ptr), C.c_void_p(y.ptr), 5, 64,
                  None, 1e-6, 0, None, 1, None)
    with pytest.raises(DoeError):  # gated and residual are exclusive
        _lib.call("doe_q8_0_gemv_fused", C.c_void_p(w.ptr), C.c_void_p(x.ptr), C.c_void_p(y.ptr), 6, 64,
                  None, 1e-6, 0, C.c_void_p(y.ptr), 1, None)
