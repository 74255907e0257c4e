"""doe_q4k_gemv_ex: the K-range output parts and activation parts that chain
the decode layer's GEMVs without atomics.  Producer: the parts summed in
range order equal the GEMV (against the oracle, within the GEMV contract).
Consumer: activation + parts is added in order, so a consumer given
(x, parts) is bit-identical to the same GEMV given the host's in-order f32
sum, and keeps that sum bit for bit; residual + parts likewise in the
epilogue.  Through the C ABI."""
import numpy as np
import pytest

from doe_amd import DeviceBuffer, DoeError, ops, q4k

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def up(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


@pytest.mark.parametrize("with_residual", [False, True])
@pytest.mark.parametrize("n,k,expect", [(2304, 9216, 3), (2304, 2048, 2), (9216, 2304, 1), (96, 300, 2),
                                        (2304, 21504, 4), (512, 65536, 4)])
def test_output_parts_sum_to_the_gemv(dev, ora, n, k, expect, with_residual):
    # range 0 carries the residual: part 0 - residual + the other parts is the GEMV
    rng = np.random.default_rng(n + k)
    w = q4k.random_q4k(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    res = (rng.standard_normal(n) * 4).astype(np.float32) if with_residual else None
    parts = DeviceBuffer.empty((ops.MAX_GEMV_PARTS, n), np.float32)
    got_n = ops.q4k_gemv_ex(up(w), n, k, activation=up(x), residual=up(res) if with_residual else None,
                            output_parts=parts, max_output_parts=ops.MAX_GEMV_PARTS)
    dev.synchronize()
    assert got_n == expect
    p = parts.download()[:got_n].astype(np.float64)
    want = ora.q4k_gemv(w, x, n, k) + (res if with_residual else 0.0)
    assert rel_l2(p.sum(0), want) < 1e-5


def test_output_parts_attention_prologue(dev, ora):
    # o_proj over the combine of 3 attention splits, as parts, equals the
    # attn_out form without them (same combine, then the sum of the ranges)
    rng = np.random.default_rng(5)
    heads, hd, S, n = 8, 256, 3, 2304
    k = heads * hd
    w = q4k.random_q4k(rng, n, k)
    o = rng.standard_normal((heads, S, hd)).astype(np.float32)
    ml = np.stack([rng.standard_normal((heads, S)) * 3, rng.uniform(1, 5, (heads, S))], -1).astype(np.float32)
    part_buf = up(np.concatenate([o.reshape(-1), ml.reshape(-1)]))
    parts = DeviceBuffer.empty((ops.MAX_GEMV_PARTS, n), np.float32)
    np_ = ops.q4k_gemv_ex(up(w), n, k, attn_partials=part_buf, attn_splits=S, attn_num_heads=heads,
                          attn_head_dim=hd, output_parts=parts, max_output_parts=ops.MAX_GEMV_PARTS)
    ref = DeviceBuffer.empty((n,), np.float32)
    ops.matmul_q4k_attn_out(up(w), part_buf, S, heads, hd, ref, n)
    dev.synchronize()
    p = parts.download()[:np_]
    total = p[0].copy()
    for i in range(1, np_):
        total = total + p[i]
    m = ml[..., 0].max(1, keepdims=True)
    f = np.exp2(ml[..., 0] - m)
    attn = ((o * f[..., None]).sum(1) / (ml[..., 1] * f).sum(1, keepdims=True)).reshape(-1)
    assert np_ == 2
    assert rel_l2(total, ref.download()) < 1e-6
    assert rel_l2(total, ora.q4k_gemv(w, attn.astype(np.float32), n, k)) < 1e-5


@pytest.mark.parametrize("nparts", [1, 2, 3, 4])
@pytest.mark.parametrize("form", ["norm_gated", "rope_kv", "plain"])
def test_activation_parts_bit_identical_to_host_sum(dev, nparts, form):
    rng = np.random.default_rng(nparts * 7 + len(form))
    k = 2304
    x = rng.standard_normal(k).astype(np.float32)
    parts = (rng.standard_normal((nparts, k)) * 0.3).astype(np.float32)
    xs = x.copy()
    for p in parts:
        xs = (xs + p).astype(np.float32)  # f32 adds, in part order
    nw = (0.1 * rng.standard_normal(k)).astype(np.float32)
    kw = dict(norm_weight=up(nw), norm_eps=1e-6, norm_weight_offset=True)
    if form == "norm_gated":
        n = 2 * 1536
        w = q4k.random_q4k(rng, n, k)
        kw.update(gated=True)
        out_len = n // 2
    elif form == "rope_kv":
        from doe_amd.model import rope_table

        heads, kvh, hd, ms = 4, 2, 128, 16
        n = (heads + 2 * kvh) * hd
        w = q4k.random_q4k(rng, n, k)
        out_len = n
        caches = [DeviceBuffer.empty((kvh, ms, hd), np.float16) for _ in range(4)]
        pos = up(np.array([5], np.int32))
        freq = up(rope_table(ms, hd, 10000.0))
    else:
        n = 1000
        w = q4k.random_q4k(rng, n, k)
        kw = {}
        out_len = n
    dw = up(w)
    got = DeviceBuffer.empty((out_len,), np.float32)
    want = DeviceBuffer.empty((out_len,), np.float32)
    kept = DeviceBuffer.empty((k,), np.float32)
    if form == "rope_kv":
        r1 = dict(num_heads=heads, num_kv_heads=kvh, head_dim=hd, freq_cis=freq, position_buffer=pos,
                  key_cache=caches[0], val_cache=caches[1], max_seq_len=ms)
        r2 = dict(r1, key_cache=caches[2], val_cache=caches[3])
        ops.q4k_gemv_ex(dw, n, k, activation=up(x), activation_parts=up(parts), activation_nparts=nparts,
                        activation_sum=kept, output=got, rope=r1, **kw)
        ops.q4k_gemv_ex(dw, n, k, activation=up(xs), output=want, rope=r2, **kw)
    else:
        ops.q4k_gemv_ex(dw, n, k, activation=up(x), activation_parts=up(parts), activation_nparts=nparts,
                        activation_sum=kept, output=got, **kw)
        ops.q4k_gemv_ex(dw, n, k, activation=up(xs), output=want, **kw)
    dev.synchronize()
    assert np.array_equal(kept.download().view(np.uint32), xs.view(np.uint32))
    assert np.array_equal(got.download().view(np.uint32), want.download().view(np.uint32))
    if form == "rope_kv":
        for a, b in ((caches[0], caches[2]), (caches[1], caches[3])):
            assert np.array_equal(a.download()[:, 5].view(np.uint16), b.download()[:, 5].view(np.uint16))


@pytest.mark.parametrize("nparts", [1, 2, 4])
@pytest.mark.parametrize("form", ["plain", "output_parts", "attention"])
def test_residual_parts_bit_identical_to_host_sum(dev, nparts, form):
    # residual + parts added in order in the epilogue: the same bits as the
    # GEMV given the host's in-order f32 sum as its residual (whole rows,
    # K-range output parts where range 0 carries it, the attention prologue)
    rng = np.random.default_rng(nparts * 11 + len(form))
    n = 2304
    res = (rng.standard_normal(n) * 4).astype(np.float32)
    rparts = (rng.standard_normal((nparts, n)) * 0.5).astype(np.float32)
    rs = res.copy()
    for p in rparts:
        rs = (rs + p).astype(np.float32)
    if form == "attention":
        heads, hd, S = 8, 256, 3
        k = heads * hd
        o = rng.standard_normal((heads, S, hd)).astype(np.float32)
        ml = np.stack([rng.standard_normal((heads, S)) * 3, rng.uniform(1, 5, (heads, S))], -1).astype(np.float32)
        src = dict(attn_partials=up(np.concatenate([o.reshape(-1), ml.reshape(-1)])), attn_splits=S,
                   attn_num_heads=heads, attn_head_dim=hd)
    else:
        k = 9216 if form == "output_parts" else 2048
        src = dict(activation=up(rng.standard_normal(k).astype(np.float32)))
    dw = up(q4k.random_q4k(rng, n, k))
    if form == "plain":
        got, want = DeviceBuffer.empty((n,), np.float32), DeviceBuffer.empty((n,), np.float32)
        # (a residual apart from the output: whole rows, no atomic K split)
        ops.q4k_gemv_ex(dw, n, k, residual=up(res), residual_parts=up(rparts), residual_nparts=nparts, output=got,
                        **src)
        ops.q4k_gemv_ex(dw, n, k, residual=up(rs), output=want, **src)
        dev.synchronize()
        a, b = got.download(), want.download()
    else:
        got = DeviceBuffer.empty((ops.MAX_GEMV_PARTS, n), np.float32)
        want = DeviceBuffer.empty((ops.MAX_GEMV_PARTS, n), np.float32)
        n1 = ops.q4k_gemv_ex(dw, n, k, residual=up(res), residual_parts=up(rparts), residual_nparts=nparts,
                             output_parts=got, max_output_parts=ops.MAX_GEMV_PARTS, **src)
        n2 = ops.q4k_gemv_ex(dw, n, k, residual=up(rs), output_parts=want, max_output_parts=ops.MAX_GEMV_PARTS,
                             **src)
        dev.synchronize()
        assert n1 == n2 and n1 > 1
        a, b = got.download()[:n1], want.download()[:n2]
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_parts_argument_checks(dev):
    rng = np.random.default_rng(1)
    w = up(q4k.random_q4k(rng, 64, 512))
    x = up(np.ones(512, np.float32))
    y = DeviceBuffer.empty((64,), np.float32)
    with pytest.raises(DoeError):  # five activation parts
        ops.q4k_gemv_ex(w, 64, 512, activation=x, activation_parts=up(np.zeros((5, 512), np.float32)),
                        activation_nparts=5, output=y)
    with pytest.raises(DoeError):  # output parts with the RMSNorm prologue (it needs whole rows)
        ops.q4k_gemv_ex(w, 64, 512, activation=x, norm_weight=x, output_parts=DeviceBuffer.empty((4, 64), np.float32),
                        max_output_parts=4)
    r = up(np.ones(64, np.float32))
    with pytest.raises(DoeError):  # residual parts without a residual
        ops.q4k_gemv_ex(w, 64, 512, activation=x, residual_parts=up(np.zeros((1, 64), np.float32)),
                        residual_nparts=1, output=y)
    with pytest.raises(DoeError):  # residual parts with the residual in place (the atomic K split)
        ops.q4k_gemv_ex(w, 64, 512, activation=x, residual=y, residual_parts=up(np.zeros((1, 64), np.float32)),
                        residual_nparts=1, output=y)
    with pytest.raises(DoeError):  # residual parts with the RMSNorm prologue
        ops.q4k_gemv_ex(w, 64, 512, activation=x, norm_weight=x, residual=r,
                        residual_parts=up(np.zeros((1, 64), np.float32)), residual_nparts=1, output=y)
    with pytest.raises(DoeError):  # five residual parts
        ops.q4k_gemv_ex(w, 64, 512, activation=x, residual=r, residual_parts=up(np.zeros((5, 64), np.float32)),
                        residual_nparts=5, output=y)
    with pytest.raises(DoeError):  # k = 65536 needs 4 output parts, room for 2
        big = up(q4k.random_q4k(rng, 16, 65536))
        ops.q4k_gemv_ex(big, 16, 65536, activation=up(np.ones(65536, np.float32)),
                        output_parts=DeviceBuffer.empty((2, 16), np.float32), max_output_parts=2)


@pytest.mark.parametrize("n,k,nres", [(5376, 21504, 1), (2304, 9216, 2), (3000, 8192, 0)])
def test_streaming_output_parts_bit_identical_to_one_shot(dev, ora, n, k, nres):
    # K ranges as output parts through the streaming kernel (two blocks per
    # wave where a range holds 17..22 blocks), range 0 with the residual and
    # its parts: the same parts, bit for bit, as the one-shot kernel's, and
    # their sum the GEMV
    rng = np.random.default_rng(n + k + nres)
    w = up(q4k.random_q4k(rng, n, k))
    xh = rng.standard_normal(k).astype(np.float32)
    res = (rng.standard_normal(n) * 3).astype(np.float32)
    rparts = (rng.standard_normal((max(nres, 1), n)) * 0.5).astype(np.float32)
    x, dres, drp = up(xh), up(res), up(rparts)
    got = []
    for st in (4, -1):  # streaming (four row groups per workgroup), then never
        ops.tune("q4k_gemv.stream", st)
        try:
            parts = DeviceBuffer.empty((ops.MAX_GEMV_PARTS, n), np.float32)
            np_ = ops.q4k_gemv_ex(w, n, k, activation=x, residual=dres, residual_parts=drp if nres else None,
                                  residual_nparts=nres, output_parts=parts, max_output_parts=ops.MAX_GEMV_PARTS)
            dev.synchronize()
            got.append(parts.download()[:np_])
        finally:
            ops.tune("q4k_gemv.stream", 0)
    assert got[0].shape == got[1].shape and got[0].shape[0] > 1
    assert np.array_equal(got[0].view(np.uint32), got[1].view(np.uint32))
    rs = res.copy()
    for i in range(nres):
        rs = (rs + rparts[i]).astype(np.float32)
    want = ora.q4k_gemv(w.download().reshape(n, -1), xh, n, k) + rs.astype(np.float64)
    assert rel_l2(got[0].astype(np.float64).sum(0), want) < 1e-5


@pytest.mark.parametrize("splits,nparts", [(7, 2), (3, 4), (1, 2), (6, 4)])
def test_streaming_attention_prologue_bit_identical_to_one_shot(dev, ora, splits, nparts):
    # o_proj over the combine of the attention splits through the streaming
    # kernel (32 heads of 256, K ranges as output parts -- as many as the
    # parts allow past 16 blocks -- the residual with a part): the same bits
    # as the one-shot kernel, and the oracle GEMV over the combine
    rng = np.random.default_rng(splits * 10 + nparts)
    heads, hd, n = 32, 256, 5376
    k = heads * hd
    wn = q4k.random_q4k(rng, n, k)
    w = up(wn)
    o = rng.standard_normal((heads, splits, hd)).astype(np.float32)
    ml = np.stack([rng.standard_normal((heads, splits)) * 3, rng.uniform(1, 5, (heads, splits))], -1)
    pb = up(np.concatenate([o.reshape(-1), ml.astype(np.float32).reshape(-1)]))
    res, rp = up(rng.standard_normal(n).astype(np.float32)), up(rng.standard_normal((1, n)).astype(np.float32))
    got = []
    for st in (3, -1):
        ops.tune("q4k_gemv.stream", st)
        try:
            parts = DeviceBuffer.empty((ops.MAX_GEMV_PARTS, n), np.float32)
            np_ = ops.q4k_gemv_ex(w, n, k, attn_partials=pb, attn_splits=splits, attn_num_heads=heads,
                                  attn_head_dim=hd, residual=res, residual_parts=rp, residual_nparts=1,
                                  output_parts=parts, max_output_parts=nparts)
            dev.synchronize()
            got.append(parts.download()[:np_])
        finally:
            ops.tune("q4k_gemv.stream", 0)
    assert got[0].shape == got[1].shape == (nparts, n)
    assert np.array_equal(got[0].view(np.uint32), got[1].view(np.uint32))
    m = ml[..., 0].max(1, keepdims=True)
    f = np.exp2(ml[..., 0] - m)
    attn = ((o * f[..., None]).sum(1) / (ml[..., 1] * f).sum(1, keepdims=True)).reshape(-1).astype(np.float32)
    want = ora.q4k_gemv(wn, attn, n, k) + res.download().astype(np.float64) + rp.download()[0].astype(np.float64)
    assert rel_l2(got[0].astype(np.float64).sum(0), want) < 1e-5


def test_range_count_tuning(dev, ora):
    # q4k_gemv.ksplit 2-4 sets the least number of K ranges where output
    # parts are written; q4k_gemv.forms bit 2 keeps the attention-prologue
    # o_proj in its fewest ranges.  Every count sums to the same GEMV.
    rng = np.random.default_rng(77)
    n, k = 9216, 2304  # 576 row groups: one range unless forced
    w = q4k.random_q4k(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    want = ora.q4k_gemv(w, x, n, k)
    dw, dx = up(w), up(x)
    for least in (2, 3, 4):
        ops.tune("q4k_gemv.ksplit", least)
        try:
            parts = DeviceBuffer.empty((ops.MAX_GEMV_PARTS, n), np.float32)
            got_n = ops.q4k_gemv_ex(dw, n, k, activation=dx, output_parts=parts, max_output_parts=ops.MAX_GEMV_PARTS)
            dev.synchronize()
        finally:
            ops.tune("q4k_gemv.ksplit", 0)
        assert got_n == least
        assert rel_l2(parts.download()[:got_n].astype(np.float64).sum(0), want) < 1e-5
    with pytest.raises(DoeError):
        ops.tune("q4k_gemv.ksplit", ops.MAX_GEMV_PARTS + 1)
    heads, hd, S, n = 32, 256, 2, 5376  # 336 row groups
    k = heads * hd
    wn = q4k.random_q4k(rng, n, k)
    o = rng.standard_normal((heads, S, hd)).astype(np.float32)
    ml = np.stack([rng.standard_normal((heads, S)), rng.uniform(1, 5, (heads, S))], -1).astype(np.float32)
    pb = up(np.concatenate([o.reshape(-1), ml.reshape(-1)]))
    m = ml[..., 0].max(1, keepdims=True)
    f = np.exp2(ml[..., 0] - m)
    attn = ((o * f[..., None]).sum(1) / (ml[..., 1] * f).sum(1, keepdims=True)).reshape(-1).astype(np.float32)
    want = ora.q4k_gemv(wn, attn, n, k)
    dw = up(wn)
    for forms, expect in ((0, 4), (2, 2)):
        ops.tune("q4k_gemv.forms", forms)
        try:
            parts = DeviceBuffer.empty((ops.MAX_GEMV_PARTS, n), np.float32)
            got_n = ops.q4k_gemv_ex(dw, n, k, attn_partials=pb, attn_splits=S, attn_num_heads=heads,
                                    attn_head_dim=hd, output_parts=parts, max_output_parts=ops.MAX_GEMV_PARTS)
            dev.synchronize()
        finally:
            ops.tune("q4k_gemv.forms", 0)
        assert got_n == expect
        assert rel_l2(parts.download()[:got_n].astype(np.float64).sum(0), want) < 1e-5
