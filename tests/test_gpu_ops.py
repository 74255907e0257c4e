"""GPU parity of the decode-loop ops (RMSNorm, RoPE, GeGLU, residual, argmax,
KV write, embed gather, f16 lm_head GEMV in both layouts and with several
activation rows, fused Q4_K GEMVs) against the CPU
oracle, through the C ABI.  Byte/index work and exactly-rounded elementwise
ops are compared bit-exactly; reductions and transcendentals by rel-L2."""
import math

import numpy as np
import pytest

from doe_amd import DeviceBuffer, ops, q4k

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def up(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


@pytest.mark.parametrize("rows,h,offset", [(1, 2304, True), (3, 2304, False), (2, 5, True), (4, 9216, True)])
def test_rmsnorm(dev, ora, rows, h, offset):
    rng = np.random.default_rng(h + rows)
    x = rng.standard_normal((rows, h)).astype(np.float32) * 3
    w = (0.1 * rng.standard_normal(h)).astype(np.float32)
    out = DeviceBuffer.empty((rows, h), np.float32)
    ops.rmsnorm(up(x), up(w), out, rows, h, 1e-6, offset)
    assert rel_l2(out.download(), ora.rmsnorm(x, w, 1e-6, offset)) < 1e-6


def test_rmsnorm_reference_fixture(dev, known_answers):
    e = known_answers["fixture_rmsnorm"]
    out = DeviceBuffer.empty((4,), np.float32)
    ops.rmsnorm(up(np.array(e["input"], np.float32)), up(np.array(e["weight"], np.float32)), out, 1, 4, e["eps"])
    got = out.download()
    want = np.array(e["output"], np.float32)
    assert np.abs(got.view(np.int32) - want.view(np.int32)).max() <= 2


def test_rope_bit_exact(dev, ora):
    rng = np.random.default_rng(2)
    seq, heads, d, maxpos = 3, 12, 256, 600
    table = ora.rope_table(maxpos, d, 10000.0)
    x = rng.standard_normal(seq * heads * d).astype(np.float32)
    for off in (0, 7, 512):
        buf = up(x)
        ops.rope(buf, up(table), seq, heads, d, off)
        assert np.array_equal(buf.download(), ora.rope(x, table, seq, heads, d, off)), off
    # device-side position
    buf = up(x)
    ops.rope(buf, up(table), seq, heads, d, 0, position_buffer=up(np.array([41], np.int32)))
    assert np.array_equal(buf.download(), ora.rope(x, table, seq, heads, d, 41))


def test_geglu_and_residual(dev, ora):
    rng = np.random.default_rng(3)
    n = 9216 * 3 + 5
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    out = DeviceBuffer.empty((n,), np.float32)
    ops.gelu_gated(up(g), up(u), out, n)
    assert rel_l2(out.download(), ora.geglu(g, u)) < 1e-6
    ops.residual(up(g), up(u), out, n)
    assert np.array_equal(out.download(), ora.residual(g, u))


def test_rope_half_kv_rows_equals_rope_and_kv_write(dev, ora):
    # the prompt-row form in head order against doe_rope (same rotate-half
    # pairing and arithmetic) token by token and doe_kv_write: bit-exact
    rng = np.random.default_rng(31)
    tokens, hq, hkv, d, max_seq, start = 5, 4, 2, 64, 16, 3
    table = ora.rope_table(max_seq, d, 10000.0)
    stride = (hq + 2 * hkv) * d + 8
    qkv = rng.standard_normal((tokens, stride)).astype(np.float32)
    buf = up(qkv)
    kc = DeviceBuffer.from_array(np.zeros((hkv, max_seq, d), np.float16))
    vc = DeviceBuffer.from_array(np.zeros((hkv, max_seq, d), np.float16))
    ops.qkv_rope_half_kv_rows(buf, tokens, stride, hq, hkv, d, up(table), start, kc, vc, max_seq)
    got = buf.download()
    kref = np.zeros((hkv, max_seq, d), np.float16)
    vref = np.zeros((hkv, max_seq, d), np.float16)
    for t in range(tokens):
        qk = qkv[t, : (hq + hkv) * d]
        want = ora.rope(qk, table, 1, hq + hkv, d, start + t)
        assert np.array_equal(got[t, : (hq + hkv) * d], want), t
        assert np.array_equal(got[t, (hq + hkv) * d:], qkv[t, (hq + hkv) * d:]), t  # v and padding untouched
        kref[:, start + t] = want[hq * d:].reshape(hkv, d).astype(np.float16)
        vref[:, start + t] = qkv[t, (hq + hkv) * d: (hq + 2 * hkv) * d].reshape(hkv, d).astype(np.float16)
    assert np.array_equal(kc.download(), kref)
    assert np.array_equal(vc.download(), vref)


def test_geglu_halves(dev, ora):
    rng = np.random.default_rng(32)
    rows, n = 7, 1000
    gu = (rng.standard_normal((rows, 2 * n)) * 4).astype(np.float32)
    out = DeviceBuffer.empty((rows, n), np.float32)
    ops.geglu_halves(up(gu), out, rows, n)
    want = np.stack([ora.geglu(gu[t, :n], gu[t, n:]) for t in range(rows)])
    # the kernel runs the per-row gelu_gated kernel's arithmetic
    single = DeviceBuffer.empty((n,), np.float32)
    ops.gelu_gated(up(gu[3, :n]), up(gu[3, n:]), single, n)
    got = out.download()
    assert np.array_equal(got[3], single.download())
    assert rel_l2(got, want) < 1e-6


def test_argmax(dev, ora, known_answers):
    ws = DeviceBuffer(8192)
    tok = DeviceBuffer.empty((1,), np.int32)
    e = known_answers["emulator_sample"]
    for logits in (e["logits"], e["tie_logits"]):
        x = np.array(logits, np.float32)
        ops.sample(up(x), x.size, tok, ws)
        assert tok.download()[0] == ora.argmax(x)
    rng = np.random.default_rng(4)
    for n in (1, 255, 256000):
        x = rng.standard_normal(n).astype(np.float32)
        ops.sample(up(x), n, tok, ws)
        assert tok.download()[0] == ora.argmax(x)
    # ties at the maximum: lowest index wins; NaN never wins; all -inf -> 0
    x = np.zeros(100000, np.float32)
    x[[99999, 31337, 777]] = 5.0
    x[5] = np.nan
    ops.sample(up(x), x.size, tok, ws)
    assert tok.download()[0] == 777
    x = np.full(1000, -np.inf, np.float32)
    ops.sample(up(x), x.size, tok, ws)
    assert tok.download()[0] == 0


@pytest.mark.parametrize("layout", [0, 1])
def test_kv_write_bit_exact(dev, ora, layout):
    rng = np.random.default_rng(5)
    kvh, maxs, d = 4, 64, 256
    kp = (rng.standard_normal((kvh, d)) * 100).astype(np.float32)
    vp = rng.standard_normal((kvh, d)).astype(np.float32)
    shape = (kvh, maxs, d) if layout == 0 else (maxs, kvh, d)
    kc_h = np.zeros(shape, np.float16)
    vc_h = np.zeros(shape, np.float16)
    kc, vc = up(kc_h), up(vc_h)
    ops.kv_write(up(kp), up(vp), kc, vc, kvh, maxs, d, 13, kv_layout=layout)
    ops.kv_write(up(kp * 2), up(vp * 2), kc, vc, kvh, maxs, d, 0, position_buffer=up(np.array([20], np.int32)),
                 kv_layout=layout)
    ora.kv_write(kp, vp, kc_h, vc_h, kvh, maxs, d, 13, layout)
    ora.kv_write(kp * 2, vp * 2, kc_h, vc_h, kvh, maxs, d, 20, layout)
    assert np.array_equal(kc.download().view(np.uint16), kc_h.view(np.uint16))
    assert np.array_equal(vc.download().view(np.uint16), vc_h.view(np.uint16))


def test_embed_gather_bit_exact(dev, ora):
    rng = np.random.default_rng(6)
    vocab, hidden = 1000, 2304
    table = (rng.standard_normal((vocab, hidden)) * 0.02).astype(np.float16)
    ids = np.array([5, 999, 0, 1000, -3, 512], np.int32)
    out = DeviceBuffer.empty((ids.size, hidden), np.float32)
    ops.embed(up(table), up(ids), out, ids.size, vocab, hidden)
    assert np.array_equal(out.download(), ora.embed_gather(table, ids))
    ops.embed(up(table), up(ids), out, ids.size, vocab, hidden, scale=48.0)
    assert np.array_equal(out.download(), ora.embed_gather(table, ids, 48.0))


def test_gather_f32_interpreter_known_answer(dev, known_answers):
    # reference_interpreter.zig:4143-4219: rows [2, 0, 3] of a 4x2 table
    e = known_answers["interp_gather"]
    table = np.array(e["table_f32"], np.float32)
    ids = np.array(e["indices_u32"], np.uint32)
    out = DeviceBuffer.empty((3, 2), np.float32)
    ops.gather_f32(up(table), up(ids), out, 3, 4, 2)
    assert np.array_equal(out.download(), np.array(e["output"], np.float32))
    # :4221-4276: an index outside the table is rejected, not clamped
    e = known_answers["interp_gather_oob"]
    out1 = DeviceBuffer.empty((1, 1), np.float32)
    with pytest.raises(ValueError):
        ops.gather_f32(up(np.array(e["table_f32"], np.float32)), up(np.array(e["indices_u32"], np.uint32)),
                       out1, 1, 2, 1)


@pytest.mark.parametrize("n_ids,vocab,hidden", [(40, 50, 7), (128, 262144 // 64, 2304), (3, 9, 1), (0, 4, 8)])
def test_gather_f32_bit_exact(dev, ora, n_ids, vocab, hidden):
    rng = np.random.default_rng(n_ids + vocab + hidden)
    table = rng.standard_normal((vocab, hidden)).astype(np.float32)
    table.view(np.uint32)[0, 0] = 0x7FC01234  # NaN payloads move unchanged
    ids = rng.integers(0, vocab, n_ids).astype(np.uint32)
    if n_ids:
        ids[0] = 0
    out = DeviceBuffer.empty((max(n_ids, 1), hidden), np.float32)
    ops.gather_f32(up(table), up(ids if n_ids else np.zeros(1, np.uint32)), out, n_ids, vocab, hidden)
    if n_ids:
        assert np.array_equal(out.download()[:n_ids].view(np.uint32), ora.gather_f32(table, ids).view(np.uint32))
    # non-strict: out-of-range rows zero-filled and counted on the device
    bad = DeviceBuffer.from_array(np.array([77], np.int32))
    ids2 = np.array([1, vocab, 0xFFFFFFFF, 0], np.uint32)
    out2 = DeviceBuffer.empty((4, hidden), np.float32)
    ops.gather_f32(up(table), up(ids2), out2, 4, vocab, hidden, strict=False, bad_ids=bad)
    got = out2.download()
    assert bad.download()[0] == 2
    assert np.array_equal(got[[0, 3]].view(np.uint32), table[[1, 0]].view(np.uint32))
    assert not got[1:3].any()


@pytest.mark.parametrize("n,k", [(256000 // 8, 2304), (1000, 2304), (7, 8), (100, 5120), (33, 512)])
def test_f16_gemv(dev, ora, n, k):
    rng = np.random.default_rng(n + k)
    b = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    a = rng.standard_normal(k).astype(np.float32)
    out = DeviceBuffer.empty((n,), np.float32)
    ops.lm_head(up(b), up(a), out, n, k, alpha=0.5)
    assert rel_l2(out.download(), ora.f16_gemv(b, a, 0.5)) < 1e-5


def test_f16_gemv_full_vocab_shape(dev):
    # 256000 x 2304 (the 2B-class lm_head): float64 check on sampled rows
    rng = np.random.default_rng(7)
    n, k = 256000, 2304
    b = (rng.standard_normal((n, k), dtype=np.float32) * 0.02).astype(np.float16)
    a = rng.standard_normal(k).astype(np.float32)
    out = DeviceBuffer.empty((n,), np.float32)
    ops.lm_head(up(b), up(a), out, n, k)
    got = out.download()
    rows = rng.integers(0, n, 2000)
    want = b[rows].astype(np.float64) @ a.astype(np.float64)
    assert rel_l2(got[rows], want) < 1e-5


@pytest.mark.parametrize("m,n,k,tb", [
    (1, 1000, 2304, 0), (1, 999, 777, 0), (3, 4096, 2304, 0), (4, 37, 5120, 0), (9, 1032, 300, 0),
    (17, 513, 64, 0), (1, 1000, 777, 1), (1, 333, 10000, 1), (2, 1000, 2304, 1), (5, 77, 129, 1),
    (12, 1001, 5120, 1), (1, 8, 1, 0), (1, 3, 1, 1)])
def test_lm_head_gemv_layouts_and_rows(dev, ora, m, n, k, tb):
    # lm_head_gemv.wgsl:105-143: both layouts of B, odd and large K, and
    # several activation rows, against the oracle (f32 sums, rel-L2 1e-5)
    rng = np.random.default_rng(m * 7 + n + k + tb)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = (rng.standard_normal((n, k) if tb else (k, n)) * 0.02).astype(np.float16)
    out = DeviceBuffer.empty((m, n), np.float32)
    ops.lm_head_gemv(up(a), up(b), out, m, n, k, alpha=-0.75, transpose_b=tb)
    assert rel_l2(out.download(), ora.lm_head_gemv(a, b, -0.75, tb)) < 1e-5


def test_lm_head_gemv_one_row_is_doe_f16_gemv(dev):
    # one row against [N][K] runs the same kernel as doe_f16_gemv: identical bits
    rng = np.random.default_rng(21)
    n, k = 3000, 2304
    a = rng.standard_normal(k).astype(np.float32)
    b = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    o1 = DeviceBuffer.empty((n,), np.float32)
    o2 = DeviceBuffer.empty((n,), np.float32)
    ops.lm_head(up(b), up(a), o1, n, k, alpha=0.5)
    ops.lm_head_gemv(up(a), up(b), o2, 1, n, k, alpha=0.5, transpose_b=1)
    assert np.array_equal(o1.download(), o2.download())


def test_lm_head_gemv_full_vocab_column_major(dev):
    # 256000 x 2304 stored [K][N] (transpose_b = 0), two rows: float64 on sampled columns
    rng = np.random.default_rng(22)
    m, n, k = 2, 256000, 2304
    b = (rng.standard_normal((k, n), dtype=np.float32) * 0.02).astype(np.float16)
    a = rng.standard_normal((m, k)).astype(np.float32)
    out = DeviceBuffer.empty((m, n), np.float32)
    ops.lm_head_gemv(up(a), up(b), out, m, n, k, transpose_b=0)
    got = out.download()
    cols = rng.integers(0, n, 2000)
    want = a.astype(np.float64) @ b[:, cols].astype(np.float64)
    assert rel_l2(got[:, cols], want) < 1e-5


def test_lm_head_gemv_edges(dev):
    from doe_amd import DoeError
    out = DeviceBuffer.from_array(np.full((2, 5), 7.0, np.float32))
    a = DeviceBuffer.empty((2, 1), np.float32)
    b = DeviceBuffer.empty((5, 1), np.float16)
    ops.lm_head_gemv(a, b, out, 2, 5, 0)  # k = 0: all-zero output
    assert not out.download().any()
    ops.lm_head_gemv(a, b, out, 0, 5, 1)  # m = 0: nothing written
    with pytest.raises(DoeError):
        ops.lm_head_gemv(a, b, out, 1, 5, 1, transpose_b=2)


def test_fused_gemv_norm_residual_gated(dev, ora, gemv_kernel):
    rng = np.random.default_rng(8)
    k = 2304
    x = (rng.standard_normal(k) * 5).astype(np.float32)
    nw = (0.1 * rng.standard_normal(k)).astype(np.float32)
    xn = ora.rmsnorm(x, nw, 1e-6, True)
    # norm prologue: QKV-shaped GEMV (4096 rows)
    n = 4096
    w = q4k.random_q4k(rng, n, k)
    out = DeviceBuffer.empty((n,), np.float32)
    ops.matmul_q4k_fused(up(w), up(x), out, n, k, norm_weight=up(nw), norm_eps=1e-6, norm_weight_offset=True)
    assert rel_l2(out.download(), ora.q4k_gemv(w, xn, n, k)) < 1e-5
    # residual epilogue: O-projection shape
    n2, k2 = 2304, 2048
    w2 = q4k.random_q4k(rng, n2, k2)
    x2 = rng.standard_normal(k2).astype(np.float32)
    res = rng.standard_normal(n2).astype(np.float32)
    out2 = DeviceBuffer.empty((n2,), np.float32)
    ops.matmul_q4k_fused(up(w2), up(x2), out2, n2, k2, residual=up(res))
    want2 = ora.residual(ora.q4k_gemv(w2, x2, n2, k2), res)
    assert rel_l2(out2.download(), want2) < 1e-5
    # gated epilogue with the norm prologue: interleaved gate/up rows
    ff = 9216
    wg = q4k.random_q4k(rng, 2 * ff, k)
    out3 = DeviceBuffer.empty((ff,), np.float32)
    ops.matmul_q4k_fused(up(wg), up(x), out3, 2 * ff, k, norm_weight=up(nw), norm_eps=1e-6, gated=True)
    y = ora.q4k_gemv(wg, xn, 2 * ff, k)
    want3 = ora.geglu(y[0::2], y[1::2])
    assert rel_l2(out3.download(), want3) < 1e-5


@pytest.mark.parametrize("pos", [0, 17, 63, 64])
def test_qkv_rope_kv(dev, ora, pos, gemv_kernel):
    # the fused input_norm + q/k/v_proj + rope + cache write, 2B-class head
    # shape (8 q / 4 kv heads of 256 over hidden 2304); pos 64 is outside the
    # 64-position cache: unrotated q/k and no cache write
    rng = np.random.default_rng(9 + pos)
    hidden, hq, hkv, d, maxs = 2304, 8, 4, 256, 64
    qd, kd = hq * d, hkv * d
    n = qd + 2 * kd
    w_plain = q4k.random_q4k(rng, n, hidden).reshape(n, -1)
    w_dev = w_plain.copy()
    w_dev[: qd + kd] = ops.interleave_rope_rows(w_plain[: qd + kd], d)
    x = (rng.standard_normal(hidden) * 3).astype(np.float32)
    nw = (0.1 * rng.standard_normal(hidden)).astype(np.float32)
    table = ora.rope_table(maxs, d, 10000.0)
    kc0 = (rng.standard_normal((hkv, maxs, d))).astype(np.float16)
    vc0 = (rng.standard_normal((hkv, maxs, d))).astype(np.float16)
    kc, vc = up(kc0), up(vc0)
    out = DeviceBuffer.empty((n,), np.float32)
    ops.qkv_rope_kv(up(w_dev), up(x), out, hidden=hidden, num_heads=hq, num_kv_heads=hkv, head_dim=d,
                    freq_cis=up(table), position_buffer=up(np.array([pos], np.int32)), key_cache=kc,
                    val_cache=vc, max_seq_len=maxs, norm_weight=up(nw), norm_eps=1e-6, norm_weight_offset=True)
    qkv = ora.q4k_gemv(w_plain, ora.rmsnorm(x, nw, 1e-6, True), n, hidden)
    inside = pos < maxs
    qk = ora.rope(qkv[: qd + kd], table, 1, hq + hkv, d, pos) if inside else qkv[: qd + kd]
    want = np.concatenate([ops.interleave_rope_rows(qk, d), qkv[qd + kd:]])
    got = out.download()
    assert rel_l2(got, want) < 1e-5
    kc_want, vc_want = kc0.copy(), vc0.copy()
    if inside:
        kc_want[:, pos] = ops.interleave_rope_rows(qk[qd:], d).reshape(hkv, d)
        vc_want[:, pos] = qkv[qd + kd:].reshape(hkv, d)
    # untouched rows bit-exact; the written row within f16 rounding of the oracle
    kg, vg = kc.download(), vc.download()
    other = [p for p in range(maxs) if p != pos]
    assert np.array_equal(kg[:, other].view(np.uint16), kc0[:, other].view(np.uint16))
    assert np.array_equal(vg[:, other].view(np.uint16), vc0[:, other].view(np.uint16))
    if inside:
        assert rel_l2(kg[:, pos].astype(np.float32), kc_want[:, pos].astype(np.float32)) < 1e-3
        assert rel_l2(vg[:, pos].astype(np.float32), vc_want[:, pos].astype(np.float32)) < 1e-3
        # the cache row is exactly the f16 rounding of the device's own output
        assert np.array_equal(kg[:, pos].reshape(-1).view(np.uint16),
                              got[qd: qd + kd].astype(np.float16).view(np.uint16))


def _advance_token(parts, nparts):
    """Reduces lm_head argmax partials through doe_decode_advance and returns
    (token, recorded id, state) for a step past the prompt."""
    import ctypes as C

    from doe_amd import _lib
    state = up(np.array([5, 6, 0, -1], np.int32))
    tok = DeviceBuffer.empty((1,), np.int32)
    ids = up(np.full(16, -7, np.int32))
    _lib.call("doe_decode_advance", C.c_void_p(state.ptr), C.c_void_p(tok.ptr), C.c_void_p(ids.ptr), 16,
              C.c_void_p(parts.ptr), nparts, C.c_void_p(None))
    return int(tok.download()[0]), int(ids.download()[6]), state.download().tolist()


@pytest.mark.parametrize("n,seed", [(256000, 11), (256000, 12), (4096, 13), (77, 14)])
def test_lm_head_sample(dev, ora, n, seed):
    # final norm + lm_head + greedy sample: logits to rel-L2 1e-5 and the
    # token equal to the oracle's argmax (when the top two logits are apart
    # by more than the GEMV tolerance)
    rng = np.random.default_rng(seed)
    k = 2304
    b = (rng.standard_normal((n, k), dtype=np.float32) * 0.02).astype(np.float16)
    a = (rng.standard_normal(k) * 4).astype(np.float32)
    nw = (0.1 * rng.standard_normal(k)).astype(np.float32)
    logits = DeviceBuffer.empty((n,), np.float32)
    parts = DeviceBuffer(1024 * 8)
    cnt = ops.lm_head_sample(up(b), up(a), n, k, parts, logits=logits, norm_weight=up(nw), norm_eps=1e-6)
    assert 1 <= cnt <= 1024
    want = ora.f16_gemv(b, ora.rmsnorm(a, nw, 1e-6, True))
    got = logits.download()
    assert rel_l2(got, want) < 1e-5
    tok, rec, state = _advance_token(parts, cnt)
    assert tok == int(np.argmax(got))  # exact reduction of the device's own logits
    top = np.sort(want)[-2:]
    if top[1] - top[0] > 1e-4 * abs(top[1]):
        assert tok == ora.argmax(want)
    assert rec == tok and state == [6, 7, 0, tok]
    # without the logits output the partials are the same
    parts2 = DeviceBuffer(1024 * 8)
    cnt2 = ops.lm_head_sample(up(b), up(a), n, k, parts2, norm_weight=up(nw), norm_eps=1e-6)
    assert cnt2 == cnt and np.array_equal(parts2.download()[: cnt * 8], parts.download()[: cnt * 8])


def test_lm_head_sample_ties_and_nan(dev, ora):
    # equal logits across workgroups: the lowest index wins; NaN never wins;
    # all NaN gives index 0 (the reference's starting index)
    rng = np.random.default_rng(15)
    n, k = 50000, 256
    row = (rng.standard_normal(k) * 0.02).astype(np.float16)
    b = np.tile(row, (n, 1))
    a = rng.standard_normal(k).astype(np.float32)
    b[:10] = np.float16(np.nan)
    parts = DeviceBuffer(1024 * 8)
    cnt = ops.lm_head_sample(up(b), up(a), n, k, parts)
    logits = np.where(np.arange(n) < 10, np.nan, 1.0).astype(np.float32)
    assert _advance_token(parts, cnt)[0] == 10 == ora.argmax(logits)
    b[:] = np.float16(np.nan)
    cnt = ops.lm_head_sample(up(b), up(a), n, k, parts)
    assert _advance_token(parts, cnt)[0] == 0 == ora.argmax(np.full(n, np.nan, np.float32))


@pytest.mark.parametrize("kv_len,max_splits", [(200, 8), (384, 8), (17, 8), (300, 1), (300, 3)])
def test_attention_partials_and_fused_o_projection(dev, ora, kv_len, max_splits, gemv_kernel):
    # attention split partials combined inside the Wo GEMV (+ residual), the
    # 2B-class decode shapes: 8 q / 4 kv heads of 256, Wo 2304 x 2048
    rng = np.random.default_rng(kv_len + max_splits)
    hq, hkv, d, maxs, hidden = 8, 4, 256, 384, 2304
    q = rng.standard_normal((hq, d)).astype(np.float32)
    kc = rng.standard_normal((hkv, maxs, d)).astype(np.float16)
    vc = rng.standard_normal((hkv, maxs, d)).astype(np.float16)
    wo = q4k.random_q4k(rng, hidden, hq * d)
    res = rng.standard_normal(hidden).astype(np.float32)
    parts = DeviceBuffer.empty((hq * 8 * (d + 2),), np.float32)
    scale = 1 / 16
    splits = ops.attention_partials(up(q), up(kc), up(vc), parts, batch=1, num_heads=hq, num_kv_heads=hkv,
                                    head_dim=d, kv_len=0, kv_stride=maxs, scale=scale, max_splits=max_splits,
                                    kv_len_buffer=up(np.array([kv_len], np.int32)))
    assert 1 <= splits <= max_splits
    out = DeviceBuffer.empty((hidden,), np.float32)
    ops.matmul_q4k_attn_out(up(wo), parts, splits, hq, d, out, hidden, residual=up(res))
    attn = ora.attn_decode(q, kc, vc, hq, hkv, d, kv_len, maxs, scale).reshape(-1)
    want = ora.residual(ora.q4k_gemv(wo, attn, hidden, hq * d), res)
    assert rel_l2(out.download(), want) < 1e-5
    # in place (output = residual, as the decode step calls it): the K range
    # is split over workgroups that add their row sums atomically
    inplace = up(res)
    ops.matmul_q4k_attn_out(up(wo), parts, splits, hq, d, inplace, hidden, residual=inplace)
    assert rel_l2(inplace.download(), want) < 1e-5
    # the same partials through the plain attention op give the same activation
    full = DeviceBuffer.empty((1, hq, d), np.float32)
    ops.attention(up(q), up(kc), up(vc), full, batch=1, num_heads=hq, num_kv_heads=hkv, head_dim=d,
                  kv_len=kv_len, kv_stride=maxs, scale=scale)
    assert rel_l2(full.download().reshape(-1), attn) < 1e-5


def test_fills_replay_in_graphs(dev):
    # Empty reductions clear their outputs and doe_memset fills bytes with a
    # kernel (no memset node): captured once, replayed with garbage written
    # in between, every replay rewrites the outputs.
    import ctypes as C

    from doe_amd import Graph, Stream, _lib

    s = Stream()
    sp = C.c_void_p(s.handle)
    m, n = 37, 300
    c = DeviceBuffer.empty((m, n), np.float32)
    y = DeviceBuffer.empty((n,), np.float32)
    raw = DeviceBuffer(4096)
    dummy = DeviceBuffer(1 << 12)

    def body():
        _lib.call("doe_q4k_gemm", C.c_void_p(dummy.ptr), C.c_void_p(dummy.ptr), C.c_void_p(c.ptr), m, n, 0, sp)
        _lib.call("doe_q4k_gemv", C.c_void_p(dummy.ptr), C.c_void_p(dummy.ptr), C.c_void_p(y.ptr), n, 0, sp)
        _lib.call("doe_memset", C.c_void_p(raw.ptr + 3), 0x5A, 1001, sp)   # unaligned head and tail
        _lib.call("doe_memset", C.c_void_p(raw.ptr + 2048), 0x00, 1024, sp)  # aligned

    g = Graph.capture(s, body)
    rng = np.random.default_rng(5)
    for i in range(4):
        c.upload(rng.standard_normal((m, n)).astype(np.float32))
        y.upload(rng.standard_normal(n).astype(np.float32))
        before = rng.integers(0, 256, 4096, dtype=np.uint8)
        raw.upload(before)
        g.launch(s)
        s.synchronize()
        assert not c.download().any() and not y.download().any(), i
        got = raw.download().view(np.uint8)
        want = before.copy()
        want[3:1004] = 0x5A
        want[2048:3072] = 0
        assert np.array_equal(got, want), i
    g.destroy()
    s.destroy()


@pytest.mark.parametrize("nbytes,wgs", [(16, 0), (4096 * 16 + 48, 0), (3 << 20, 7), (1 << 24, 0)])
def test_read_xor_checksum(dev, nbytes, wgs):
    """doe_read_xor_u32 (the read-stream probe beside the HBM copy figure):
    the XOR of every 32-bit word, for word counts that leave remainders in
    its four-deep loop and with a forced small grid."""
    import ctypes as C

    from doe_amd import _lib

    rng = np.random.default_rng(nbytes)
    a = rng.integers(0, 2 ** 32, nbytes // 4, dtype=np.uint64).astype(np.uint32)
    buf = up(a)
    ck = DeviceBuffer.empty((1,), np.uint32)
    _lib.call("doe_read_xor_u32", C.c_void_p(buf.ptr), nbytes, C.c_void_p(ck.ptr), wgs, C.c_void_p(None))
    dev.synchronize()
    assert int(ck.download()[0]) == int(np.bitwise_xor.reduce(a))


def test_device_timestamp_orders_stream_work(dev):
    """doe_device_timestamp: the device clock stored when the stream reaches
    it, so stamps around work on one stream increase, at the rate
    doe_device_timestamp_hz reports (a 1 GiB read takes well over 10 us)."""
    import ctypes as C

    from doe_amd import Stream, _lib

    hz = C.c_int64()
    _lib.call("doe_device_timestamp_hz", C.byref(hz))
    assert hz.value > 0
    s = Stream()
    ts = DeviceBuffer.empty((2,), np.uint64)
    big = DeviceBuffer(1 << 30)
    ck = DeviceBuffer.empty((1,), np.uint32)
    _lib.call("doe_device_timestamp", C.c_void_p(ts.ptr), C.c_void_p(s.handle))
    _lib.call("doe_read_xor_u32", C.c_void_p(big.ptr), big.nbytes, C.c_void_p(ck.ptr), 0, C.c_void_p(s.handle))
    _lib.call("doe_device_timestamp", C.c_void_p(ts.ptr + 8), C.c_void_p(s.handle))
    s.synchronize()
    t = ts.download().astype(np.int64)
    s.destroy()
    big.free()
    assert (t[1] - t[0]) / hz.value > 10e-6
