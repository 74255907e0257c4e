"""Pins the CPU oracle against the reference's golden vectors, known answers and
what the mathematics fixes (closed forms, exact rational arithmetic, invariants,
float64 library routines).  CPU only."""
import math
from fractions import Fraction

import numpy as np
import pytest

from doe_amd import q4k


def _block(ka, **over):
    e = dict(ka["q4k_scale_min_block"])
    e.update(over)
    quant = [i % 16 for i in range(256)]
    return q4k.pack_blocks(np.array([e["d"]]), np.array([e["dmin"]]), np.array([e["scale_bits"]]),
                           np.array([e["min_bits"]]), np.array([quant]))[0]


def test_q4k_constants(known_answers):
    c = known_answers["q4k_constants"]
    assert (c["block_elements"], c["block_bytes"], c["subblocks"], c["subblock_elements"],
            c["quant_bytes_offset"]) == (q4k.BLOCK_ELEMS, q4k.BLOCK_BYTES, 8, 32, 16)


def test_q4k_packer_matches_hand_derived_header(known_answers):
    blk = _block(known_answers)
    want = bytes.fromhex(known_answers["q4k_scale_min_block"]["header_hex_hand_derived"])
    assert bytes(blk[:16]) == want


def test_q4k_unpack_known_answer(ora, known_answers):
    e = known_answers["q4k_scale_min_block"]
    blk = np.zeros(144, np.uint8)
    blk[:16] = np.frombuffer(bytes.fromhex(e["header_hex_hand_derived"]), np.uint8)
    sc, mn, d, dmin = ora.q4k_unpack_scale_min(blk)
    assert sc.tolist() == e["scale_bits"]
    assert mn.tolist() == e["min_bits"]
    assert (d, dmin) == (e["d"], e["dmin"])


def test_q4k_dequant_known_answers(ora, known_answers):
    vals = ora.q4k_dequant_block(_block(known_answers))
    for idx, want in known_answers["q4k_scale_min_block"]["expected_values"].items():
        assert vals[int(idx)] == np.float32(want)
    assert vals.shape == (256,)


def test_q4k_rowwise_tail_padding(ora, known_answers):
    e = known_answers["q4k_rowwise_tail"]
    blocks = [
        q4k.pack_blocks(np.array([e["block_d"]]), np.array([e["block_dmin"]]),
                        np.full((1, 8), e["block_scale_bits"]), np.full((1, 8), e["block_min_bits"]),
                        np.full((1, 256), fill))[0]
        for fill in e["block_quant_fill"]
    ]
    raw = np.concatenate(blocks)
    rows, cols = e["shape"]
    out = ora.q4k_dequant_rowwise(raw, rows, cols).reshape(-1)
    want = np.concatenate([np.full(n, v, np.float32) for v, n in e["expected_runs"]])
    assert out.shape == want.shape
    assert np.array_equal(out, want)


def test_q4k_scale_min_exhaustive_roundtrip(ora):
    # Every 6-bit (scale, min) value in every sub-block position survives
    # pack -> oracle unpack; a swapped byte group or shift fails here.
    rng = np.random.default_rng(1)
    for pos in range(8):
        for s in range(64):
            sc = rng.integers(0, 64, 8)
            mn = rng.integers(0, 64, 8)
            sc[pos] = s
            mn[pos] = 63 - s
            blk = q4k.pack_blocks(np.array([1.0]), np.array([0.5]), sc[None], mn[None],
                                  np.zeros((1, 256), np.uint8))[0]
            gsc, gmn, _, _ = ora.q4k_unpack_scale_min(blk)
            assert gsc.tolist() == sc.tolist() and gmn.tolist() == mn.tolist()


def test_q4k_numpy_unpack_agrees_with_oracle(ora):
    rng = np.random.default_rng(2)
    w = q4k.random_q4k(rng, 7, 512)
    blocks = w.reshape(-1, 144)
    sc, mn, d, dmin = q4k.unpack_scale_min(blocks)
    for i in range(blocks.shape[0]):
        osc, omn, od, odmin = ora.q4k_unpack_scale_min(blocks[i])
        assert osc.tolist() == sc[i].tolist() and omn.tolist() == mn[i].tolist()
        assert od == d[i] and odmin == dmin[i]


def _f16_values():
    # extreme f16 scale factors: smallest subnormal, largest subnormal,
    # smallest normal, ordinary values, largest finite
    return [2.0 ** -24, 1023 * 2.0 ** -24, 2.0 ** -14, 0.0123, 0.5, 3.0, 1000.0, 65504.0]


def test_q4k_dequant_is_one_rounding_of_the_exact_value(ora):
    # Exact rational evaluation of d*sc*q - dmin*m, rounded once to f32
    # (float64 -> float32 casts are RNE, and the Fraction is exactly
    # representable in float64 because all terms are).
    rng = np.random.default_rng(3)
    vals = _f16_values()
    for trial in range(24):
        d = np.float16(vals[trial % len(vals)])
        dmin = np.float16(vals[(trial * 5 + 3) % len(vals)])
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        qv = rng.integers(0, 16, 256)
        blk = q4k.pack_blocks(np.array([d]), np.array([dmin]), sc[None], mn[None], qv[None])[0]
        got = ora.q4k_dequant_block(blk)
        for i in range(0, 256, 7):
            sb = i // 32
            exact = Fraction(float(d)) * sc[sb] * int(qv[i]) - Fraction(float(dmin)) * mn[sb]
            want = np.float32(float(exact))  # float(Fraction) is correctly rounded
            assert float(exact) == exact, "term not representable in float64"
            assert got[i] == want, (trial, i)


def test_interp_gemv_known_answer(ora, known_answers):
    e = known_answers["interp_fused_gemv"]
    y = ora.f32_gemv(np.array(e["W"], np.float32), np.array(e["x"], np.float32))
    assert y.tolist() == e["y"]


def test_fixture_fused_gemv(ora, known_answers):
    e = known_answers["fixture_fused_gemv"]
    y = ora.f32_gemv(np.array(e["W"], np.float32), np.array(e["x"], np.float32))
    assert y.tolist() == e["y"]


def test_q4k_gemv_matches_float64_dense(ora):
    rng = np.random.default_rng(4)
    for n, k in [(5, 256), (3, 300), (17, 1024), (8, 2304)]:
        w = q4k.random_q4k(rng, n, k)
        x = rng.standard_normal(k).astype(np.float32)
        y = ora.q4k_gemv(w, x, n, k)
        wd = ora.q4k_dequant_rowwise(w, n, k).astype(np.float64)
        ref = wd @ x.astype(np.float64)
        assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 1e-5
        # row-range variant is the same computation
        part = ora.q4k_gemv(w, x, n, k, rows=(1, n))
        assert np.array_equal(part[1:], y[1:])
        # and so is the rows-over-threads form (the all-core CPU baseline)
        for threads in (1, 3, 8):
            assert np.array_equal(ora.q4k_gemv_threads(w, x, n, k, threads), y)


def test_q4k_gemv_one_hot_selects_a_column(ora):
    rng = np.random.default_rng(5)
    n, k = 6, 512
    w = q4k.random_q4k(rng, n, k)
    wd = ora.q4k_dequant_rowwise(w, n, k)
    for col in (0, 31, 32, 255, 256, 300, 511):
        x = np.zeros(k, np.float32)
        x[col] = 1.0
        assert np.array_equal(ora.q4k_gemv(w, x, n, k), wd[:, col])


def test_interp_rmsnorm_known_answer(ora, known_answers):
    e = known_answers["interp_rms_norm"]
    out = ora.rmsnorm(np.array(e["input"], np.float32), np.array(e["weight"], np.float32), e["eps"])
    assert out.tolist() == e["output"]


def test_fixture_rmsnorm_transcript(ora, known_answers):
    e = known_answers["fixture_rmsnorm"]
    out = ora.rmsnorm(np.array(e["input"], np.float32), np.array(e["weight"], np.float32), e["eps"])
    want = np.array(e["output"], np.float32)
    ulp = np.abs(out.view(np.int32) - want.view(np.int32))
    assert ulp.max() <= 1, (out, want)


def test_rmsnorm_weight_offset_and_float64(ora):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((3, 2304)).astype(np.float32)
    w = (0.1 * rng.standard_normal(2304)).astype(np.float32)
    out = ora.rmsnorm(x, w, 1e-6, weight_offset=True)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(axis=1, keepdims=True) + 1e-6) * (1.0 + w.astype(np.float64))
    assert np.abs(out - ref).max() / np.abs(ref).max() < 1e-5


def test_emulator_rope_known_answer(ora, known_answers):
    e = known_answers["emulator_rope"]
    out = ora.rope_pairs(np.array(e["input"], np.float32), np.array(e["cos"], np.float32),
                         np.array(e["sin"], np.float32), e["head_dim"], e["num_pairs"], e["interleaved"])
    assert out.tolist() == e["output"]


def test_rope_rotate_half_properties(ora):
    rng = np.random.default_rng(7)
    seq, heads, dim, maxpos = 3, 2, 8, 16
    table = ora.rope_table(maxpos, dim, 10000.0)
    # closed form of the table
    half = dim // 2
    for p in (0, 1, 5, 15):
        for i in range(half):
            ang = p * 10000.0 ** (-2.0 * i / dim)
            assert table[(p * half + i) * 2] == np.float32(math.cos(ang))
            assert table[(p * half + i) * 2 + 1] == np.float32(math.sin(ang))
    x = rng.standard_normal(seq * heads * dim).astype(np.float32)
    # position 0 is the identity
    assert np.array_equal(ora.rope(x, table, seq, heads, dim, 0)[: heads * dim], x[: heads * dim])
    out = ora.rope(x, table, seq, heads, dim, 4).reshape(seq, heads, dim).astype(np.float64)
    xr = x.reshape(seq, heads, dim).astype(np.float64)
    # each (i, i + D/2) pair keeps its norm and rotates by pos * theta_i
    for s in range(seq):
        pos = s + 4
        for i in range(half):
            a = xr[:, :, i][s] + 1j * xr[:, :, i + half][s]
            b = out[:, :, i][s] + 1j * out[:, :, i + half][s]
            ang = pos * 10000.0 ** (-2.0 * i / dim)
            assert np.allclose(b, a * np.exp(1j * ang), rtol=1e-5, atol=1e-5)
    # rotate-half equals the split-pair emulator form with this position's table
    cos_t = np.array([table[((5) * half + i) * 2] for i in range(half)], np.float32)
    sin_t = np.array([table[((5) * half + i) * 2 + 1] for i in range(half)], np.float32)
    row = x[heads * dim: heads * dim + dim]
    split = ora.rope_pairs(row, cos_t, sin_t, dim, half, interleaved=False)
    assert np.array_equal(split, ora.rope(x, table, seq, heads, dim, 4)[heads * dim: heads * dim + dim])


def _attn_f64(q, k, v, scale):
    s = (k.astype(np.float64) @ q.astype(np.float64)) * scale
    p = np.exp(s - s.max())
    p /= p.sum()
    return p @ v.astype(np.float64)


def test_emulator_attention_known_answer(ora, known_answers):
    e = known_answers["emulator_attention_decode"]
    q = np.array(e["query"], np.float32)
    kk = np.array(e["key"], np.float16)
    vv = np.array(e["val"], np.float16)
    out = ora.attn_decode(q[None], kk, vv, 1, 1, e["head_dim"], e["kv_len"], e["kv_len"], e["scale"])[0]
    w = math.exp(-1.0)
    want = [(10 + w * 20) / (1 + w), (11 + w * 21) / (1 + w)]
    # The emulator evaluates in f64 and stores f32 (its test allows 6 places);
    # this oracle follows the f32 interpreter, which lands within 2 f32 ulp.
    for a, b in zip(out, want):
        assert abs(float(a) - b) <= 2 * np.spacing(np.float32(b))


def test_attention_invariants_and_gqa(ora):
    rng = np.random.default_rng(8)
    hq, hkv, d, t = 8, 4, 16, 40
    q = rng.standard_normal((hq, d)).astype(np.float32)
    k = rng.standard_normal((hkv, t, d)).astype(np.float16)
    v = rng.standard_normal((hkv, t, d)).astype(np.float16)
    scale = 1.0 / math.sqrt(d)
    out = ora.attn_decode(q, k, v, hq, hkv, d, t, t, scale)
    for h in range(hq):
        ref = _attn_f64(q[h], k[h // 2], v[h // 2], scale)
        assert np.abs(out[h] - ref).max() < 1e-5
    # a single key returns its value row
    one = ora.attn_decode(q, k, v, hq, hkv, d, 1, t, scale)
    for h in range(hq):
        assert np.allclose(one[h], v[h // 2, 0].astype(np.float32), atol=1e-6)
    # equal scores (q = 0) average V
    zero = ora.attn_decode(np.zeros_like(q), k, v, hq, hkv, d, t, t, scale)
    assert np.allclose(zero[0], v[0].astype(np.float64).mean(axis=0), atol=1e-5)
    # [pos][kv_head][dim] layout gives the same answer
    k1 = np.ascontiguousarray(k.transpose(1, 0, 2))
    v1 = np.ascontiguousarray(v.transpose(1, 0, 2))
    out1 = ora.attn_decode(q, k1, v1, hq, hkv, d, t, t, scale, kv_layout=1)
    assert np.array_equal(out, out1)
    # sliding window keeps the last `window` keys only
    win = ora.attn_decode(q, k, v, hq, hkv, d, t, t, scale, sliding_window=8)
    ref = _attn_f64(q[3], k[1, t - 8:], v[1, t - 8:], scale)
    assert np.abs(win[3] - ref).max() < 1e-5


def test_attention_prefill_causal_matches_float64(ora):
    rng = np.random.default_rng(9)
    hq, hkv, d, s = 4, 2, 8, 12
    q = rng.standard_normal((s, hq, d)).astype(np.float32)
    k = rng.standard_normal((hkv, s, d)).astype(np.float32)
    v = rng.standard_normal((hkv, s, d)).astype(np.float32)
    out = ora.attn_prefill(q, k, v, hq, hkv, d, s, s, 0, 0.3)
    for i in range(s):
        for h in range(hq):
            ref = _attn_f64(q[i, h], k[h // 2, : i + 1], v[h // 2, : i + 1], 0.3)
            assert np.abs(out[i, h] - ref).max() < 1e-5
    # first query sees only key 0
    assert np.allclose(out[0, 0], v[0, 0], atol=1e-6)


def test_geglu_matches_closed_form(ora):
    x = np.linspace(-40, 40, 4001, dtype=np.float32)
    up = np.linspace(-2, 2, 4001, dtype=np.float32)
    out = ora.geglu(x, up)
    xd = x.astype(np.float64)
    inner = np.clip(0.7978845608028654 * (xd + 0.044715 * xd ** 3), -15, 15)
    ref = 0.5 * xd * (1 + np.tanh(inner)) * up
    assert np.abs(out - ref).max() <= 1e-5 * np.abs(ref).max()
    # GELU(0) = 0 and the clamp makes GELU(x) = x exactly for large x
    assert ora.geglu(np.array([0.0, 30.0], np.float32), np.ones(2, np.float32)).tolist() == [0.0, 30.0]


def test_argmax_known_answers(ora, known_answers):
    e = known_answers["emulator_sample"]
    assert ora.argmax(np.array(e["logits"], np.float32)) == e["token"]
    assert ora.argmax(np.array(e["tie_logits"], np.float32)) == e["tie_token"]
    rng = np.random.default_rng(10)
    for _ in range(20):
        x = rng.integers(-5, 5, 1000).astype(np.float32)
        assert ora.argmax(x) == int(np.argmax(x))  # numpy returns the first maximum too


def test_f16_bf16_conversions(ora):
    rng = np.random.default_rng(11)
    vals = np.concatenate([
        rng.standard_normal(2000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 2000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 2 ** -24, 2 ** -25, 3 * 2 ** -26,
                  2 ** -14, 2 ** -14 * (1 - 2 ** -11), np.inf, -np.inf], np.float32),
    ]).astype(np.float32)
    lib = ora.lib()
    for v in vals:
        h = lib.ora_f32_to_f16(float(v))
        assert h == int(np.float32(v).astype(np.float16).view(np.uint16)), v
        assert lib.ora_f16_to_f32(h) == float(np.float16(v))
    # bf16 RNE (ulp 2^-7 at 1.0): 1 + 2^-8 is a tie -> even (1.0); 1 + 3*2^-9 rounds up
    assert lib.ora_f32_to_bf16(1.0 + 2 ** -8) == 0x3F80
    assert lib.ora_f32_to_bf16(1.0 + 3 * 2 ** -9) == 0x3F81
    assert lib.ora_bf16_to_f32(0x3F81) == 1.0078125


def test_int4g32_gemv_closed_form(ora):
    # complex_fused_gemv_dequant.wgsl:18-23: element idx sits at bits
    # 4*(idx%8) of word idx/8, value nib - 8, scale [row][col/32].
    rng = np.random.default_rng(12)
    m, n, k = 2, 3, 64
    nib = rng.integers(0, 16, (n, k)).astype(np.uint32)
    words = np.zeros(n * k // 8, np.uint32)
    flat = nib.reshape(-1)
    for i in range(flat.size):
        words[i // 8] |= flat[i] << (4 * (i % 8))
    scales = np.abs(rng.standard_normal((n, k // 32))).astype(np.float16)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = ora.int4g32_gemv(words, scales, x, m, n, k)
    wd = (nib.astype(np.float64) - 8.0) * np.repeat(scales.astype(np.float64), 32, axis=1)
    ref = x.astype(np.float64) @ wd.T
    assert np.abs(y - ref).max() < 1e-5 * np.abs(ref).max()
    # hand-computed: word 0x76543210 holds nibbles 0..7 -> values -8..-1
    y1 = ora.int4g32_gemv(np.array([0x76543210, 0x88888888, 0x88888888, 0x88888888], np.uint32),
                          np.array([1.0], np.float16), np.ones((1, 32), np.float32), 1, 1, 32)
    assert y1.tolist() == [[-36.0]]


def test_kv_write_and_gather(ora):
    rng = np.random.default_rng(13)
    kvh, maxs, d = 2, 5, 4
    kc = np.zeros((kvh, maxs, d), np.float16)
    vc = np.zeros((kvh, maxs, d), np.float16)
    kp = rng.standard_normal((kvh, d)).astype(np.float32)
    vp = rng.standard_normal((kvh, d)).astype(np.float32)
    ora.kv_write(kp, vp, kc, vc, kvh, maxs, d, 3)
    assert np.array_equal(kc[:, 3], kp.astype(np.float16)) and np.array_equal(vc[:, 3], vp.astype(np.float16))
    assert not kc[:, :3].any() and not kc[:, 4].any()
    with pytest.raises(ValueError):
        ora.kv_write(kp, vp, kc, vc, kvh, maxs, d, 5)  # pos >= max_seq_len is an error
    table = rng.standard_normal((6, 3)).astype(np.float16)
    out = ora.embed_gather(table, np.array([4, 0, 9, -1], np.int32))
    assert np.array_equal(out[0], table[4].astype(np.float32))
    assert np.array_equal(out[1], table[0].astype(np.float32))
    assert not out[2].any() and not out[3].any()


def test_q4k_gemm_matches_float64_and_sampled(ora):
    rng = np.random.default_rng(14)
    m, n, k = 5, 7, 512
    a = rng.standard_normal((m, k)).astype(np.float32)
    a_bf16 = (a.view(np.uint32) >> 16).astype(np.uint16)  # truncation is fine for an input
    b = q4k.random_q4k(rng, n, k)
    c = ora.q4k_gemm(a_bf16, b, m, n, k)
    a64 = (a_bf16.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    ref = a64 @ ora.q4k_dequant_rowwise(b, n, k).astype(np.float64).T
    assert np.abs(c - ref).max() < 1e-5 * np.abs(ref).max()
    mi = np.array([0, 4, 2])
    ni = np.array([6, 0, 3])
    assert np.array_equal(ora.q4k_gemm_sampled(a_bf16, b, m, n, k, mi, ni), c[mi, ni])


def test_f16_gemv_matches_float64_dense(ora):
    # lm_head_gemv.wgsl:78-180 (transpose_b = 1): C[n] = alpha * sum_k A[k] *
    # f32(B[n][k]).  float64 dense at the decode widths (2304, 5120) and an
    # odd K; alpha != 1 on both signs.
    rng = np.random.default_rng(15)
    for n, k, alpha in [(37, 2304, 0.37), (19, 5120, -2.5), (23, 777, 1.0), (5, 1, 0.125)]:
        b = (0.02 * rng.standard_normal((n, k))).astype(np.float16)
        a = rng.standard_normal(k).astype(np.float32)
        c = ora.f16_gemv(b, a, alpha)
        ref = alpha * (b.astype(np.float64) @ a.astype(np.float64))
        # f32 left-fold rounding: ~sqrt(k) ulps; one dropped term would cost ~1e-2
        assert np.linalg.norm(c - ref) / np.linalg.norm(ref) < 1e-5, (n, k, alpha)
        # alpha scales the finished sum once (f32 product), not each term
        c1 = ora.f16_gemv(b, a, 1.0)
        assert np.array_equal(c, (c1 * np.float32(alpha)).astype(np.float32))


def test_f16_gemv_one_hot_and_zero(ora):
    rng = np.random.default_rng(16)
    n, k = 9, 300
    b = rng.standard_normal((n, k)).astype(np.float16)
    for col in (0, 1, 150, 299):
        a = np.zeros(k, np.float32)
        a[col] = 1.0
        # a one-hot activation selects column `col` exactly (power-of-two alpha)
        assert np.array_equal(ora.f16_gemv(b, a, 0.25), b[:, col].astype(np.float32) * np.float32(0.25))
    # the reference transcript's all-zero lm_head input gives all-zero logits
    assert not ora.f16_gemv(b, np.zeros(k, np.float32), 1.0).any()
    # rows are independent: row j only reads B[j]
    a = rng.standard_normal(k).astype(np.float32)
    assert np.array_equal(ora.f16_gemv(b[3:5], a), ora.f16_gemv(b, a)[3:5])


def test_lm_head_gemv_layouts_and_rows_match_float64(ora):
    # lm_head_gemv.wgsl:105-143: transpose_b = 1 reads B[col*K + k], 0 reads
    # B[k*N + col].  float64 dense for both layouts, odd and decode-width K,
    # several activation rows; alpha != 1.
    rng = np.random.default_rng(17)
    for m, n, k, alpha in [(1, 29, 2304, 0.5), (3, 17, 777, -1.25), (5, 8, 1, 2.0), (2, 40, 5120, 1.0)]:
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = (0.02 * rng.standard_normal((n, k))).astype(np.float16)
        ref = alpha * (a.astype(np.float64) @ b.astype(np.float64).T)
        c1 = ora.lm_head_gemv(a, b, alpha, transpose_b=1)
        c0 = ora.lm_head_gemv(a, np.ascontiguousarray(b.T), alpha, transpose_b=0)
        assert c1.shape == c0.shape == (m, n)
        assert np.linalg.norm(c1 - ref) / np.linalg.norm(ref) < 1e-5, (m, n, k)
        # the two layouts name the same matrix: same sums in the same order
        assert np.array_equal(c0, c1), (m, n, k)
        # a transposed index (B[k*K + col]) would only agree for square B
        if n != k and m == 1:
            assert np.array_equal(c1[0], ora.f16_gemv(b, a[0], alpha))


def test_lm_head_gemv_rows_are_independent(ora):
    rng = np.random.default_rng(18)
    m, n, k = 6, 11, 300
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float16)
    c = ora.lm_head_gemv(a, b, 1.0, transpose_b=0)
    for r in range(m):
        assert np.array_equal(ora.lm_head_gemv(a[r], b, 1.0, transpose_b=0)[0], c[r])
    # a one-hot row selects row k of the [K][N] matrix exactly
    e = np.zeros((1, k), np.float32)
    e[0, 123] = 1.0
    assert np.array_equal(ora.lm_head_gemv(e, b, 1.0, transpose_b=0)[0], b[123].astype(np.float32))
    # transpose_b is a flag: other values are rejected before any access
    assert ora.lib().ora_lm_head_gemv(None, None, None, 1, 1, 1, 1.0, 2) == -1


def test_gather_f32_interpreter_known_answers(ora, known_answers):
    e = known_answers["interp_gather"]
    out = ora.gather_f32(np.array(e["table_f32"], np.float32), np.array(e["indices_u32"], np.uint32))
    assert np.array_equal(out, np.array(e["output"], np.float32))
    # an index one past the table rejects the run instead of clamping to the last row
    e = known_answers["interp_gather_oob"]
    with pytest.raises(ValueError):
        ora.gather_f32(np.array(e["table_f32"], np.float32), np.array(e["indices_u32"], np.uint32))
    # the largest u32 is not read as -1
    with pytest.raises(ValueError):
        ora.gather_f32(np.ones((3, 2), np.float32), np.array([0, 0xFFFFFFFF], np.uint32))
    # in range: a row copy, bit for bit (NaN payloads and -0.0 included)
    rng = np.random.default_rng(19)
    table = rng.standard_normal((50, 7)).astype(np.float32)
    table[3, 1] = -0.0
    table.view(np.uint32)[4, 2] = 0x7FC01234
    ids = rng.integers(0, 50, 40).astype(np.uint32)
    ids[:2] = [3, 4]
    got = ora.gather_f32(table, ids)
    assert np.array_equal(got.view(np.uint32), table[ids].view(np.uint32))


def test_residual_is_ieee_f32_addition(ora):
    # run_csl_webgpu_emulator.mjs:482-489 / residual.wgsl: out = a + b, one f32
    # addition per element: bit-equal to numpy's IEEE float32 add, including
    # signed zeros, infinities, overflow, subnormals and NaN.
    rng = np.random.default_rng(17)
    special = np.array([0.0, -0.0, -0.0, np.inf, -np.inf, np.inf, np.nan, 3e38, -3e38, 1e-45, -1e-45,
                        2.0 ** -126, 1.0, 1.0], np.float32)
    other = np.array([-0.0, 0.0, -0.0, 1.0, -np.inf, -np.inf, 1.0, 3e38, -3e38, 1e-45, 1e-45,
                      -2.0 ** -127, 2.0 ** -24, 2.0 ** -23], np.float32)
    a = np.concatenate([special, rng.standard_normal(4000).astype(np.float32) * 1e3])
    b = np.concatenate([other, rng.standard_normal(4000).astype(np.float32)])
    out = ora.residual(a, b)
    want = np.add(a, b, dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(out), nan)
    assert np.array_equal(out[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # the cases that separate a correct add from a plausible slip
    assert np.signbit(out[0]) == False and np.signbit(out[2]) == True  # +0 + -0 = +0; -0 + -0 = -0
    assert np.isnan(out[5]) and out[7] == np.inf and out[8] == -np.inf  # inf - inf; overflow
    assert out[12] == 1.0 and out[13] == np.float32(1.0 + 2.0 ** -23)  # a tie rounds to even


# Every function the oracle header declares and the tests above that pin it
# against something other than its own formula (golden vectors, exact
# arithmetic, float64 library routines, invariants).
PINS = {
    "ora_f16_to_f32": ["test_f16_bf16_conversions"],
    "ora_f32_to_f16": ["test_f16_bf16_conversions"],
    "ora_bf16_to_f32": ["test_f16_bf16_conversions"],
    "ora_f32_to_bf16": ["test_f16_bf16_conversions"],
    "ora_q4k_unpack_scale_min": ["test_q4k_unpack_known_answer", "test_q4k_scale_min_exhaustive_roundtrip"],
    "ora_q4k_dequant_block": ["test_q4k_dequant_known_answers", "test_q4k_dequant_is_one_rounding_of_the_exact_value"],
    "ora_q4k_dequant_rowwise": ["test_q4k_rowwise_tail_padding"],
    "ora_q4k_gemv": ["test_q4k_gemv_matches_float64_dense", "test_q4k_gemv_one_hot_selects_a_column"],
    "ora_q4k_gemv_rows": ["test_q4k_gemv_matches_float64_dense"],
    "ora_q4k_gemm_sampled": ["test_q4k_gemm_matches_float64_and_sampled"],
    "ora_q4k_gemm": ["test_q4k_gemm_matches_float64_and_sampled"],
    "ora_f32_gemv": ["test_interp_gemv_known_answer", "test_fixture_fused_gemv"],
    "ora_f16_gemv": ["test_f16_gemv_matches_float64_dense", "test_f16_gemv_one_hot_and_zero"],
    "ora_lm_head_gemv": ["test_lm_head_gemv_layouts_and_rows_match_float64", "test_lm_head_gemv_rows_are_independent"],
    "ora_int4g32_gemv": ["test_int4g32_gemv_closed_form"],
    "ora_q8_0_element_count": ["test_q8_0.py::test_reference_size_checks"],
    "ora_q8_0_dequant": ["test_q8_0.py::test_known_block_bytes", "test_q8_0.py::test_matches_int4_group32_oracle"],
    "ora_q8_0_gemv": ["test_q8_0.py::test_tail_block_residual_and_brute_force"],
    "ora_rmsnorm": ["test_interp_rmsnorm_known_answer", "test_fixture_rmsnorm_transcript",
                    "test_rmsnorm_weight_offset_and_float64"],
    "ora_rope_table": ["test_rope_rotate_half_properties"],
    "ora_rope": ["test_rope_rotate_half_properties"],
    "ora_rope_pairs": ["test_emulator_rope_known_answer"],
    "ora_geglu": ["test_geglu_matches_closed_form"],
    "ora_residual": ["test_residual_is_ieee_f32_addition"],
    "ora_argmax": ["test_argmax_known_answers"],
    "ora_embed_gather": ["test_kv_write_and_gather"],
    "ora_gather_f32": ["test_gather_f32_interpreter_known_answers"],
    "ora_kv_write": ["test_kv_write_and_gather"],
    "ora_attn_decode": ["test_emulator_attention_known_answer", "test_attention_invariants_and_gqa"],
    "ora_attn_prefill": ["test_attention_prefill_causal_matches_float64"],
    "ora_gated": ["test_oracle_ssm.py::test_gated_closed_forms_and_clamps"],
    "ora_l2_normalize": ["test_oracle_ssm.py::test_l2_normalize_fixture_closed_form_and_eps"],
    "ora_conv1d_depthwise": ["test_oracle_ssm.py::test_conv1d_depthwise_brute_force_fixture_and_causality"],
    "ora_linear_attention": ["test_oracle_ssm.py::test_linear_attention_recurrence_and_closed_forms"],
}


def test_every_oracle_function_has_a_pinning_test():
    import ast
    import re

    from conftest import ROOT

    header = (ROOT / "oracle" / "doe_oracle.h").read_text()
    header = re.sub(r"/\*.*?\*/", "", header, flags=re.S)
    declared = set(re.findall(r"\b(ora_[a-z0-9_]+)\s*\(", header))
    assert declared == set(PINS), (sorted(declared - set(PINS)), sorted(set(PINS) - declared))

    def test_names(path):
        tree = ast.parse(path.read_text())
        return {n.name for n in tree.body if isinstance(n, ast.FunctionDef) and n.name.startswith("test_")}

    here = test_names(ROOT / "tests" / "test_oracle_golden.py")
    for fn, tests in PINS.items():
        assert tests, fn
        for t in tests:
            if "::" in t:
                mod, name = t.split("::")
                assert name in test_names(ROOT / "tests" / mod), (fn, t)
            else:
                assert t in here, (fn, t)
