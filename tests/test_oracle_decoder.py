"""The oracle decoder's model of the batched prompt's precision, on the CPU:
its f16-operand projection and its attention with f16 probabilities, pinned
on cases whose answers are exact (products and sums representable, so f16
mode must equal the f32 oracle bit for bit; single roundings whose
round-to-nearest-even result is known; softmax weights of exactly 1 and 1/2;
a window that leaves a known subset of keys)."""
import math
from types import SimpleNamespace

import numpy as np

from doe_amd import q8_0


def _bare(heads=2, kv_heads=1, softcap=0.0):
    from oracle.decoder import OracleDecoder

    o = OracleDecoder.__new__(OracleDecoder)
    o.cfg = SimpleNamespace(weight_format="q8_0", heads=heads, kv_heads=kv_heads, attn_softcap=softcap)
    o.f16_operands = False
    o._f16w = {}
    return o


def test_f16_projection_exact_when_operands_are_representable(ora):
    # d = 0.25 and |q| <= 128: every weight is a multiple of 1/4 below 32, and
    # x in halves below 8: both exact in f16, every product and partial sum
    # exact in f32, so the f16-operand GEMV equals the f32 oracle exactly
    rng = np.random.default_rng(5)
    n, k = 7, 96
    w = q8_0.pack_rows(np.full((n, 3), 0.25), rng.integers(-128, 128, (n, 3, 32)))
    x = (rng.integers(-16, 17, k) / 2).astype(np.float32)
    o = _bare()
    exact = o.gemv(w, x, n, k)
    o.f16_operands = True
    assert np.array_equal(o.gemv(w, x, n, k), exact)
    assert np.array_equal(exact, ora.q8_0_dequant(w, n, k).astype(np.float64) @ x.astype(np.float64))


def test_f16_projection_rounds_activation_and_weight_to_nearest_even():
    # weight d * q = (1 + 2^-10) * 3 = 3 + 1.5 ulp of f16 in [2, 4): a tie,
    # rounded to the even mantissa 3 + 2^-8 (d and q are not rounded apart);
    # activations 1 + 2^-11 (a tie -> 1.0) and 1 + 3 * 2^-12 (-> 1 + 2^-10)
    w = q8_0.pack_rows([[1.0 + 2.0 ** -10]], [[[3, 3] + [0] * 30]])
    o = _bare()
    o.f16_operands = True
    for xv, xr in ((1.0 + 2.0 ** -11, 1.0), (1.0 + 3 * 2.0 ** -12, 1.0 + 2.0 ** -10)):
        x = np.zeros(32, np.float32)
        x[0] = xv
        assert o.gemv(w, x, 1, 32)[0] == np.float32(xr * (3.0 + 2.0 ** -8))
    x = np.zeros(32, np.float32)
    x[1] = 1.0
    o.f16_operands = False
    assert o.gemv(w, x, 1, 32)[0] == np.float32((1.0 + 2.0 ** -10) * 3)


def _cache(kv_heads, max_seq, hd, rows):
    c = np.zeros((kv_heads, max_seq, hd), np.float16)
    c[0, : len(rows)] = rows
    return c


def test_f16_attention_equal_scores_give_the_mean():
    # zero keys: every score 0, every probability exactly 1 -> the mean of V
    rng = np.random.default_rng(1)
    hd, n = 4, 5
    kc = np.zeros((1, 8, hd), np.float16)
    vc = _cache(1, 8, hd, rng.standard_normal((n, hd)))
    q = rng.standard_normal(2 * hd).astype(np.float32)
    out = _bare()._attn_p_f16(q, kc, vc, hd, n, 0, 1).reshape(2, hd)
    want = vc[0, :n].astype(np.float64).mean(axis=0)
    np.testing.assert_allclose(out, np.stack([want, want]), rtol=1e-6)
    # a window of 2 keeps keys n-2 and n-1 only
    out = _bare()._attn_p_f16(q, kc, vc, hd, n, 2, 1).reshape(2, hd)
    np.testing.assert_allclose(out[0], vc[0, n - 2:n].astype(np.float64).mean(axis=0), rtol=1e-6)


def test_f16_attention_half_weight_and_underflow():
    # head 0: scores 0 and -ln 2, so exp2 of the log2 scores is 1 and 1/2 (the
    # f16 rounding absorbs the float error); head 1: one key 40 above the
    # other, whose weight 2^-57.7 rounds to 0 in f16 -> exactly that V row
    hd = 4
    kc = _cache(1, 8, hd, [[0, 0, 0, 0], [-1, 0, 0, 0]])
    vc = _cache(1, 8, hd, [[1, 2, 3, 4], [4, 2, -2, 1]])
    q = np.array([2 * math.log(2), 0, 0, 0, -80, 0, 0, 0], np.float32)  # / sqrt(4)
    out = _bare()._attn_p_f16(q, kc, vc, hd, 2, 0, 1).reshape(2, hd)
    v = vc[0, :2].astype(np.float64)
    np.testing.assert_allclose(out[0], (v[0] + 0.5 * v[1]) / 1.5, rtol=1e-6)
    assert np.array_equal(out[1], v[1].astype(np.float32))


def test_f16_attention_rounds_probabilities():
    # second key's weight exp2(-delta) = 1 - 0.3 * 2^-11, within 0.3 f16 ulp
    # below 1, so it rounds to 1 and the output is the plain mean of the two
    # V rows (unrounded it would lie 7.5e-5 of the V difference away)
    hd = 4
    delta = -math.log2(1 - 0.3 * 2.0 ** -11)
    kc = _cache(1, 8, hd, [[0, 0, 0, 0], [-1, 0, 0, 0]])
    vc = _cache(1, 8, hd, [[1, 2, 3, 4], [4, 2, -2, 1]])
    q = np.array([2 * delta * math.log(2), 0, 0, 0, 0, 0, 0, 0], np.float32)
    out = _bare()._attn_p_f16(q, kc, vc, hd, 2, 0, 1).reshape(2, hd)
    v = vc[0, :2].astype(np.float64)
    np.testing.assert_allclose(out[0], (v[0] + v[1]) / 2, rtol=1e-7, atol=0)
    unrounded = (v[0] + 2.0 ** -delta * v[1]) / (1 + 2.0 ** -delta)
    assert np.abs(unrounded - (v[0] + v[1]) / 2).max() > 1e-4


def test_rotation_pair_rows_back_to_plain_order():
    # two heads of head_dim 4: the device holds each head's rows as rotation
    # pairs (dim 0, dim 2, dim 1, dim 3); the oracle reads them in plain order
    from oracle.decoder import plain_rows_from_rotation_pairs

    dev_rows = np.array([[10], [12], [11], [13], [20], [22], [21], [23]])
    got = plain_rows_from_rotation_pairs(dev_rows, 4)
    assert got[:, 0].tolist() == [10, 11, 12, 13, 20, 21, 22, 23]
    # and it undoes the product's own pairing of head_dim 256 rows
    from doe_amd.ops import interleave_rope_rows

    rows = np.arange(2 * 256 * 3).reshape(2 * 256, 3)
    assert np.array_equal(plain_rows_from_rotation_pairs(interleave_rope_rows(rows, 256), 256), rows)
