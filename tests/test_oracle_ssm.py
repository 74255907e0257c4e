"""The oracle's restatements of the Qwen 3.6 graph ops (gated activations,
l2_normalize, conv1d_depthwise, gated-DeltaNet linear_attention;
reference_interpreter.zig:954-1052, 1284-1596), pinned on the CPU by what the
mathematics fixes: float64 closed forms, the interpreter's ±15 clamps at
points where they change the result, brute-force loops and recurrences on
tiny inputs, and invariants a dropped term or a swapped operand breaks."""
import math

import numpy as np


def _sig64(x):
    z = np.clip(-np.asarray(x, np.float64), -15.0, 15.0)
    return 1.0 / (1.0 + np.exp(z))


def test_gated_closed_forms_and_clamps(ora):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(200) * 4, [0.0, -0.0, 20.0, -20.0, 15.0, -15.0, 40.0, -40.0]])
    u = rng.standard_normal(x.size)
    x32, u32 = x.astype(np.float32), u.astype(np.float32)
    x64 = x32.astype(np.float64)
    silu = ora.gated(x32, u32, "silu").astype(np.float64)
    sig = ora.gated(x32, u32, "sigmoid").astype(np.float64)
    gelu = ora.gated(x32, u32, "gelu")
    np.testing.assert_allclose(silu, x64 * _sig64(x64) * u32, rtol=2e-6, atol=1e-30)
    np.testing.assert_allclose(sig, _sig64(x64) * u32, rtol=2e-6, atol=1e-30)
    # the clamp: exp(-z) is taken at z = +-15, not at the argument itself
    ones = np.ones(2, np.float32)
    s = ora.gated(np.array([-20.0, -40.0], np.float32), ones, "sigmoid")
    assert np.allclose(s, 1.0 / (1.0 + math.exp(15.0)), rtol=1e-6)  # both clamped to the same value
    assert abs(s[0] - 1.0 / (1.0 + math.exp(20.0))) > 1e-7          # not the unclamped sigmoid(-20)
    si = ora.gated(np.array([20.0], np.float32), ones[:1], "silu")[0]
    assert abs(si - 20.0 / (1.0 + math.exp(-15.0))) < 4e-6  # two f32 ulps at 20
    assert si != np.float32(20.0)  # the unclamped 20 / (1 + e^-20) rounds to 20 in f32
    # gelu is the GeGLU step (tanh inner clamp)
    assert np.array_equal(gelu, ora.geglu(x32, u32))
    # act(x) * input, not act(input) * x
    assert not np.allclose(ora.gated(u32, x32, "silu"), silu)


def test_l2_normalize_fixture_closed_form_and_eps(ora):
    v = np.array([0.5, -0.25, 0.125, 0.75], np.float32)  # bench/fixtures/tsir-bootstrap-inputs/ssm_l2_normalize.json
    got = ora.l2_normalize(v, 1e-6).astype(np.float64)
    want = v / math.sqrt(float(np.sum(v.astype(np.float64) ** 2)) + 1e-6)
    np.testing.assert_allclose(got, want, rtol=1e-6)
    rng = np.random.default_rng(2)
    rows = rng.standard_normal((5, 128)).astype(np.float32) * rng.uniform(0.01, 100, (5, 1)).astype(np.float32)
    out = ora.l2_normalize(rows, 1e-6).astype(np.float64)
    np.testing.assert_allclose(np.linalg.norm(out, axis=1), 1.0, rtol=1e-5)  # unit rows
    np.testing.assert_allclose(out * np.linalg.norm(rows.astype(np.float64), axis=1, keepdims=True), rows,
                               rtol=2e-5, atol=1e-6)  # parallel to the input
    assert np.array_equal(ora.l2_normalize(np.zeros((1, 8), np.float32)), np.zeros((1, 8), np.float32))
    # eps inside the root: a tiny row does not blow up
    tiny = ora.l2_normalize(np.array([1e-4, 0.0], np.float32), 1e-6)[0]
    assert abs(tiny - 1e-4 / math.sqrt(1e-8 + 1e-6)) < 1e-6


def test_conv1d_depthwise_brute_force_fixture_and_causality(ora):
    # the bootstrap fixture (bench/fixtures/tsir-bootstrap-inputs/
    # ssm_conv1d_depthwise.json): one token, 4 channels, kernel_size 1
    x = np.array([[0.5, -0.25, 0.125, 0.75]], np.float32)
    w = np.array([[0.25], [-0.125], [0.5], [-0.25]], np.float32)
    b = np.array([0.0, 0.125, -0.125, 0.25], np.float32)
    assert np.array_equal(ora.conv1d_depthwise(x, w, b)[0], x[0] * w[:, 0] + b)
    # brute force in the interpreter's order (f32 products and sums), 4 taps
    rng = np.random.default_rng(3)
    T, Cn, K = 9, 6, 4
    x = rng.standard_normal((T, Cn)).astype(np.float32)
    w = rng.standard_normal((Cn, K)).astype(np.float32)
    b = rng.standard_normal(Cn).astype(np.float32)
    want = np.zeros((T, Cn), np.float32)
    for t in range(T):
        for c in range(Cn):
            acc = np.float32(b[c])
            for k in range(K):
                ti = t - (K - 1 - k)
                if ti >= 0:
                    acc = np.float32(acc + np.float32(x[ti, c] * w[c, k]))
            want[t, c] = acc
    got = ora.conv1d_depthwise(x, w, b)
    assert np.array_equal(got, want)
    # float64 convolution: weight tap K-1 meets the current token
    for c in range(Cn):
        full = np.convolve(x[:, c].astype(np.float64), w[c, ::-1].astype(np.float64))[:T] + b[c]
        np.testing.assert_allclose(got[:, c], full, rtol=1e-5, atol=1e-6)
    # causal: a later token does not change earlier outputs; no bias = 0
    x2 = x.copy()
    x2[6:] += 1.0
    assert np.array_equal(ora.conv1d_depthwise(x2, w, b)[:6], got[:6])
    assert np.array_equal(ora.conv1d_depthwise(x, w, None), ora.conv1d_depthwise(x, w, np.zeros(Cn, np.float32)))


def _deltanet64(q, k, v, g, S, a_log):
    S = S.astype(np.float64).copy()
    out = np.zeros(q.shape, np.float64)
    T, H, Vd = q.shape
    for t in range(T):
        for h in range(H):
            alpha = 1.0 - math.exp(-a_log[h])
            for d in range(Vd):
                dot = S[h, d] @ k[t, h]
                S[h, d] = (1.0 - alpha) * S[h, d] + alpha * (q[t, h, d] - dot) * k[t, h]
            out[t, h] = S[h] @ v[t, h] + q[t, h] / (1.0 + np.exp(-g[t, h].astype(np.float64)))
    return S, out


def test_linear_attention_recurrence_and_closed_forms(ora):
    rng = np.random.default_rng(4)
    T, H, Kd, Vd = 5, 2, 3, 4
    q = rng.standard_normal((T, H, Vd)).astype(np.float32)
    k = rng.standard_normal((T, H, Kd)).astype(np.float32) * 0.5
    v = rng.standard_normal((T, H, Kd)).astype(np.float32)
    g = rng.standard_normal((T, H, Vd)).astype(np.float32)
    S0 = rng.standard_normal((H, Vd, Kd)).astype(np.float32)
    a_log = np.array([0.5, 1.5], np.float32)
    S, out = ora.linear_attention(q, k, v, g, S0, a_log)
    S64, out64 = _deltanet64(q, k, v, g, S0, a_log)
    np.testing.assert_allclose(S, S64, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out, out64, rtol=1e-5, atol=1e-6)
    # a_log NULL is the interpreter's 0.5 in every head
    S_n, out_n = ora.linear_attention(q, k, v, g, S0, None)
    S_h, out_h = ora.linear_attention(q, k, v, g, S0, np.full(H, 0.5, np.float32))
    assert np.array_equal(S_n, S_h) and np.array_equal(out_n, out_h)
    # k = 0: the state only decays by exp(-A_log) and the output is S.v + sigmoid(g) q
    kz = np.zeros_like(k[:1])
    S1, o1 = ora.linear_attention(q[:1], kz, v[:1], g[:1], S0, None)
    np.testing.assert_allclose(S1, S0 * math.exp(-0.5), rtol=1e-6)
    want = np.einsum("hdk,hk->hd", S1.astype(np.float64), v[0].astype(np.float64)) + q[0] / (1 + np.exp(-g[0].astype(np.float64)))
    np.testing.assert_allclose(o1[0], want, rtol=1e-5, atol=1e-6)
    # zero state, k = e_1: row d of the new state is alpha q[d] e_1
    e = np.zeros((1, H, Kd), np.float32)
    e[0, :, 1] = 1.0
    S2, _ = ora.linear_attention(q[:1], e, v[:1], g[:1], np.zeros_like(S0), None)
    alpha = 1.0 - math.exp(-0.5)
    np.testing.assert_allclose(S2[:, :, 1], alpha * q[0], rtol=1e-6)
    assert np.all(S2[:, :, [0, 2]] == 0.0)
