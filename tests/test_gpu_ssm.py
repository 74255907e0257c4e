"""GPU parity of the Qwen 3.6 graph ops (doe_gated, doe_l2_normalize,
doe_conv1d_depthwise, doe_linear_attention) against the CPU oracle, through
the C ABI: conv1d bit-exact (the interpreter's f32 loop, no fused
multiply-add); the activations within a few f32 ulps (device expf / tanhf
against the host's); l2_normalize and linear_attention (reassociated f32
dot products) within rel-L2 1e-5."""
import numpy as np
import pytest

from doe_amd import DeviceBuffer, DoeError, ops

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def up(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


@pytest.mark.parametrize("kind", ["gelu", "silu", "sigmoid"])
def test_gated(dev, ora, kind):
    rng = np.random.default_rng(len(kind))
    n = 17408 + 3
    g = np.concatenate([rng.standard_normal(n - 6) * 5, [20.0, -20.0, 40.0, -40.0, 0.0, 15.0]]).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    out = DeviceBuffer.empty((n,), np.float32)
    ops.gated(up(g), up(x), out, n, kind)
    got = out.download()
    want = ora.gated(g, x, kind)
    # (near gelu's zero crossing 1 + tanh cancels: compare absolutely there)
    np.testing.assert_allclose(got, want, rtol=3e-6, atol=1e-6)
    assert rel_l2(got, want) <= 1e-6


@pytest.mark.parametrize("rows,hidden", [(1, 4), (48, 128), (3, 1000), (7, 5120)])
def test_l2_normalize(dev, ora, rows, hidden):
    rng = np.random.default_rng(rows + hidden)
    x = (rng.standard_normal((rows, hidden)) * rng.uniform(0.01, 50, (rows, 1))).astype(np.float32)
    x[0, :] = 0.0 if rows > 2 else x[0, :]  # an all-zero row stays zero
    out = DeviceBuffer.empty((rows, hidden), np.float32)
    ops.l2_normalize(up(x), out, rows, hidden, 1e-6)
    got = out.download()
    want = ora.l2_normalize(x, 1e-6)
    assert rel_l2(got, want) <= 1e-6
    if rows > 2:
        assert np.array_equal(got[0], np.zeros(hidden, np.float32))


def test_l2_normalize_reference_fixture(dev, ora):
    v = np.array([[0.5, -0.25, 0.125, 0.75]], np.float32)  # ssm_l2_normalize.json
    out = DeviceBuffer.empty((1, 4), np.float32)
    ops.l2_normalize(up(v), out, 1, 4, 1e-6)
    np.testing.assert_allclose(out.download(), ora.l2_normalize(v, 1e-6), rtol=1e-6)


@pytest.mark.parametrize("tokens,channels,ks,bias", [(1, 4, 1, True), (128, 10240, 4, True), (1, 10240, 4, False),
                                                     (37, 300, 7, True)])
def test_conv1d_depthwise_bit_exact(dev, ora, tokens, channels, ks, bias):
    rng = np.random.default_rng(tokens + channels + ks)
    x = rng.standard_normal((tokens, channels)).astype(np.float32)
    w = rng.standard_normal((channels, ks)).astype(np.float32)
    b = rng.standard_normal(channels).astype(np.float32) if bias else None
    out = DeviceBuffer.empty((tokens, channels), np.float32)
    ops.conv1d_depthwise(up(x), up(w), up(b) if bias else None, out, tokens, channels, ks)
    assert np.array_equal(out.download(), ora.conv1d_depthwise(x, w, b))


def test_conv1d_reference_fixture(dev):
    # ssm_conv1d_depthwise.json: one token, 4 channels, kernel_size 1
    x = np.array([[0.5, -0.25, 0.125, 0.75]], np.float32)
    w = np.array([[0.25], [-0.125], [0.5], [-0.25]], np.float32)
    b = np.array([0.0, 0.125, -0.125, 0.25], np.float32)
    out = DeviceBuffer.empty((1, 4), np.float32)
    ops.conv1d_depthwise(up(x), up(w), up(b), out, 1, 4, 1)
    assert np.array_equal(out.download()[0], x[0] * w[:, 0] + b)


@pytest.mark.parametrize("tokens,heads,kd,vd,per_head", [(1, 48, 128, 128, False), (16, 4, 128, 128, True),
                                                         (3, 2, 5, 7, True), (9, 3, 200, 33, False),
                                                         (1, 1, 64, 16, False)])
def test_linear_attention(dev, ora, tokens, heads, kd, vd, per_head):
    rng = np.random.default_rng(tokens * 7 + heads + kd + vd)
    q = rng.standard_normal((tokens, heads, vd)).astype(np.float32)
    # unit keys (the graph l2-normalises q and k before this step)
    k = rng.standard_normal((tokens, heads, kd)).astype(np.float32)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((tokens, heads, kd)).astype(np.float32)
    g = rng.standard_normal((tokens, heads, vd)).astype(np.float32)
    S0 = (0.1 * rng.standard_normal((heads, vd, kd))).astype(np.float32)
    a_log = rng.uniform(0.1, 2.0, heads).astype(np.float32) if per_head else None
    dS, out = up(S0), DeviceBuffer.empty((tokens, heads, vd), np.float32)
    ops.linear_attention(up(q), up(k), up(v), up(g), dS, out, tokens, heads, kd, vd,
                         a_log=up(a_log) if per_head else None)
    S_want, o_want = ora.linear_attention(q, k, v, g, S0, a_log)
    assert rel_l2(dS.download(), S_want) <= 1e-5
    assert rel_l2(out.download(), o_want) <= 1e-5


def test_linear_attention_tokens_equal_steps(dev):
    # a 6-token call equals six 1-token calls on the same state
    rng = np.random.default_rng(5)
    T, H, Kd, Vd = 6, 2, 128, 128
    q, g = (rng.standard_normal((T, H, Vd)).astype(np.float32) for _ in range(2))
    k, v = (rng.standard_normal((T, H, Kd)).astype(np.float32) * 0.1 for _ in range(2))
    S0 = rng.standard_normal((H, Vd, Kd)).astype(np.float32) * 0.1
    dS, out = up(S0), DeviceBuffer.empty((T, H, Vd), np.float32)
    ops.linear_attention(up(q), up(k), up(v), up(g), dS, out, T, H, Kd, Vd)
    dS1, outs = up(S0), []
    for t in range(T):
        o1 = DeviceBuffer.empty((1, H, Vd), np.float32)
        ops.linear_attention(up(q[t:t + 1]), up(k[t:t + 1]), up(v[t:t + 1]), up(g[t:t + 1]), dS1, o1, 1, H, Kd, Vd)
        outs.append(o1.download()[0])
    assert np.array_equal(dS.download(), dS1.download())
    assert np.array_equal(out.download(), np.stack(outs))


def test_ssm_argument_checks(dev):
    a = DeviceBuffer.empty((16,), np.float32)
    with pytest.raises(DoeError):
        ops._lib.call("doe_gated", a.ptr, a.ptr, a.ptr, 16, 3, None)
    with pytest.raises(ValueError):
        ops.gated(a, a, a, 16, "relu")
    with pytest.raises(DoeError):  # key_dim > 256
        big = DeviceBuffer.empty((300 * 300,), np.float32)
        ops.linear_attention(big, big, big, big, big, big, 1, 1, 300, 1)
