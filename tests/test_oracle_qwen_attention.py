"""The oracle's Qwen 3.6 attention composition against real activations of
the reference's frozen Doppler run (tests/golden/qwen36_layer3_attention.npz,
cut by tests/golden/make_qwen36_attention_fixture.py from
bench/fixtures/r3-2-27b-doppler-frozen-af16/layer_3): q and k after their
RMSNorms, rotated over the first 64 of 256 dims (partialRotaryFactor 0.25,
ropeTheta 1e7, qwen-3-6-27b-smoke.json:22-30), then causal attention of six
query heads on their KV head at scale 1/16, gives the run's attention output
before the output gate.  Doppler computes in f16 (the graph's activation
dtype): the oracle, in f32 on the same inputs, sits 2.1e-3 from it; rotating
all 256 dims, or interleaved pairs, misses by 7e-2 or more."""
import numpy as np
import pytest

from conftest import ROOT

T, G, D, ROT, THETA = 18, 6, 256, 64, 1e7


@pytest.fixture(scope="module")
def fx():
    with np.load(ROOT / "tests" / "golden" / "qwen36_layer3_attention.npz", allow_pickle=False) as z:
        return {k: z[k].astype(np.float32) for k in z.files}


def oracle_attention(ora, fx, rot):
    tab = ora.rope_table(T, rot, THETA)
    q = ora.rope_partial(fx["q"], tab, T, G, D, rot, 0).reshape(T, G, D)
    k = ora.rope_partial(fx["k"], tab, T, 1, D, rot, 0).reshape(T, 1, D)
    kc = np.zeros((1, T, D), np.float16)
    vc = np.zeros((1, T, D), np.float16)
    out = np.zeros((T, G, D), np.float32)
    for t in range(T):
        ora.kv_write(k[t], fx["v"][t], kc, vc, 1, T, D, t)
        out[t] = ora.attn_decode(q[t], kc, vc, G, 1, D, t + 1, T, 1.0 / 16)
    return out


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def test_oracle_matches_the_reference_run(ora, fx):
    assert rel(oracle_attention(ora, fx, ROT), fx["out"]) <= 3e-3


def test_full_rotation_misses(ora, fx):
    # the same check rejects a full-width rotation
    assert rel(oracle_attention(ora, fx, D), fx["out"]) > 5e-2


def test_rope_partial_leaves_the_other_dims(ora):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 3, 16)).astype(np.float32)
    tab = ora.rope_table(4, 8, 1e4)
    y = ora.rope_partial(x, tab, 2, 3, 16, 8, 1).reshape(2, 3, 16)
    assert np.array_equal(y[..., 8:], x[..., 8:])
    # the rotated part is ora_rope at head_dim 8
    want = ora.rope(np.ascontiguousarray(x[..., :8]), tab, 2, 3, 8, 1).reshape(2, 3, 8)
    assert np.array_equal(y[..., :8], want)
