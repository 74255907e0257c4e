"""GPU parity of causal GQA prefill attention (bf16 q/K/V, head_dim 128)
against the CPU oracle's two-pass f32 softmax (bf16 inputs upcast exactly),
through the C ABI.  Contract: rel-L2 <= 1e-3."""
import ctypes as C
import math

import numpy as np
import pytest

from doe_amd import DeviceBuffer, Graph, Stream, _lib, ops

pytestmark = pytest.mark.gpu

TOL = 1e-3
D = 128


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def to_bf16(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def up(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


def run(q, k, v, hq, hkv, q_len, kv_len, kv_stride, start_pos, scale, causal, out_bf16=False):
    out = DeviceBuffer.empty((q_len, hq, D), np.uint16 if out_bf16 else np.float32)
    ops.attention_prefill(up(q), up(k), up(v), out, num_heads=hq, num_kv_heads=hkv, head_dim=D, q_len=q_len,
                          kv_len=kv_len, kv_stride=kv_stride, start_pos=start_pos, scale=scale, causal=causal,
                          out_bf16=out_bf16)
    got = out.download()
    return bf16_to_f32(got) if out_bf16 else got


def oracle(ora, q, k, v, hq, hkv, q_len, kv_len, kv_stride, start_pos, scale, causal, rows=None):
    kf = bf16_to_f32(k).reshape(hkv, kv_stride, D)[:, :kv_len]
    vf = bf16_to_f32(v).reshape(hkv, kv_stride, D)[:, :kv_len]
    return ora.attn_prefill(bf16_to_f32(q), kf, vf, hq, hkv, D, q_len, kv_len, start_pos, scale, causal, rows)


@pytest.mark.parametrize("hq,hkv,s", [(4, 2, 200), (2, 2, 64), (8, 1, 129), (4, 4, 1)])
def test_prefill_causal_matches_oracle(dev, ora, hq, hkv, s):
    rng = np.random.default_rng(hq * 100 + s)
    q = to_bf16(rng.standard_normal((s, hq, D), dtype=np.float32))
    k = to_bf16(rng.standard_normal((hkv, s, D), dtype=np.float32))
    v = to_bf16(rng.standard_normal((hkv, s, D), dtype=np.float32))
    scale = 1.0 / math.sqrt(D)
    got = run(q, k, v, hq, hkv, s, s, s, 0, scale, True)
    want = oracle(ora, q, k, v, hq, hkv, s, s, s, 0, scale, True)
    err = rel_l2(got, want)
    print(f"[prefill {hq}/{hkv} S={s}] rel_l2 {err:.2e}", flush=True)
    assert err <= TOL
    # query 0 sees only key 0: its output is v[kvh][0] exactly up to f16 rounding of V
    for h in range(hq):
        np.testing.assert_allclose(got[0, h], bf16_to_f32(v[h // (hq // hkv), 0]), rtol=1e-3, atol=1e-3)


def test_prefill_chunked_and_noncausal(dev, ora):
    # a later prompt chunk (start_pos 200) against a 300-key cache with a
    # longer row stride, causal and non-causal, f32 and bf16 output
    rng = np.random.default_rng(7)
    hq, hkv, q_len, kv_len, stride, start = 8, 2, 100, 300, 512, 200
    q = to_bf16(rng.standard_normal((q_len, hq, D), dtype=np.float32) * 2)
    k = to_bf16(rng.standard_normal((hkv, stride, D), dtype=np.float32))
    v = to_bf16(rng.standard_normal((hkv, stride, D), dtype=np.float32))
    scale = 0.1
    for causal in (True, False):
        want = oracle(ora, q, k, v, hq, hkv, q_len, kv_len, stride, start, scale, causal)
        got = run(q, k, v, hq, hkv, q_len, kv_len, stride, start, scale, causal)
        assert rel_l2(got, want) <= TOL, causal
        got16 = run(q, k, v, hq, hkv, q_len, kv_len, stride, start, scale, causal, out_bf16=True)
        assert rel_l2(got16, want) <= 5e-3, causal  # bf16 output rounding (2^-9)


def test_prefill_config_rows(dev, ora):
    # the 31B-class prefill attention: 32 query / 16 KV heads, head_dim 128,
    # 2048 tokens, causal; oracle on the first, a middle and the last rows
    rng = np.random.default_rng(8)
    hq, hkv, s = 32, 16, 2048
    q = to_bf16(rng.standard_normal((s, hq, D), dtype=np.float32))
    k = to_bf16(rng.standard_normal((hkv, s, D), dtype=np.float32))
    v = to_bf16(rng.standard_normal((hkv, s, D), dtype=np.float32))
    scale = 1.0 / math.sqrt(D)
    got = run(q, k, v, hq, hkv, s, s, s, 0, scale, True)
    assert np.isfinite(got).all()
    for r0, r1 in ((0, 24), (1000, 1016), (2032, 2048)):
        want = oracle(ora, q, k, v, hq, hkv, s, s, s, 0, scale, True, rows=(r0, r1))
        err = rel_l2(got[r0:r1], want[r0:r1])
        print(f"[prefill config] rows {r0}:{r1} rel_l2 {err:.2e}", flush=True)
        assert err <= TOL


@pytest.mark.parametrize("hq,hkv,s", [(4, 2, 1000), (2, 1, 640), (3, 3, 1500)])
def test_prefill_long_prompts(dev, ora, hq, hkv, s):
    # longer causal prompts checked per 128-query block (even and odd block
    # counts, a ragged last block)
    rng = np.random.default_rng(s + hq)
    q = to_bf16(rng.standard_normal((s, hq, D), dtype=np.float32))
    k = to_bf16(rng.standard_normal((hkv, s, D), dtype=np.float32))
    v = to_bf16(rng.standard_normal((hkv, s, D), dtype=np.float32))
    scale = 1.0 / math.sqrt(D)
    got = run(q, k, v, hq, hkv, s, s, s, 0, scale, True)
    want = oracle(ora, q, k, v, hq, hkv, s, s, s, 0, scale, True)
    err = rel_l2(got, want)
    print(f"[prefill {hq}/{hkv} S={s}] rel_l2 {err:.2e}", flush=True)
    assert err <= TOL
    for r0 in range(0, s, 128):
        assert rel_l2(got[r0:r0 + 128], want[r0:r0 + 128]) <= TOL, r0


def test_prefill_more_workgroups_than_slots(dev, ora):
    # 64 heads x 16 query blocks = 1024 workgroups, twice what the CUs hold at once
    rng = np.random.default_rng(11)
    hq, hkv, s = 64, 8, 2048
    q = to_bf16(rng.standard_normal((s, hq, D), dtype=np.float32))
    k = to_bf16(rng.standard_normal((hkv, s, D), dtype=np.float32))
    v = to_bf16(rng.standard_normal((hkv, s, D), dtype=np.float32))
    scale = 1.0 / math.sqrt(D)
    got = run(q, k, v, hq, hkv, s, s, s, 0, scale, True)
    assert np.isfinite(got).all()
    for r0, r1 in ((0, 8), (1020, 1030), (1900, 1910), (2040, 2048)):
        want = oracle(ora, q, k, v, hq, hkv, s, s, s, 0, scale, True, rows=(r0, r1))
        assert rel_l2(got[r0:r1], want[r0:r1]) <= TOL, (r0, r1)


def test_prefill_graph_replays(dev):
    # replays of one captured call (the V^T pre-pass and the attention kernel),
    # with eager calls in between, all reproduce the eager result exactly
    rng = np.random.default_rng(12)
    hq, hkv, s = 8, 2, 1024
    q = up(to_bf16(rng.standard_normal((s, hq, D), dtype=np.float32)))
    k = up(to_bf16(rng.standard_normal((hkv, s, D), dtype=np.float32)))
    v = up(to_bf16(rng.standard_normal((hkv, s, D), dtype=np.float32)))
    out = DeviceBuffer.empty((s, hq, D), np.float32)

    def call(stream=None):
        ops.attention_prefill(q, k, v, out, num_heads=hq, num_kv_heads=hkv, head_dim=D, q_len=s, kv_len=s,
                              kv_stride=s, start_pos=0, scale=0.125, causal=True, stream=stream)

    call()
    want = out.download().copy()
    st = Stream()
    g = Graph.capture(st, lambda: call(st))
    for i in range(4):
        out.upload(np.zeros((s, hq, D), np.float32))
        g.launch(st)
        st.synchronize()
        np.testing.assert_array_equal(out.download(), want, err_msg=f"replay {i}")
        call()
    g.destroy()
    st.destroy()


def test_prefill_softmax_invariants(dev):
    # equal keys: every query's output is the mean of the values it sees;
    # large logits (scale 50) stay finite
    rng = np.random.default_rng(9)
    hq, hkv, s = 2, 1, 96
    q = to_bf16(rng.standard_normal((s, hq, D), dtype=np.float32))
    k = to_bf16(np.tile(rng.standard_normal((1, 1, D), dtype=np.float32), (hkv, s, 1)))
    v = to_bf16(rng.standard_normal((hkv, s, D), dtype=np.float32))
    got = run(q, k, v, hq, hkv, s, s, s, 0, 50.0, True)
    vf = bf16_to_f32(v)[0].astype(np.float64)
    want = np.cumsum(vf, axis=0) / np.arange(1, s + 1)[:, None]
    for h in range(hq):
        assert rel_l2(got[:, h], want) <= TOL
    assert np.isfinite(got).all()


def test_prefill_rejects_bad_head_dim(dev):
    buf = DeviceBuffer(1 << 16)
    with pytest.raises(_lib.DoeError):
        _lib.call("doe_attn_prefill", C.c_void_p(buf.ptr), C.c_void_p(buf.ptr), C.c_void_p(buf.ptr),
                  C.c_void_p(buf.ptr), 0, 2, 1, 64, 4, 4, 4, 0, C.c_float(1.0), 1, C.c_void_p(None))
