"""The allocation-free attention entry point (doe_attn_decode_noalloc)
against doe_attn_decode through the C ABI: two calls in a row, the second
smaller, each bit-equal to the allocating entry point (same split choice and
kernels) and within 1e-3 of the oracle; oversized partials are rejected."""
import ctypes as C

import numpy as np
import pytest

from doe_amd import DeviceBuffer, DoeError, Stream, _lib

pytestmark = pytest.mark.gpu


def _call(fn, q, kc, vc, out, b, hq, hkv, d, t, s):
    _lib.call(fn, C.c_void_p(q.ptr), 0, C.c_void_p(kc.ptr), C.c_void_p(vc.ptr), C.c_void_p(out.ptr), 0, b, hq, hkv,
              d, t, None, t, 0, C.c_float(1.0 / np.sqrt(d)), C.c_float(0.0), 0, C.c_void_p(s.handle))


@pytest.mark.parametrize("order", ["large_then_small"])
def test_noalloc_attention_matches_allocating_entry_point(dev, ora, order):
    s = Stream()
    # (batch, q heads, kv heads, head_dim, context): 64 splits, then a smaller
    # call with a different split count over the same scratch
    for b, hq, hkv, d, t in [(2, 8, 4, 256, 4096), (1, 4, 2, 128, 700)]:
        print(f"[noalloc] batch={b} heads={hq}/{hkv} d={d} t={t}", flush=True)
        rng = np.random.default_rng(b * 100 + t)
        q = rng.standard_normal((b, hq, d)).astype(np.float32)
        k = rng.standard_normal((b, hkv, t, d)).astype(np.float16)
        v = rng.standard_normal((b, hkv, t, d)).astype(np.float16)
        dq, dk, dv = DeviceBuffer.from_array(q), DeviceBuffer.from_array(k), DeviceBuffer.from_array(v)
        o_ref = DeviceBuffer.empty((b, hq, d), np.float32)
        o_na = DeviceBuffer.empty((b, hq, d), np.float32)
        _call("doe_attn_decode", dq, dk, dv, o_ref, b, hq, hkv, d, t, s)
        _call("doe_attn_decode_noalloc", dq, dk, dv, o_na, b, hq, hkv, d, t, s)
        s.synchronize()
        got, ref = o_na.download(), o_ref.download()
        assert np.array_equal(got, ref)
        for bi in range(b):
            want = ora.attn_decode(q[bi], k[bi], v[bi], hq, hkv, d, t, t, 1.0 / np.sqrt(d))
            err = float(np.linalg.norm(got[bi] - want) / np.linalg.norm(want))
            assert err <= 1e-3, err
    s.destroy()


def test_noalloc_attention_rejects_oversized_partials(dev):
    # batch 8, 64/8 heads of 256 over 32768 positions: 32 splits of 512 heads
    # need 16 MiB + 128 KiB of partials, over the 16 MiB scratch.  Buffers of
    # the full size, so nothing would read out of bounds if a kernel ran.
    b, hq, hkv, d, t = 8, 64, 8, 256, 32768
    q = DeviceBuffer.empty((b, hq, d), np.float32)
    kc = DeviceBuffer.empty((b, hkv, t, d), np.float16)
    vc = DeviceBuffer.empty((b, hkv, t, d), np.float16)
    out = DeviceBuffer.empty((b, hq, d), np.float32)
    s = Stream()
    with pytest.raises(DoeError, match="allocation-free scratch"):
        _call("doe_attn_decode_noalloc", q, kc, vc, out, b, hq, hkv, d, t, s)
    s.synchronize()
    for x in (q, kc, vc, out):
        x.free()
    s.destroy()
