"""Q8_0 on the CPU: the oracle (oracle/doe_oracle.c ora_q8_0_*) pinned against
the reference's own Q8_0 size checks (runtime/zig/src/doe_wgsl/csl_spec.zig:
231-236 test "Q8_0 validation accepts valid sizes" and q8_0ElementCount
:150-153), hand-decoded known answers for the byte layout (:121-125: f16
scale, then 32 int8 quants), and a bit-exact cross-check with the int4
group-32 oracle (pinned to the reference's golden vectors): a Q8_0 block whose
quants lie in -8..7 encodes the same weights as an int4 group.  Plus the host
packer and the RDRR Q8_0 reader."""
import json

import numpy as np
import pytest

from doe_amd import q8_0, rdrr


def test_reference_size_checks(ora):
    # csl_spec.zig:231-236 and q8_0ElementCount
    assert ora.q8_0_element_count(34) == 32
    assert ora.q8_0_element_count(34 * 5) == 160
    assert ora.q8_0_element_count(0) is None
    assert ora.q8_0_element_count(33) is None
    assert ora.q8_0_element_count(35) is None


def test_known_block_bytes(ora):
    # d = 1.0 (f16 0x3c00, little-endian), quants 0, 1, ..., 15, -1, -2, ..., -16
    quants = list(range(16)) + [-(i + 1) for i in range(16)]
    blk = bytes([0x00, 0x3C]) + bytes(q & 0xFF for q in quants)
    # second block: d = -0.5 (0xb800), quants -128 and 127 then zeros
    blk2 = bytes([0x00, 0xB8, 0x80, 0x7F]) + bytes(30)
    w = np.frombuffer(blk + blk2, np.uint8).reshape(1, 68)
    vals = ora.q8_0_dequant(w, 1, 64)[0]
    assert np.array_equal(vals[:32], np.array(quants, np.float32))
    assert vals[32] == 64.0 and vals[33] == -63.5 and not vals[34:].any()
    x = np.zeros(64, np.float32)
    x[5], x[20], x[33] = 2.0, 0.25, 4.0  # 5*2 + (-5)*0.25 + (-63.5)*4
    assert ora.q8_0_gemv(w, x, 1, 64)[0] == 10.0 - 1.25 - 254.0
    # the host packer writes the same bytes
    assert q8_0.pack_rows([[1.0, -0.5]], [[quants, [-128, 127] + [0] * 30]]).tobytes() == blk + blk2


def test_matches_int4_group32_oracle(ora):
    rng = np.random.default_rng(3)
    n, k = 7, 256
    qv = rng.integers(-8, 8, (n, k))
    sc = (rng.standard_normal((n, k // 32)) * 0.05).astype(np.float16)
    x = rng.standard_normal(k, dtype=np.float32)
    nib = (qv + 8).astype(np.uint32).reshape(-1, 8)
    words = np.zeros(nib.shape[0], np.uint32)
    for j in range(8):
        words |= nib[:, j] << np.uint32(4 * j)
    want = ora.int4g32_gemv(words, sc, x, 1, n, k)[0]
    w = q8_0.pack_rows(sc, qv.reshape(n, k // 32, 32))
    got = ora.q8_0_gemv(w, x, n, k)
    assert np.array_equal(got, want)  # same weights, same f32 fold: bit-exact


def test_tail_block_residual_and_brute_force(ora):
    rng = np.random.default_rng(4)
    n, k = 5, 70  # three blocks per row, 26 padding quants
    w = q8_0.random_q8_0(rng, n, k)
    x = rng.standard_normal(k, dtype=np.float32)
    r = rng.standard_normal(n, dtype=np.float32)
    blocks = w.reshape(n, 3, 34)
    d = blocks[:, :, :2].copy().view("<f2")[..., 0].astype(np.float64)
    q = blocks[:, :, 2:].view(np.int8).astype(np.float64)
    dense = (q * d[..., None]).reshape(n, 96)[:, :k]
    want = dense @ x.astype(np.float64) + r
    got = ora.q8_0_gemv(w, x, n, k, residual=r)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5)
    assert not blocks.reshape(n, -1)[:, 34 * 2 + 2 + 6:].any()  # padding quants are zero
    with pytest.raises(ValueError):
        ora.q8_0_gemv(w[:, :-1], x, n, k)


def test_pack_rejects_bad_input():
    with pytest.raises(ValueError):
        q8_0.pack_rows(np.ones((2, 1)), np.zeros((2, 1, 31)))
    with pytest.raises(ValueError):
        q8_0.pack_rows(np.ones((1, 1)), np.full((1, 1, 32), 128))
    assert q8_0.row_bytes(1) == 34 and q8_0.row_bytes(32) == 34 and q8_0.row_bytes(33) == 68


def test_rdrr_q8_0_rows(tmp_path):
    rng = np.random.default_rng(5)
    w = q8_0.random_q8_0(rng, 3, 100)  # 4 blocks per row
    raw = w.tobytes()
    (tmp_path / "shard_00000.bin").write_bytes(raw)
    base = {"shard": 0, "offset": 0, "size": len(raw), "shape": [3, 100], "dtype": "Q8_0"}
    man = {"shards": [{"index": 0, "size": len(raw)}], "tensors": {
        "ok": base, "row": {**base, "layout": "row"}, "col": {**base, "layout": "col"},
        "short": {**base, "shape": [4, 100]}, "ragged": {**base, "size": len(raw) - 2},
        "q4": {**base, "dtype": "Q4_K_M"}}}
    (tmp_path / "manifest.json").write_text(json.dumps(man))
    art = rdrr.RdrrArtifact(tmp_path)
    assert np.array_equal(art.q8_0_rows("ok"), w) and np.array_equal(art.q8_0_rows("row"), w)
    for name, msg in (("col", "layout"), ("short", "Q8_0 matrix has"), ("ragged", "whole number"),
                      ("q4", "not Q8_0")):
        with pytest.raises(rdrr.RdrrError, match=msg):
            art.q8_0_rows(name)
