"""Host-side logic: Q4_K packer and the operator interface's argument checks
(CPU only; nothing reaches the GPU)."""
import numpy as np
import pytest

from doe_amd import ops, q4k


class FakeBuf:
    def __init__(self, nbytes):
        self.nbytes = nbytes
        self.ptr = 0


def test_row_bytes():
    assert q4k.row_bytes(2304) == 9 * 144
    assert q4k.row_bytes(300) == 2 * 144
    assert q4k.blocks_per_row(256) == 1


def test_random_q4k_is_seeded_and_shaped():
    a = q4k.random_q4k(np.random.default_rng(0), 3, 512)
    b = q4k.random_q4k(np.random.default_rng(0), 3, 512)
    assert a.shape == (3, 2 * 144) and a.dtype == np.uint8
    assert np.array_equal(a, b)
    sc, mn, d, dmin = q4k.unpack_scale_min(a)
    assert sc.max() <= 63 and mn.max() <= 63 and (d >= 0).all() and (dmin >= 0).all()


def test_pack_rejects_out_of_range():
    with pytest.raises(ValueError):
        q4k.pack_blocks(np.ones(1), np.ones(1), np.full((1, 8), 64), np.zeros((1, 8)), np.zeros((1, 256)))


def test_matmul_q4k_rejects_wrong_weight_length():
    with pytest.raises(ValueError, match="Q4_K_M rowwise byte length"):
        ops.matmul_q4k(FakeBuf(144 * 9 * 10 - 1), FakeBuf(2304 * 4), FakeBuf(40), 10, 2304)
    with pytest.raises(ValueError, match="activation"):
        ops.matmul_q4k(FakeBuf(144 * 9 * 10), FakeBuf(2303 * 4), FakeBuf(40), 10, 2304)
    with pytest.raises(ValueError, match="output"):
        ops.matmul_q4k(FakeBuf(144 * 9 * 10), FakeBuf(2304 * 4), FakeBuf(36), 10, 2304)


def test_bench_refuses_more_than_one_gpu():
    # bench.py measures one GPU: --gpus above 1 exits with status 2 and a
    # message, before anything touches a device
    import subprocess
    import sys

    from conftest import ROOT

    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd="/tmp")
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""
