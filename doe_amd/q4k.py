"""Q4_K_M block packing and seeded synthetic weights (host side, numpy).

Block layout (bench/tools/doppler_rdrr_q4k.py:11-15): 256 weights in 144
bytes -- [0:2] f16 d, [2:4] f16 dmin, [4:16] packed 6-bit scales/mins,
[16:144] nibbles.  The packer is the inverse of the reference's
``unpack_q4k_scale_min_bits`` and nibble order, as written out by its own test
packer (bench/tests/test_doppler_rdrr_q4k.py:22-57), vectorised over blocks.
"""
from __future__ import annotations

import numpy as np

BLOCK_BYTES = 144
BLOCK_ELEMS = 256
SUBBLOCKS = 8


def blocks_per_row(k: int) -> int:
    return (int(k) + BLOCK_ELEMS - 1) // BLOCK_ELEMS


def row_bytes(k: int) -> int:
    return blocks_per_row(k) * BLOCK_BYTES


def pack_blocks(d: np.ndarray, dmin: np.ndarray, scales: np.ndarray, mins: np.ndarray,
                quants: np.ndarray) -> np.ndarray:
    """Packs ``B`` blocks into a uint8 array of shape ``[B, 144]``.

    d, dmin: float16 [B]; scales, mins: ints in 0..63 [B, 8]; quants: ints in
    0..15 [B, 256] (element order of the dequantized block).
    """
    d = np.asarray(d, dtype=np.float16).reshape(-1)
    dmin = np.asarray(dmin, dtype=np.float16).reshape(-1)
    nblk = d.shape[0]
    sc = np.asarray(scales, dtype=np.uint8).reshape(nblk, SUBBLOCKS)
    mn = np.asarray(mins, dtype=np.uint8).reshape(nblk, SUBBLOCKS)
    q = np.asarray(quants, dtype=np.uint8).reshape(nblk, BLOCK_ELEMS)
    if np.any(sc > 63) or np.any(mn > 63) or np.any(q > 15):
        raise ValueError("scales/mins must be < 64 and quants < 16")
    out = np.zeros((nblk, BLOCK_BYTES), dtype=np.uint8)
    out[:, 0:2] = d.view(np.uint8).reshape(nblk, 2)
    out[:, 2:4] = dmin.view(np.uint8).reshape(nblk, 2)
    # bytes 4..7 / 8..11: low 6 bits of sub-blocks 0..3, top 2 bits of 4..7
    out[:, 4:8] = (sc[:, 0:4] & 0x3F) | (((sc[:, 4:8] >> 4) & 0x03) << 6)
    out[:, 8:12] = (mn[:, 0:4] & 0x3F) | (((mn[:, 4:8] >> 4) & 0x03) << 6)
    # bytes 12..15: low nibbles of sub-blocks 4..7 (scale low, min high)
    out[:, 12:16] = (sc[:, 4:8] & 0x0F) | ((mn[:, 4:8] & 0x0F) << 4)
    # nibbles: byte 16 + 32c + i = q[64c + i] | q[64c + 32 + i] << 4
    qc = q.reshape(nblk, 4, 2, 32)
    out[:, 16:] = (qc[:, :, 0, :] | (qc[:, :, 1, :] << 4)).reshape(nblk, 128)
    return out


def random_q4k(rng: np.random.Generator, n: int, k: int, d_sigma: float = 0.02,
               dmin_sigma: float = 0.01) -> np.ndarray:
    """Seeded random Q4_K_M weight matrix ``[n][row_bytes(k)]`` (uint8).

    Generation order: d = f16(|N(0, d_sigma)|), dmin = f16(|N(0, dmin_sigma)|),
    scales, mins = integers(0, 64, [B, 8]), quants = integers(0, 16, [B, 256]).
    """
    nb = blocks_per_row(k)
    nblk = n * nb
    d = np.abs(rng.normal(0.0, d_sigma, nblk)).astype(np.float16)
    dmin = np.abs(rng.normal(0.0, dmin_sigma, nblk)).astype(np.float16)
    sc = rng.integers(0, 64, (nblk, SUBBLOCKS), dtype=np.uint8)
    mn = rng.integers(0, 64, (nblk, SUBBLOCKS), dtype=np.uint8)
    q = rng.integers(0, 16, (nblk, BLOCK_ELEMS), dtype=np.uint8)
    return pack_blocks(d, dmin, sc, mn, q).reshape(n, nb * BLOCK_BYTES)


def unpack_scale_min(blocks: np.ndarray):
    """Vectorised scale/min decode of ``[B, 144]`` blocks -> (sc, mn, d, dmin)."""
    b = np.asarray(blocks, dtype=np.uint8).reshape(-1, BLOCK_BYTES)
    d = b[:, 0:2].copy().view(np.float16).reshape(-1).astype(np.float32)
    dmin = b[:, 2:4].copy().view(np.float16).reshape(-1).astype(np.float32)
    sc = np.empty((b.shape[0], 8), np.uint8)
    mn = np.empty((b.shape[0], 8), np.uint8)
    sc[:, 0:4] = b[:, 4:8] & 0x3F
    mn[:, 0:4] = b[:, 8:12] & 0x3F
    sc[:, 4:8] = (b[:, 12:16] & 0x0F) | ((b[:, 4:8] >> 6) << 4)
    mn[:, 4:8] = (b[:, 12:16] >> 4) | ((b[:, 8:12] >> 6) << 4)
    return sc, mn, d, dmin
