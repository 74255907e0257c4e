"""Q8_0 block packing and seeded synthetic weights (host side, numpy).

Block layout (runtime/zig/src/doe_wgsl/csl_spec.zig:121-125): 32 weights in
34 bytes -- [0:2] f16 scale d (little-endian), [2:34] int8 quants q; weight =
d * q.  Row-wise matrices hold ceil(k / 32) blocks per row, the tail block
zero padded, which is the layout doe_q8_0_gemv reads.
"""
from __future__ import annotations

import numpy as np

BLOCK_BYTES = 34
BLOCK_ELEMS = 32
_BLOCK = np.dtype([("d", "<f2"), ("q", "i1", (BLOCK_ELEMS,))])
assert _BLOCK.itemsize == BLOCK_BYTES


def blocks_per_row(k: int) -> int:
    return (int(k) + BLOCK_ELEMS - 1) // BLOCK_ELEMS


def row_bytes(k: int) -> int:
    return blocks_per_row(k) * BLOCK_BYTES


def pack_rows(d: np.ndarray, q: np.ndarray) -> np.ndarray:
    """Row-wise Q8_0 bytes ``[n][row_bytes]`` from scales d ``[n][nb]`` (cast
    to f16) and quants q ``[n][nb][32]`` (ints in -128..127)."""
    d = np.asarray(d, np.float16)
    q = np.asarray(q)
    if q.ndim != 3 or q.shape[2] != BLOCK_ELEMS or d.shape != q.shape[:2]:
        raise ValueError("d must be [n][nb] and q [n][nb][32]")
    if q.size and (q.min() < -128 or q.max() > 127):
        raise ValueError("quants must be in -128..127")
    blocks = np.empty(d.shape, _BLOCK)
    blocks["d"], blocks["q"] = d, q.astype(np.int8)
    return blocks.view(np.uint8).reshape(d.shape[0], -1)


def random_q8_0(rng: np.random.Generator, n: int, k: int, d_sigma: float = 0.01) -> np.ndarray:
    """Seeded random row-wise Q8_0 matrix ``[n][row_bytes(k)]`` (uint8); the
    tail block's quants past k are zero, as a quantiser writes them."""
    nb = blocks_per_row(k)
    d = np.abs(rng.standard_normal((n, nb)) * d_sigma) + d_sigma / 8
    q = rng.integers(-128, 128, (n, nb, BLOCK_ELEMS))
    q.reshape(n, nb * BLOCK_ELEMS)[:, k:] = 0
    return pack_rows(d, q)
