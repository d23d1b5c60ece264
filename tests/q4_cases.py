"""Seeded 4-bit weights in the reference's format and an independent float64
decode of them.

Format (engine/weights.js:99-104, engine/weight-index.json, read by
kernels/matmul_nbits_sg.wgsl): for a [K -> N] projection with n_blocks =
K / 32, quant is uint8 [N][n_blocks][16] (element 2j of a block in the low
nibble of byte j, element 2j+1 in the high nibble), scales float32
[N][n_blocks], zp the 4-bit zero points packed two per byte in order of the
flat index col * n_blocks + blk, low nibble first.

Shapes of the attention layer of the Nano-4B model (engine/config.js:2-26):
q/k/v projections K = hidden = 3136 (98 blocks) to N = 5120 / 1024 / 1024;
o_proj K = 5120 (160 blocks) to N = 3136.
"""
from __future__ import annotations

import numpy as np

HIDDEN = 3136
Q_COLS, KV_COLS = 5120, 1024


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def random_q4(g: np.random.Generator, n: int, n_blocks: int, scale: float = 0.02):
    """Random quant bytes, positive scales around `scale`, random zero points."""
    quant = g.integers(0, 256, size=(n, n_blocks, 16), dtype=np.uint8)
    scales = (g.uniform(0.5, 1.5, size=(n, n_blocks)) * scale).astype(np.float32)
    zp = g.integers(0, 256, size=(n * n_blocks + 1) // 2, dtype=np.uint8)
    return quant, scales, zp


def nibbles(quant: np.ndarray) -> np.ndarray:
    """[N][n_blocks][16] bytes -> [N][n_blocks][32] nibbles in element order."""
    out = np.empty(quant.shape[:-1] + (32,), np.uint8)
    out[..., 0::2] = quant & 15
    out[..., 1::2] = quant >> 4
    return out


def zero_points(zp: np.ndarray, n: int, n_blocks: int) -> np.ndarray:
    """Packed zero points -> [N][n_blocks] values."""
    idx = np.arange(n * n_blocks)
    byte = zp[idx // 2]
    return np.where(idx % 2 == 0, byte & 15, byte >> 4).reshape(n, n_blocks).astype(np.uint8)


def dequant_f64(quant, scales, zp) -> np.ndarray:
    n, n_blocks = scales.shape
    w = (nibbles(quant).astype(np.float64) - zero_points(zp, n, n_blocks)[..., None]) \
        * scales.astype(np.float64)[..., None]
    return w.reshape(n, n_blocks * 32)


def dequant_f32(quant, scales, zp) -> np.ndarray:
    """(nib - zp) * scale rounded once in float32, as the WGSL forms it."""
    n, n_blocks = scales.shape
    w = (nibbles(quant).astype(np.float32) - zero_points(zp, n, n_blocks)[..., None].astype(np.float32)) \
        * scales[..., None]
    return w.reshape(n, n_blocks * 32)


def gemv_f64(a, quant, scales, zp, rows: int = 4096):
    """Y = dequant(W) . a in float64, and the bound sum_k |w_k a_k| that the
    float32 tolerances are stated against (computed `rows` columns at a
    time, so a 131072-column lm_head fits in memory)."""
    n, n_blocks = scales.shape
    a64 = np.asarray(a, np.float64).reshape(-1)
    z = zero_points(zp, n, n_blocks)
    y, bound = np.empty(n), np.empty(n)
    for r0 in range(0, n, rows):
        r1 = min(n, r0 + rows)
        w = ((nibbles(quant[r0:r1]).astype(np.float64) - z[r0:r1, :, None])
             * scales[r0:r1].astype(np.float64)[..., None]).reshape(r1 - r0, -1)
        y[r0:r1] = w @ a64
        bound[r0:r1] = np.abs(w) @ np.abs(a64)
    return y, bound
