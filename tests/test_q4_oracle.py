"""Pins the 4-bit GEMV oracle (oracle/q4_oracle.c, a restatement of
kernels/matmul_nbits_sg.wgsl:81-137) against checks that do not share its
code: a float64 numpy dequantise-and-multiply, one-hot activations, zero
points equal to the nibbles, and the relu2 epilogue. CPU only."""
import numpy as np
import pytest

import oracle
from q4_cases import (HIDDEN, dequant_f32, gemv_f64, nibbles, random_q4, rng, zero_points)

# float32 accumulation of K products: |y - y64| <= TOL * sum_k |w_k a_k|.
TOL = 1e-6


@pytest.mark.parametrize("n,n_blocks", [(1, 1), (7, 5), (64, 98), (12, 300), (130, 160)])
def test_matches_float64(n, n_blocks):
    g = rng(100 + n + n_blocks)
    quant, scales, zp = random_q4(g, n, n_blocks)
    a = g.standard_normal(32 * n_blocks).astype(np.float32)
    y = oracle.q4_gemv_f32(a, quant, scales, zp)
    y64, bound = gemv_f64(a, quant, scales, zp)
    assert np.all(np.abs(y - y64) <= TOL * bound)


def test_one_hot_activations_fix_the_layout():
    """With a = e_i the output is exactly (nib - zp) * scale of element i of
    every column: this fixes the nibble order inside a byte, the byte order
    inside a block, the block index and the zero-point index."""
    g = rng(7)
    n, n_blocks = 9, 6
    quant, scales, zp = random_q4(g, n, n_blocks)
    w32 = dequant_f32(quant, scales, zp)
    for i in [0, 1, 2, 7, 8, 31, 32, 33, 95, 191]:
        a = np.zeros(32 * n_blocks, np.float32)
        a[i] = 1.0
        y = oracle.q4_gemv_f32(a, quant, scales, zp)
        np.testing.assert_array_equal(y, w32[:, i])


def test_dequant_matches_numpy():
    g = rng(8)
    quant, scales, zp = random_q4(g, 33, 7)
    np.testing.assert_array_equal(oracle.q4_dequant(quant, scales, zp), dequant_f32(quant, scales, zp))


def test_zero_points_equal_to_nibbles_give_zero():
    g = rng(9)
    n, n_blocks = 11, 4
    _, scales, zp = random_q4(g, n, n_blocks)
    z = zero_points(zp, n, n_blocks)
    byte = (z | (z << 4)).astype(np.uint8)  # both nibbles of every byte = zp
    quant = np.repeat(byte[..., None], 16, axis=2)
    a = g.standard_normal(32 * n_blocks).astype(np.float32)
    assert np.all(oracle.q4_gemv_f32(a, quant, scales, zp) == 0.0)


def test_relu2_epilogue():
    g = rng(10)
    quant, scales, zp = random_q4(g, 23, 9)
    a = g.standard_normal(32 * 9).astype(np.float32)
    y = oracle.q4_gemv_f32(a, quant, scales, zp)
    r = np.maximum(y, np.float32(0))
    np.testing.assert_array_equal(oracle.q4_gemv_f32(a, quant, scales, zp, epilogue=1), r * r)


def test_threads_bitwise_equal():
    g = rng(11)
    quant, scales, zp = random_q4(g, 257, 98)
    a = g.standard_normal(HIDDEN).astype(np.float32)
    np.testing.assert_array_equal(oracle.q4_gemv_f32(a, quant, scales, zp),
                                  oracle.q4_gemv_f32(a, quant, scales, zp, threads=4))


def test_rejects_bad_k():
    g = rng(12)
    quant, scales, zp = random_q4(g, 4, 3)
    with pytest.raises(AssertionError):
        oracle.q4_gemv_f32(np.zeros(95, np.float32), quant, scales, zp)


@pytest.mark.parametrize("mistake", ["nibbles_swapped", "zp_per_column", "zp_hi_first", "scale_of_next_block"])
def test_checks_catch_planted_mistakes(mistake):
    """Plants a plausible decoding mistake in a numpy copy and shows the
    float64 comparison above rejects it — so agreement is evidence."""
    g = rng(13)
    n, n_blocks = 40, 98
    quant, scales, zp = random_q4(g, n, n_blocks)
    a = g.standard_normal(32 * n_blocks).astype(np.float32)
    nib = nibbles(quant).astype(np.float64)
    z = zero_points(zp, n, n_blocks).astype(np.float64)
    s = scales.astype(np.float64)
    if mistake == "nibbles_swapped":
        nib = nib.reshape(n, n_blocks, 16, 2)[..., ::-1].reshape(n, n_blocks, 32)
    if mistake == "zp_per_column":
        z = np.repeat(z[:, :1], n_blocks, axis=1)
    if mistake == "zp_hi_first":
        idx = np.arange(n * n_blocks)
        byte = zp[idx // 2]
        z = np.where(idx % 2 == 0, byte >> 4, byte & 15).reshape(n, n_blocks).astype(np.float64)
    if mistake == "scale_of_next_block":
        s = np.roll(s, -1, axis=1)
    wrong = ((nib - z[..., None]) * s[..., None]).reshape(n, -1) @ a.astype(np.float64)
    _, bound = gemv_f64(a, quant, scales, zp)
    y = oracle.q4_gemv_f32(a, quant, scales, zp)
    assert np.any(np.abs(y - wrong) > TOL * bound)
