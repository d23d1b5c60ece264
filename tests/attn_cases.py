"""Seeded inputs for the decode-attention shapes and layout helpers.

The five workloads (all 32 query heads / 8 KV heads / head_dim 128, fp16):
  1. decode, past 152 (L = 153)          — the reference's runnable case
  2. decode, past 4096, per-head K/V scale U[0.5, 2], 64 appended steps
  3. decode, past 32768, 1% outliers at +-8 (split-K + merge)
  4. ragged batch of 64, past lengths U{512..16384}
  5. causal chunked prefill, 512 new tokens onto 8192

Position convention (engine/runtime.js:451-452): the new token is written at
pos = past, and attention reads L = pos + 1 keys.

Layouts: the oracle takes the reference's token-major [L][Hkv][D] f32 view
(kernels/sparse_attn.wgsl:49); the library's cache is head-major
[B][Hkv][max_seq][D] fp16. `to_cache` / `from_cache` convert.
"""
from __future__ import annotations

import numpy as np

D = 128


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def normal_f16(g: np.random.Generator, shape, scale=1.0) -> np.ndarray:
    return (g.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float16)


def kv_rows(g: np.random.Generator, L: int, n_kv: int, head_scale=None, outlier_frac=0.0):
    """K and V token-major [L][n_kv][D] fp16, optionally scaled per KV head
    and with a fraction of entries replaced by +-8."""
    k = g.standard_normal((L, n_kv, D), dtype=np.float32)
    v = g.standard_normal((L, n_kv, D), dtype=np.float32)
    if head_scale is not None:
        s = np.asarray(head_scale, np.float32).reshape(1, n_kv, 1)
        k *= s
        v *= s
    if outlier_frac > 0:
        for a in (k, v):
            hit = g.random(a.shape) < outlier_frac
            sign = np.where(g.random(a.shape) < 0.5, -8.0, 8.0).astype(np.float32)
            a[hit] = sign[hit]
    return k.astype(np.float16), v.astype(np.float16)


def to_cache(rows_per_seq, n_kv: int, cap: int) -> np.ndarray:
    """List of [L_b][n_kv][D] fp16 -> head-major cache [B][n_kv][cap][D]
    (D taken from the rows)."""
    B = len(rows_per_seq)
    c = np.zeros((B, n_kv, cap, rows_per_seq[0].shape[2]), np.float16)
    for b, r in enumerate(rows_per_seq):
        c[b, :, : r.shape[0], :] = np.transpose(r, (1, 0, 2))
    return c


def from_cache(cache: np.ndarray, b: int, L: int) -> np.ndarray:
    """Head-major cache -> token-major [L][n_kv][D] of sequence b."""
    return np.ascontiguousarray(np.transpose(cache[b, :, :L, :], (1, 0, 2)))


def f32(x: np.ndarray) -> np.ndarray:
    """Exact fp16 -> f32 widening (the reference's buffers are f32)."""
    return np.asarray(x, np.float16).astype(np.float32)


def max_abs(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))
