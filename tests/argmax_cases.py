"""The greedy-pick rule of kernels/argmax_partial.wgsl + argmax_merge.wgsl
(dispatched as 256 slices of ceil(n / 256) logits, engine/runtime.js:209,
398-399) in closed form, and tie-heavy test inputs.

Rule: among the indices whose value is strictly above -3.402823466e38 (NaN
never qualifies), take the largest value. Index i sits in slice
i // n_slice at thread (i - start) % 256, step (i - start) // 256. A thread
keeps its first maximum (strict >), so the smaller step wins a tie. The
256-wide trees (threads in argmax_partial, slices in argmax_merge) keep the
left position on ties, halving the stride each round: two tied entries meet
at the lowest bit where their positions differ and the one with a 0 there
wins, so the smaller bit-reversed position wins. Ties therefore go to the
smallest (bitrev8(slice), bitrev8(thread), step). If no value qualifies the
result is 0.
"""
from __future__ import annotations

import numpy as np

NEG_FLT_MAX = np.float32(-3.402823466e38)


def bitrev8(v: np.ndarray) -> np.ndarray:
    v = np.asarray(v, np.int64)
    out = np.zeros_like(v)
    for b in range(8):
        out |= ((v >> b) & 1) << (7 - b)
    return out


def walk_key(n: int) -> np.ndarray:
    """Rank of every index in the reference's tie order (smaller wins)."""
    n_slice = (n + 255) // 256
    steps = (n_slice + 255) // 256
    i = np.arange(n, dtype=np.int64)
    wg = i // n_slice
    r = i - wg * n_slice
    return (bitrev8(wg) * 256 + bitrev8(r % 256)) * steps + r // 256


def reference_rule(x: np.ndarray) -> int:
    x = np.asarray(x, np.float32)
    ok = x > NEG_FLT_MAX
    if not ok.any():
        return 0
    best = x[ok].max()
    cand = np.nonzero(ok & (x == best))[0]
    return int(cand[np.argmin(walk_key(len(x))[cand])])


def tie_heavy(g: np.random.Generator, n: int) -> np.ndarray:
    """Few distinct values (many exact ties), some -inf / NaN / -FLT_MAX."""
    x = g.integers(-3, 3, size=n).astype(np.float32)
    specials = g.integers(0, n, size=max(1, n // 50))
    x[specials[0::3]] = -np.inf
    x[specials[1::3]] = np.nan
    x[specials[2::3]] = NEG_FLT_MAX
    return x
