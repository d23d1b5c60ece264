"""Writes tests/golden/decode_golden.npz: seeded fp16 decode-attention inputs
with float64 expected outputs.

The expected outputs come from numpy in float64 written from the definition
O[h] = sum_t softmax_t(q_h . k_t / sqrt(D)) v_t with kv head h // (H/Hkv)
(kernels/sparse_attn.wgsl:38-39,42,49,107), independently of the C oracle,
so the fixture pins the oracle rather than restating it. The reference
publishes no vectors of its own (it has no tests), so these are the only
fixtures.

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "decode_golden.npz"

# (name, n_heads, n_kv_heads, head_dim, seq, seed)
CASES = [
    ("cfg1_32q8kv_L153", 32, 8, 128, 153, 1001),   # the reference's runnable shape
    ("g5_40q8kv_L37", 40, 8, 128, 37, 1002),       # Nano-4B head layout (group 5)
    ("mha_8q8kv_L1", 8, 8, 128, 1, 1003),          # one key: O == V[0]
    ("g8_8q1kv_L300", 8, 1, 128, 300, 1004),       # group 8, > 256 keys
    ("g2_4q2kv_L65", 4, 2, 128, 65, 1005),         # one past a 64-key tile
    # shapes of the general kernels (any head size, any group)
    ("g3_6q2kv_d96_L200", 6, 2, 96, 200, 1006),    # group 3, head_dim 96
    ("d64_8q2kv_L129", 8, 2, 64, 129, 1007),       # head_dim 64
    ("d100_3q3kv_L70", 3, 3, 100, 70, 1008),       # head_dim not a multiple of 8
    ("d256_4q1kv_L90", 4, 1, 256, 90, 1009),       # head_dim 256
    ("g7_7q1kv_d32_L33", 7, 1, 32, 33, 1010),      # group 7
    ("d1_2q1kv_L5", 2, 1, 1, 5, 1011),             # head_dim 1
]


def expected(q: np.ndarray, k: np.ndarray, v: np.ndarray) -> np.ndarray:
    H, D = q.shape
    L, Hkv, _ = k.shape
    G = H // Hkv
    qd, kd, vd = (x.astype(np.float64) for x in (q, k, v))
    out = np.empty((H, D), np.float64)
    for h in range(H):
        s = kd[:, h // G, :] @ qd[h] / np.sqrt(D)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ vd[:, h // G, :]
    return out


def main() -> None:
    arrays = {}
    for name, H, Hkv, D, L, seed in CASES:
        g = np.random.Generator(np.random.PCG64(seed))
        q = g.standard_normal((H, D), dtype=np.float32).astype(np.float16)
        k = g.standard_normal((L, Hkv, D), dtype=np.float32).astype(np.float16)
        v = g.standard_normal((L, Hkv, D), dtype=np.float32).astype(np.float16)
        arrays[f"{name}__q"] = q.view(np.uint16)
        arrays[f"{name}__k"] = k.view(np.uint16)
        arrays[f"{name}__v"] = v.view(np.uint16)
        arrays[f"{name}__o"] = expected(q, k, v)
    arrays["cases"] = np.array([c[0] for c in CASES])
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


def load():
    """Yields (name, q f16, k f16 [L][Hkv][D], v f16, expected f64 [H][D])."""
    with np.load(OUT, allow_pickle=False) as z:
        for name in z["cases"]:
            name = str(name)
            yield (name, z[f"{name}__q"].view(np.float16), z[f"{name}__k"].view(np.float16),
                   z[f"{name}__v"].view(np.float16), z[f"{name}__o"])


if __name__ == "__main__":
    main()
