"""Pins the CPU oracle (oracle/attn_oracle.c) before the GPU results are checked against it.

Every oracle function is checked against something it does not restate:
numpy's float16 conversion, closed forms, an independent numpy float64
attention, the committed golden vectors, and special cases whose answer the
mathematics fixes. The last test plants mistakes in a copy of the oracle's
math (on the CPU) and shows these checks catch them.
"""
import numpy as np
import pytest

import oracle
from attn_cases import f32, kv_rows, max_abs, normal_f16, rng
from golden.make_golden import load as load_golden

D = 128


def np_attn64(q, k, v, scale=None):
    """Independent float64 attention: q [H][D], k/v [L][Hkv][D]."""
    H, Dq = q.shape
    L, Hkv, _ = k.shape
    G = H // Hkv
    scale = 1.0 / np.sqrt(Dq) if scale is None else scale
    qd, kd, vd = (np.asarray(x, np.float64) for x in (q, k, v))
    kh = kd[:, np.arange(H) // G, :]  # [L][H][D]
    vh = vd[:, np.arange(H) // G, :]
    s = np.einsum("hd,lhd->hl", qd, kh) * scale
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=1, keepdims=True)
    return np.einsum("hl,lhd->hd", p, vh)


# ------------------------------------------------------------------ fp16 ---

def test_f16_widen_every_pattern():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = oracle.f16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f16_roundtrip_every_pattern():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    back = oracle.f32_to_f16(oracle.f16_to_f32(bits))
    finite_or_inf = ~np.isnan(bits.view(np.float16))
    assert np.array_equal(back[finite_or_inf], bits[finite_or_inf])
    assert np.all(np.isnan(back[~finite_or_inf].view(np.float16)))


def test_f16_narrow_matches_numpy_rne():
    g = rng(7)
    # random magnitudes over the whole fp16 range and beyond
    x = (g.standard_normal(200000) * np.exp2(g.uniform(-30, 18, 200000))).astype(np.float32)
    # exact ties between neighbouring fp16 values (normal and subnormal)
    h = np.arange(0, 0x7BFF, 37, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    ties = ((lo + hi) / 2).astype(np.float32)
    edges = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, np.inf, -np.inf,
                      2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 2.0 ** -26, 2.0 ** -14,
                      2.0 ** -14 * (1 - 2.0 ** -11), 6.1e-5, -3e-8], np.float32)
    for arr in (x, ties, -ties, edges):
        ours = oracle.f32_to_f16(arr)
        with np.errstate(over="ignore"):  # values past 65520 are meant to overflow to inf
            ref = arr.astype(np.float16).view(np.uint16)
        assert np.array_equal(ours, ref)
    assert np.isnan(oracle.f32_to_f16(np.array([np.nan], np.float32)).view(np.float16)[0])


# ------------------------------------------------------------- kv_append ---

def test_kv_append_closed_form():
    n_kv, hd, cap = 8, 128, 6
    g = rng(11)
    canary = np.float32(-1234.5)
    cache = np.full(cap * n_kv * hd, canary, np.float32)
    src = g.standard_normal(n_kv * hd, dtype=np.float32)
    src[:4] = [np.inf, -0.0, 1e-42, np.float32(3.0)]  # bit patterns must survive
    oracle.kv_append_f32(src, cache, 3, n_kv, hd)
    rows = cache.reshape(cap, n_kv * hd)
    assert np.array_equal(rows[3].view(np.uint32), src.view(np.uint32))
    others = np.delete(rows, 3, axis=0)
    assert np.all(others == canary)


# ------------------------------------------------------------- attention ---

@pytest.mark.parametrize("H,Hkv,L", [(8, 2, 1), (8, 2, 2), (8, 2, 63), (8, 2, 64), (8, 2, 65),
                                     (32, 8, 153), (40, 8, 255), (8, 1, 256), (4, 4, 257),
                                     (16, 8, 1000)])
def test_f64_matches_numpy(H, Hkv, L):
    g = rng(100 + L)
    q = f32(normal_f16(g, (H, D)))
    k, v = (f32(a) for a in kv_rows(g, L, Hkv))
    assert max_abs(oracle.attn_f64(q, k, v), np_attn64(q, k, v)) < 1e-12


@pytest.mark.parametrize("L", [1, 2, 3, 31, 63, 64, 65, 127, 128, 129, 153, 255, 256, 257, 600])
def test_f32_restatement_tracks_f64(L):
    g = rng(200 + L)
    q = f32(normal_f16(g, (32, D)))
    k, v = (f32(a) for a in kv_rows(g, L, 8))
    assert max_abs(oracle.sparse_attn_f32(q, k, v), oracle.attn_f64(q, k, v)) < 1e-5


def test_f32_threads_bitwise_equal():
    g = rng(5)
    q = f32(normal_f16(g, (32, D)))
    k, v = (f32(a) for a in kv_rows(g, 777, 8))
    a = oracle.sparse_attn_f32(q, k, v, threads=1)
    b = oracle.sparse_attn_f32(q, k, v, threads=0)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_golden_vectors():
    n = 0
    for name, q, k, v, want in load_golden():
        o32 = oracle.sparse_attn_f32(f32(q), f32(k), f32(v))
        o64 = oracle.attn_f64(f32(q), f32(k), f32(v))
        assert max_abs(o64, want) < 1e-12, name
        assert max_abs(o32, want) < 1e-5, name
        n += 1
    assert n == 11  # 5 at head_dim 128, 6 of other head sizes and groups


def test_special_cases():
    g = rng(9)
    H, Hkv = 8, 2
    q = f32(normal_f16(g, (H, D)))
    # one key: softmax weight is exactly 1 in both precisions
    k, v = (f32(a) for a in kv_rows(g, 1, Hkv))
    for fn in (oracle.sparse_attn_f32, oracle.attn_f64):
        o = fn(q, k, v)
        assert np.array_equal(o.astype(np.float32), np.repeat(v[0], H // Hkv, axis=0))
    # V constant over t -> O is that constant
    L = 300
    k, _ = (f32(a) for a in kv_rows(g, L, Hkv))
    c = f32(normal_f16(g, (1, Hkv, D)))
    v = np.repeat(c, L, axis=0)
    want = np.repeat(c[0], H // Hkv, axis=0)
    assert max_abs(oracle.sparse_attn_f32(q, k, v), want) < 1e-5
    assert max_abs(oracle.attn_f64(q, k, v), want) < 1e-12
    # Q = 0 -> uniform weights -> mean of V
    k, v = (f32(a) for a in kv_rows(g, L, Hkv))
    z = np.zeros((H, D), np.float32)
    want = np.repeat(v.astype(np.float64).mean(axis=0), H // Hkv, axis=0)
    assert max_abs(oracle.sparse_attn_f32(z, k, v), want) < 1e-5
    assert max_abs(oracle.attn_f64(z, k, v), want) < 1e-12
    # one dominant key (K row = 8 * q) selects its V row (max tracking)
    qq = f32(normal_f16(g, (H, D)))
    kk = k.copy()
    kk[137, 0, :] = 8.0 * qq[0]
    o = oracle.sparse_attn_f32(qq, kk, v)
    assert max_abs(o[0], v[137, 0]) < 1e-5
    # joint permutation of (K, V) rows leaves O unchanged
    perm = g.permutation(L)
    assert max_abs(oracle.sparse_attn_f32(q, k[perm], v[perm]), oracle.sparse_attn_f32(q, k, v)) < 1e-5
    assert max_abs(oracle.attn_f64(q, k[perm], v[perm]), oracle.attn_f64(q, k, v)) < 1e-12
    # GQA: query heads of one group with equal queries give equal outputs
    qg = q.copy()
    qg[1:4] = qg[0]
    o = oracle.sparse_attn_f32(qg, k, v)
    assert np.array_equal(o[0], o[1]) and np.array_equal(o[0], o[3])
    assert max_abs(o[0], o[4]) > 1e-3  # the next group reads another kv head


def test_rejects_bad_shapes():
    q = np.zeros((6, D), np.float32)
    k = np.zeros((3, 4, D), np.float32)
    with pytest.raises(ValueError):
        oracle.sparse_attn_f32(q, k, k)  # 6 % 4 != 0
    with pytest.raises(ValueError):
        oracle.sparse_attn_f32(np.zeros((4, D), np.float32), np.zeros((0, 4, D), np.float32),
                               np.zeros((0, 4, D), np.float32))


@pytest.mark.parametrize("mistake", ["no_scale", "wrong_group_map", "k_transposed",
                                     "max_not_subtracted_sum_order", "v_of_next_key"])
def test_checks_catch_planted_mistakes(mistake):
    """Plants a plausible mistake in a numpy copy of the math and shows the
    checks above (comparison with the C oracle at 2e-3, the decode
    tolerance) reject it — so agreement with them is evidence."""
    g = rng(31)
    H, Hkv, L = 32, 8, 153
    q = f32(normal_f16(g, (H, D)))
    k, v = (f32(a) for a in kv_rows(g, L, Hkv))
    G = H // Hkv
    kh = k[:, np.arange(H) // G, :].astype(np.float64)
    vh = v[:, np.arange(H) // G, :].astype(np.float64)
    scale = 1 / np.sqrt(D)
    if mistake == "no_scale":
        scale = 1.0
    if mistake == "wrong_group_map":
        kh = k[:, np.arange(H) % Hkv, :].astype(np.float64)
        vh = v[:, np.arange(H) % Hkv, :].astype(np.float64)
    if mistake == "k_transposed":
        kh = kh[::-1]
    s = np.einsum("hd,lhd->hl", q.astype(np.float64), kh) * scale
    if mistake == "max_not_subtracted_sum_order":
        s = s - s.mean(axis=1, keepdims=True)  # a wrong shift changes nothing...
        s[:, -1] += 0.5                        # ...so also drop a term's weight
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    if mistake == "v_of_next_key":
        vh = np.roll(vh, 1, axis=0)
    wrong = np.einsum("hl,lhd->hd", p, vh)
    assert max_abs(wrong, oracle.sparse_attn_f32(q, k, v)) > 2e-3
