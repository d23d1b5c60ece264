"""The matrix-core split kernel of the decode (nwd_set_decode_kernel(ctx, 1)),
against the oracle and against the dot-product kernel, and the default
choice between the two.

Bar: max-abs <= 2e-3 against the oracle's op-for-op f32 restatement of
kernels/sparse_attn.wgsl (as the other decode tests); both kernels accumulate
in fp32 (the matrix-core one takes the fp32 weights as fp16 high and low
parts, and an fp32 query the same way), so their fp32 outputs agree within
1e-5; kv_append rows are bit-exact; the two merge forms give the same bits.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import nwd_attn as nw  # noqa: E402
import oracle  # noqa: E402
from attn_cases import f32, kv_rows, max_abs, normal_f16, rng, to_cache  # noqa: E402
from gpu_util import dev, host, pos_tensor, say  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 2e-3
AGREE = 1e-5
D = 128
VALU, MFMA = 0, 1


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    nw.load_library()


def _decode(ctx, kernel, q, kc, vc, pos, B, odt=torch.float32, max_len=0):
    ctx.set_decode_kernel(kernel)
    out = torch.empty((B, ctx.desc.n_heads, D), dtype=odt, device="cuda")
    ctx.decode(q, kc, vc, pos, out, B, max_len)
    return host(out).astype(np.float32)


@pytest.mark.parametrize("G", [1, 2, 4, 5, 8])
@pytest.mark.parametrize("q_dtype", ["f16", "f32"])
def test_matrix_core_kernel_matches_oracle(G, q_dtype):
    """Ragged lengths around the 32-key block and 128-key unit boundaries,
    every split count and both merges: oracle parity, agreement with the
    dot-product kernel, and merge forms bit for bit."""
    Hkv = 2 if G < 8 else 1
    H = G * Hkv
    past = [0, 31, 32, 127, 128, 1500]
    B, cap = len(past), 1600
    g = rng(900 + 10 * G + (q_dtype == "f32"))
    rows = [kv_rows(g, p + 1, Hkv) for p in past]
    q16 = normal_f16(g, (B, H, D))
    # an fp32 query off the fp16 grid: the kernel's high / low split matters
    q = f32(q16) + np.float32(1e-3) * g.standard_normal((B, H, D)).astype(np.float32) \
        if q_dtype == "f32" else q16
    with nw.AttnContext(H, Hkv, cap, max_batch=B, q_dtype=q_dtype, o_dtype="f32") as ctx:
        kc = dev(to_cache([r[0] for r in rows], Hkv, cap))
        vc = dev(to_cache([r[1] for r in rows], Hkv, cap))
        pos = pos_tensor(past)
        for n in (0, 1, 3, 16):
            ctx.set_decode_splits(n)
            outs = []
            for sep in (True, False):
                ctx.set_decode_merge(sep)
                outs.append(_decode(ctx, MFMA, dev(q), kc, vc, pos, B))
            say(f"matrix-core G={G} q={q_dtype} splits={n}")
            assert np.array_equal(outs[0], outs[1]), n
            ref = _decode(ctx, VALU, dev(q), kc, vc, pos, B)
            assert max_abs(outs[0], ref) < AGREE, n
        assert ctx.device_status() == nw.NWD_OK
    for b in range(B):
        want = oracle.sparse_attn_f32(f32(q[b]), f32(rows[b][0]), f32(rows[b][1]))
        assert max_abs(outs[0][b], want) < TOL, b


@pytest.mark.parametrize("G", [4, 5, 8])
@pytest.mark.parametrize("src", ["f16", "f32"])
def test_matrix_core_append_decode(G, src):
    """The fused append on the matrix-core kernel: new positions at the first
    and last key of a wavefront's 32-key block and of a 128-key unit; cache
    rows bit-identical to nwd_kv_append's, the output equal to kv_append +
    decode within fp32 rounding, for several split counts."""
    say(f"matrix-core append G={G} src={src}")
    Hkv = 2
    H = G * Hkv
    past = [0, 31, 32, 95, 127, 128, 700]
    B, cap = len(past), 800
    g = rng(950 + G)
    rows = [kv_rows(g, p, Hkv) for p in past]
    new16 = normal_f16(g, (B, Hkv, D), scale=3.0)
    newv16 = normal_f16(g, (B, Hkv, D))
    newk = f32(new16) if src == "f32" else new16
    newv = f32(newv16) if src == "f32" else newv16
    if src == "f32":
        newk = newk + np.float32(1e-4) * g.standard_normal(newk.shape).astype(np.float32)
    q = normal_f16(g, (B, H, D))
    with nw.AttnContext(H, Hkv, cap, max_batch=B, kv_dtype=src, o_dtype="f32") as ctx:
        ctx.set_decode_kernel(MFMA)
        base_k = to_cache([r[0] for r in rows], Hkv, cap)
        base_v = to_cache([r[1] for r in rows], Hkv, cap)
        pos = pos_tensor(past)
        kc1, vc1 = dev(base_k), dev(base_v)
        ctx.kv_append(dev(newk[:, None]), dev(newv[:, None]), kc1, vc1, pos, B, 1)
        want = _decode(ctx, MFMA, dev(q), kc1, vc1, pos, B, max_len=cap)
        for n in (0, 1, 3, 7):
            ctx.set_decode_splits(n)
            kc2, vc2 = dev(base_k), dev(base_v)
            out = torch.empty((B, H, D), dtype=torch.float32, device="cuda")
            ctx.append_decode(dev(q), dev(newk), dev(newv), kc2, vc2, pos, out, B, max_len=cap)
            assert np.array_equal(host(kc2).view(np.uint16), host(kc1).view(np.uint16)), n
            assert np.array_equal(host(vc2).view(np.uint16), host(vc1).view(np.uint16)), n
            assert max_abs(host(out), want) < AGREE, n
        assert ctx.device_status() == nw.NWD_OK
    for b in range(B):
        L = past[b] + 1
        kk = f32(host(kc1)[b, :, :L, :].transpose(1, 0, 2))
        vv = f32(host(vc1)[b, :, :L, :].transpose(1, 0, 2))
        assert max_abs(want[b], oracle.sparse_attn_f32(f32(q[b]), kk, vv)) < TOL, b


@pytest.mark.parametrize("fill", [0x7E00, 0x7C00, 0xFC00])
def test_matrix_core_stale_rows_past_length(fill):
    """Rows at or past L holding NaN or Inf (never read by the reference):
    the output is bit-identical to that of a zero-filled cache, with and
    without the fused append, for splits whose last key falls inside a
    wavefront's block."""
    Hkv, H, cap = 8, 40, 1100
    g = rng(960 + fill % 89)
    for L in (1, 5, 31, 33, 129, 1057):
        for B in (1, 3):
            rows = [kv_rows(g, L, Hkv) for _ in range(B)]
            q = normal_f16(g, (B, H, D))
            kn = normal_f16(g, (B, Hkv, D))
            vn = normal_f16(g, (B, Hkv, D))
            base_k = to_cache([r[0] for r in rows], Hkv, cap)
            base_v = to_cache([r[1] for r in rows], Hkv, cap)
            stale_k, stale_v = base_k.copy(), base_v.copy()
            stale_k[:, :, L:, :] = np.uint16(fill).view(np.float16)
            stale_v[:, :, L:, :] = np.uint16(fill).view(np.float16)
            pos = pos_tensor([L - 1] * B)
            caches = [(dev(base_k), dev(base_v)), (dev(stale_k), dev(stale_v))]
            with nw.AttnContext(H, Hkv, cap, max_batch=B, o_dtype="f32") as ctx:
                ctx.set_decode_kernel(MFMA)
                for n in (0, 3):
                    for max_len in (L, 0):
                        say(f"matrix-core stale fill={fill:#06x} L={L} B={B} splits={n} max_len={max_len}")
                        ctx.set_decode_splits(n)
                        outs = []
                        for kcd, vcd in caches:
                            o1 = _decode(ctx, MFMA, dev(q), kcd, vcd, pos, B, max_len=max_len)
                            o2 = torch.empty((B, H, D), dtype=torch.float32, device="cuda")
                            ctx.append_decode(dev(q), dev(kn), dev(vn), kcd.clone(), vcd.clone(),
                                              pos, o2, B, max_len)
                            outs.append((o1, host(o2)))
                        assert np.all(np.isfinite(outs[0][0])) and np.all(np.isfinite(outs[0][1]))
                        key = (L, B, n, max_len)
                        assert np.array_equal(outs[0][0], outs[1][0]), key
                        assert np.array_equal(outs[0][1], outs[1][1]), key
                assert ctx.device_status() == nw.NWD_OK
            want = oracle.sparse_attn_f32(f32(q[0]), f32(rows[0][0]), f32(rows[0][1]))
            assert max_abs(outs[1][0][0], want) < TOL, L


@pytest.mark.parametrize("offset", [0.0, -60.0])
def test_matrix_core_rising_and_negative_scores(offset):
    """Scores that climb ~26 log2 units across 1000 keys: the weights of
    later blocks overflow fp16 against a wavefront's first reference point,
    so the overflow path (maximum, rescale, weights again) runs; offset -60
    puts every score near -87 log2 units, where weights without a maximum
    would underflow. Checked against a float64 softmax of the same inputs."""
    say(f"matrix-core rising scores offset={offset}")
    H, Hkv, L = 40, 8, 1000
    g = rng(4477)
    u = g.standard_normal(D)
    u /= np.linalg.norm(u)
    q = (np.tile(4.0 * u, (1, H, 1)) + 0.05 * g.standard_normal((1, H, D))).astype(np.float16)
    j = np.arange(L, dtype=np.float64)[:, None]
    base = (0.05 * j + offset * np.sqrt(D) / 4.0) * u[None, :]
    k = np.stack([base + 0.05 * g.standard_normal((L, D)) for _ in range(Hkv)], axis=1).astype(np.float16)
    v = g.standard_normal((L, Hkv, D)).astype(np.float16)
    with nw.AttnContext(H, Hkv, L, o_dtype="f32") as ctx:
        kc = dev(np.ascontiguousarray(k.transpose(1, 0, 2))[None])
        vc = dev(np.ascontiguousarray(v.transpose(1, 0, 2))[None])
        for n in (1, 4):
            ctx.set_decode_splits(n)
            got = _decode(ctx, MFMA, dev(q), kc, vc, pos_tensor([L - 1]), 1)[0]
            G = H // Hkv
            worst = 0.0
            kf, vf, qf = k.astype(np.float64), v.astype(np.float64), q[0].astype(np.float64)
            for h in range(H):
                s = kf[:, h // G] @ qf[h] / np.sqrt(D)
                w = np.exp(s - s.max())
                want = (w[:, None] * vf[:, h // G]).sum(axis=0) / w.sum()
                worst = max(worst, float(np.abs(got[h] - want).max()))
            assert worst < TOL, (n, worst)
        assert ctx.device_status() == nw.NWD_OK


def test_default_kernel_choice():
    """Without nwd_set_decode_kernel a call that runs one workgroup per KV
    head takes the matrix-core kernel for G >= 5, or G = 4 with batch >= 2 or
    with splits of at least 512 keys whose workgroups fit 256 at once, and the
    dot-product kernel otherwise; a call that runs one workgroup per query
    head takes the dot-product kernel. The default result equals the chosen
    kernel's bits."""
    cases = [  # (H, Hkv, B, L, splits, expected kernel)
        (64, 8, 1, 3000, 0, MFMA),
        (40, 8, 1, 20000, 32, MFMA),
        (40, 8, 1, 3000, 32, MFMA),
        (40, 8, 1, 1000, 0, VALU),   # 6 splits x 40 heads <= 256: one workgroup per query head
        (32, 8, 1, 20000, 32, MFMA),  # 625 keys per split, 256 workgroups
        (32, 8, 1, 12000, 32, VALU),  # 375 keys per split
        (32, 8, 1, 20000, 33, VALU),  # 264 workgroups
        (32, 8, 2, 3000, 0, MFMA),
        (32, 8, 9, 300, 0, MFMA),
        (16, 8, 1, 3000, 0, VALU),
        (16, 8, 4, 3000, 0, VALU),
    ]
    for H, Hkv, B, L, n, kernel in cases:
        say(f"default kernel H={H} Hkv={Hkv} B={B} L={L} splits={n}")
        g = rng(990 + H + L + B)
        rows = [kv_rows(g, L - 7 * b, Hkv) for b in range(B)]
        q = normal_f16(g, (B, H, D))
        with nw.AttnContext(H, Hkv, L, max_batch=B, o_dtype="f32") as ctx:
            ctx.set_decode_splits(n)
            kc = dev(to_cache([r[0] for r in rows], Hkv, L))
            vc = dev(to_cache([r[1] for r in rows], Hkv, L))
            pos = pos_tensor([L - 1 - 7 * b for b in range(B)])
            default = _decode(ctx, -1, dev(q), kc, vc, pos, B)
            chosen = _decode(ctx, kernel, dev(q), kc, vc, pos, B)
            other = _decode(ctx, 1 - kernel, dev(q), kc, vc, pos, B)
            assert np.array_equal(default, chosen), (H, B, L)
            assert max_abs(default, other) < AGREE, (H, B, L)
            assert ctx.device_status() == nw.NWD_OK
        for b in range(B):
            want = oracle.sparse_attn_f32(f32(q[b]), f32(rows[b][0]), f32(rows[b][1]))
            assert max_abs(default[b], want) < TOL, (H, B, L, b)


def test_set_decode_kernel_rejects_unknown_values():
    with nw.AttnContext(32, 8, 64) as ctx:
        for bad in (2, -2, 7):
            with pytest.raises(nw.NwdError) as e:
                ctx.set_decode_kernel(bad)
            assert e.value.code == nw.NWD_ERR_INVALID
