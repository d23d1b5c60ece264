"""Parity of the HIP decode path (nwd_kv_append + nwd_decode_attn) with the
oracle, through the C ABI, on the five workload shapes and their edge cases.

Bar: kv_append bit-exact; attention max-abs <= 2e-3 against the oracle's
op-for-op f32 restatement of kernels/sparse_attn.wgsl (inputs widened
fp16 -> f32 exactly, as the reference's buffers are f32).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import nwd_attn as nw  # noqa: E402
import oracle  # noqa: E402
from attn_cases import f32, from_cache, kv_rows, max_abs, normal_f16, rng, to_cache  # noqa: E402
from golden.make_golden import load as load_golden  # noqa: E402
from gpu_util import cache_rows_f32, dev, host, pos_tensor, randn_f16, say  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 2e-3  # max-abs, fp32 accumulation with fp16 I/O
D = 128


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    nw.load_library()


def _decode(ctx, q, kc, vc, pos, batch, out_dtype=torch.float16, max_len=0):
    H = ctx.desc.n_heads
    out = torch.empty((batch, H, ctx.desc.head_dim), dtype=out_dtype, device="cuda")
    ctx.decode(q, kc, vc, pos, out, batch, max_len)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def test_loaded_library_matches_sources():
    """The library these GPU tests load was built from the sources on disk
    (nwd_source_hash against build.source_hash), so their evidence is tied to
    this tree."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("nwd_build_for_hash", nw.PKG_DIR / "build.py")
    build = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(build)
    say(f"library sources sha256 {nw.source_hash()[:16]}")
    assert nw.source_hash() == build.source_hash()


# -------------------------------------------------------------- kv_append ---

def test_kv_append_bit_exact_f16():
    say("kv_append f16 bit-exact: B=3 n_tokens=5 cap=64")
    B, n_tok, cap, n_kv = 3, 5, 64, 8
    g = rng(41)
    bits = g.integers(0, 65536, size=(2, B, n_tok, n_kv, D), dtype=np.uint32).astype(np.uint16)
    bits[0, 0, 0, 0, :8] = [0x0000, 0x8000, 0x0001, 0x03FF, 0x7C00, 0xFC00, 0x7E00, 0x7BFF]
    canary = np.uint16(0x7E5A)
    with nw.AttnContext(32, n_kv, cap, max_batch=B) as ctx:
        kc = torch.full((B, n_kv, cap, D), int(np.int16(canary.view(np.int16))), dtype=torch.int16,
                        device="cuda")
        vc = kc.clone()
        pos = [0, 17, cap - n_tok]
        ctx.kv_append(dev(bits[0].view(np.int16)), dev(bits[1].view(np.int16)), kc, vc,
                      pos_tensor(pos), B, n_tok)
        assert ctx.device_status() == nw.NWD_OK
        for which, c in ((0, kc), (1, vc)):
            want = np.full((B, n_kv, cap, D), canary, np.uint16)
            for b in range(B):
                for j in range(n_tok):
                    want[b, :, pos[b] + j, :] = bits[which, b, j]
            got = host(c).view(np.uint16)
            assert np.array_equal(got, want)
            # the documented offset helper names the same element
            assert ctx.cache_offset(1, 17, 3, 5) == ((1 * n_kv + 3) * cap + 17) * D + 5


def test_kv_append_f32_rows_round_to_nearest_even():
    say("kv_append f32 -> f16 RNE")
    n_kv, cap = 8, 16
    g = rng(42)
    x = (g.standard_normal((1, 1, n_kv, D)) * np.exp2(g.uniform(-26, 17, (1, 1, n_kv, D)))).astype(np.float32)
    h = np.arange(0x0001, 0x7BFF, 97, dtype=np.uint16)[: D]
    ties = ((h.view(np.float16).astype(np.float64) + (h + 1).view(np.float16).astype(np.float64)) / 2)
    x[0, 0, 0, : ties.size] = ties.astype(np.float32)
    x[0, 0, 1, :4] = [65520.0, -65519.0, 1e-9, -0.0]
    with nw.AttnContext(32, n_kv, cap, kv_dtype="f32") as ctx:
        kc = torch.zeros((1, n_kv, cap, D), dtype=torch.float16, device="cuda")
        vc = torch.zeros_like(kc)
        ctx.kv_append(dev(x), dev(-x), kc, vc, pos_tensor([9]), 1, 1)
        want_k = oracle.f32_to_f16(x[0, 0])
        want_v = oracle.f32_to_f16(-x[0, 0])
        assert np.array_equal(host(kc)[0, :, 9, :].view(np.uint16), want_k)
        assert np.array_equal(host(vc)[0, :, 9, :].view(np.uint16), want_v)


def test_kv_append_past_capacity_is_flagged_not_written():
    say("kv_append past capacity")
    n_kv, cap = 8, 8
    with nw.AttnContext(32, n_kv, cap) as ctx:
        kc = torch.zeros((1, n_kv, cap, D), dtype=torch.float16, device="cuda")
        vc = torch.zeros_like(kc)
        rows = torch.ones((1, 4, n_kv, D), dtype=torch.float16, device="cuda")
        ctx.kv_append(rows, rows, kc, vc, pos_tensor([6]), 1, 4)  # tokens 6, 7 fit; 8, 9 do not
        assert ctx.device_status() == nw.NWD_ERR_DEVICE
        assert "position" in ctx.last_error()
        got = host(kc)
        assert np.all(got[0, :, 6:8, :] == 1) and np.all(got[0, :, :6, :] == 0)
        assert ctx.device_status() == nw.NWD_OK  # the flag was cleared


# ---------------------------------------------------------------- decode ---

def test_golden_vectors():
    for name, q, k, v, want in load_golden():
        say("golden", name)
        H, Dq = q.shape
        L, Hkv, _ = k.shape
        with nw.AttnContext(H, Hkv, L + 3, head_dim=Dq, o_dtype="f32") as ctx:
            kc = dev(to_cache([k], Hkv, L + 3))
            vc = dev(to_cache([v], Hkv, L + 3))
            got = _decode(ctx, dev(q[None]), kc, vc, pos_tensor([L - 1]), 1, torch.float32)[0]
        assert max_abs(got, want) < TOL, name
        assert max_abs(got, oracle.sparse_attn_f32(f32(q), f32(k), f32(v))) < TOL, name


@pytest.mark.parametrize("o_dtype", ["f16", "f32"])
def test_config1_past152(o_dtype):
    """32q/8kv/d128, 152 cached tokens + 1 appended at pos 152 -> L = 153."""
    say("config1 past=152", o_dtype)
    H, Hkv, P = 32, 8, 152
    g = rng(1)
    q = normal_f16(g, (1, H, D))
    k, v = kv_rows(g, P + 1, Hkv)
    cap = 256
    with nw.AttnContext(H, Hkv, cap, o_dtype=o_dtype) as ctx:
        kc = dev(to_cache([k[:P]], Hkv, cap))
        vc = dev(to_cache([v[:P]], Hkv, cap))
        pos = pos_tensor([P])
        ctx.kv_append(dev(k[P:P + 1][None]), dev(v[P:P + 1][None]), kc, vc, pos, 1, 1)
        got = _decode(ctx, dev(q), kc, vc, pos, 1,
                      torch.float16 if o_dtype == "f16" else torch.float32, max_len=P + 1)[0]
        assert ctx.device_status() == nw.NWD_OK
        # the appended rows are bit-exact in the cache
        assert np.array_equal(host(kc)[0, :, P, :].view(np.uint16), k[P].view(np.uint16))
    want = oracle.sparse_attn_f32(f32(q[0]), f32(k), f32(v))
    assert max_abs(got, want) < TOL


@pytest.mark.parametrize("path", ["append_then_decode", "fused_append_decode"])
def test_config2_past4096_64_steps(path):
    """Per-KV-head scale U[0.5, 2]; append one token and attend, 64 times,
    either as nwd_kv_append + nwd_decode_attn or as one nwd_append_decode."""
    H, Hkv, P, steps = 32, 8, 4096, 64
    g = rng(2)
    hs = g.uniform(0.5, 2.0, Hkv)
    k, v = kv_rows(g, P + steps, Hkv, head_scale=hs)
    qs = normal_f16(g, (steps, 1, H, D))
    cap = P + steps
    kf, vf = f32(k), f32(v)
    with nw.AttnContext(H, Hkv, cap) as ctx:
        kc = dev(to_cache([k[:P]], Hkv, cap))
        vc = dev(to_cache([v[:P]], Hkv, cap))
        worst = 0.0
        for i in range(steps):
            p = P + i
            if i % 16 == 0:
                say(f"config2 step {i} pos={p}")
            pos = pos_tensor([p])
            if path == "append_then_decode":
                ctx.kv_append(dev(k[p:p + 1][None]), dev(v[p:p + 1][None]), kc, vc, pos, 1, 1)
                got = _decode(ctx, dev(qs[i]), kc, vc, pos, 1, max_len=p + 1)[0]
            else:
                out = torch.empty((1, H, D), dtype=torch.float16, device="cuda")
                ctx.append_decode(dev(qs[i]), dev(k[p:p + 1]), dev(v[p:p + 1]), kc, vc, pos, out, 1,
                                  max_len=cap)
                got = out.float().cpu().numpy()[0]
            want = oracle.sparse_attn_f32(f32(qs[i, 0]), kf[:p + 1], vf[:p + 1], threads=0)
            worst = max(worst, max_abs(got, want))
        assert ctx.device_status() == nw.NWD_OK
        assert np.array_equal(host(kc)[0].transpose(1, 0, 2).view(np.uint16), k.view(np.uint16))
    assert worst < TOL, worst


@pytest.mark.parametrize("kernel", [0, 1])
def test_config3_past32768_outliers_split_k(kernel):
    """L = 32769 with 1% +-8 outliers; split-K + merge, and split-count
    invariance; on the dot-product split kernel and on the matrix-core one."""
    H, Hkv, P = 32, 8, 32768
    say(f"config3 past=32768 kernel={kernel}")
    g = rng(3)
    k, v = kv_rows(g, P + 1, Hkv, outlier_frac=0.01)
    q = normal_f16(g, (1, H, D))
    cap = P + 1
    want = oracle.sparse_attn_f32(f32(q[0]), f32(k), f32(v), threads=0)
    with nw.AttnContext(H, Hkv, cap) as ctx:
        ctx.set_decode_kernel(kernel)
        kc = dev(to_cache([k[:P]], Hkv, cap))
        vc = dev(to_cache([v[:P]], Hkv, cap))
        pos = pos_tensor([P])
        ctx.kv_append(dev(k[P:][None]), dev(v[P:][None]), kc, vc, pos, 1, 1)
        auto = ctx.decode_splits(1, P + 1)
        assert auto > 1
        outs = {}
        for n in (0, 1, 7, 256):
            for sep in (True, False):
                say(f"config3 splits={n or auto} separate_merge={sep}")
                ctx.set_decode_splits(n)
                ctx.set_decode_merge(sep)
                o = _decode(ctx, dev(q), kc, vc, pos, 1, max_len=P + 1)[0]
                assert max_abs(o, want) < TOL, (n, sep)
                if not sep:  # same records, same merge order: bit-identical
                    assert np.array_equal(o, outs[n]), n
                outs[n] = o
        # a length bound below the true length still gives the exact result
        ctx.set_decode_splits(0)
        short = _decode(ctx, dev(q), kc, vc, pos, 1, max_len=1000)[0]
        assert max_abs(short, want) < TOL
        assert ctx.device_status() == nw.NWD_OK
    for n in (1, 7, 256):
        assert max_abs(outs[n], outs[0]) < 1e-3


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("kernel", [0, 1])
def test_config4_ragged_batch64(kernel, layout):
    """64 sequences, past lengths U{512..16384}, one query each: one new token
    per sequence appended at pos = past and attended, both as nwd_kv_append +
    nwd_decode_attn and as the fused nwd_append_decode the benchmark times.
    The fused path writes the same cache bits and gives the same output bits;
    every sequence matches the oracle. On the dot-product split kernel and
    on the matrix-core one (the default for this batch), with each split
    owning one key range (layout 0) and with the splits' key blocks
    interleaved (layout 1, the default for batches)."""
    H, Hkv, B = 32, 8, 64
    g = rng(4)
    past = g.integers(512, 16385, size=B)
    cap = int(past.max()) + 1
    say(f"config4 ragged B={B} cap={cap} sum_L={int(past.sum() + B)} kernel={kernel} layout={layout}")
    kc = randn_f16((B, Hkv, cap, D), 40)
    vc = randn_f16((B, Hkv, cap, D), 41)
    q = randn_f16((B, H, D), 42)
    kn = randn_f16((B, Hkv, D), 43)
    vn = randn_f16((B, Hkv, D), 44)
    pos = pos_tensor(past.tolist())
    with nw.AttnContext(H, Hkv, cap, max_batch=B) as ctx:
        ctx.set_decode_kernel(kernel)
        ctx.set_decode_layout(layout)
        kc2, vc2 = kc.clone(), vc.clone()
        ctx.kv_append(kn[:, None], vn[:, None], kc, vc, pos, B, 1)
        out = _decode(ctx, q, kc, vc, pos, B, max_len=cap)
        say("config4 fused append_decode B=64")
        fused = torch.empty((B, H, D), dtype=torch.float16, device="cuda")
        ctx.append_decode(q, kn, vn, kc2, vc2, pos, fused, B, cap)
        assert ctx.device_status() == nw.NWD_OK
        assert torch.equal(kc2, kc) and torch.equal(vc2, vc)  # appended rows bit-exact
        fused = fused.float().cpu().numpy()
    assert np.array_equal(fused, out)
    qh = q.float().cpu().numpy()
    worst = 0.0
    for b in range(B):
        L = int(past[b]) + 1
        want = oracle.sparse_attn_f32(qh[b], cache_rows_f32(kc, b, L), cache_rows_f32(vc, b, L),
                                      threads=0)
        worst = max(worst, max_abs(out[b], want))
    assert worst < TOL, worst


@pytest.mark.parametrize("kernel", [0, 1])
def test_strided_layout(kernel):
    """Split s owning the key blocks s, s + n, ... (nwd_set_decode_layout 1)
    against the oracle and against the contiguous layout: lengths around the
    block sizes (32 keys for the dot-product kernel, 64 for the matrix-core
    one), split counts that leave some splits without keys, the fused append
    (same cache bits as nwd_kv_append, same output bits as the two calls),
    both merge forms (same bits), a length bound below the true length,
    32K keys with outliers, and NaN rows past L that must not leak."""
    H, Hkv = 32, 8
    for L, splits in ((1, 3), (33, 2), (64, 2), (65, 2), (129, 5), (1000, 0), (1000, 7),
                      (5000, 0), (5000, 256), (32769, 0), (32769, 24)):
        say(f"strided layout kernel={kernel} L={L} splits={splits}")
        g = rng(700 + L + splits)
        k, v = kv_rows(g, L, Hkv, outlier_frac=0.01 if L > 30000 else 0.0)
        q = normal_f16(g, (1, H, D))
        want = oracle.sparse_attn_f32(f32(q[0]), f32(k), f32(v), threads=0)
        cap = L + 40
        stale_k = to_cache([k[:L - 1]], Hkv, cap)
        stale_v = to_cache([v[:L - 1]], Hkv, cap)
        stale_k[:, :, L:, :] = np.uint16(0x7E00).view(np.float16)
        stale_v[:, :, L:, :] = np.uint16(0x7E00).view(np.float16)
        pos = pos_tensor([L - 1])
        kn, vn = dev(k[L - 1:][None]), dev(v[L - 1:][None])
        with nw.AttnContext(H, Hkv, cap, o_dtype="f32") as ctx:
            ctx.set_decode_kernel(kernel)
            ctx.set_decode_splits(splits)
            outs = {}
            for layout in (0, 1):
                ctx.set_decode_layout(layout)
                for sep in (True, False):
                    ctx.set_decode_merge(sep)
                    kc, vc = dev(stale_k), dev(stale_v)
                    fused = torch.empty((1, H, D), dtype=torch.float32, device="cuda")
                    ctx.append_decode(dev(q), kn, vn, kc, vc, pos, fused, 1, L)
                    kc2, vc2 = dev(stale_k), dev(stale_v)
                    ctx.kv_append(kn[:, None], vn[:, None], kc2, vc2, pos, 1, 1)
                    assert torch.equal(kc.view(torch.int16), kc2.view(torch.int16))
                    assert torch.equal(vc.view(torch.int16), vc2.view(torch.int16))
                    two = _decode(ctx, dev(q), kc2, vc2, pos, 1, torch.float32, max_len=L)
                    short = _decode(ctx, dev(q), kc2, vc2, pos, 1, torch.float32,
                                    max_len=max(1, L // 3))
                    assert ctx.device_status() == nw.NWD_OK
                    f = host(fused)
                    assert np.array_equal(f, two), (L, splits, layout, sep)
                    assert max_abs(f[0], want) < TOL, (L, splits, layout, sep)
                    assert max_abs(short[0], want) < TOL, (L, splits, layout, sep)
                    if not sep:
                        assert np.array_equal(f, outs[(layout, True)]), (L, splits, layout)
                    outs[(layout, sep)] = f
            assert max_abs(outs[(1, True)], outs[(0, True)]) < 1e-4


@pytest.mark.parametrize("fill", [0x7E00, 0x7C00, 0xFC00])
def test_stale_rows_past_length_do_not_leak(fill):
    """Cache rows at or past L are never read by the reference (it loops
    t < seq, kernels/sparse_attn.wgsl:45-113) and may hold anything, e.g.
    NaN or Inf in an uncleared cache. The output must be bit-identical to
    that of a zero-filled cache, for every decode form: one split (one
    workgroup per query head), several splits, per-KV-head workgroups (B=9),
    both merge forms, and the fused append, with L - t0 < 32 for the split
    holding the last key."""
    Hkv, H, cap = 8, 32, 1100
    g = rng(500 + fill % 97)
    for L in (1, 5, 31, 129, 150, 257, 1025, 1057):
        for B in (1, 9):
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
                for n in (0, 1, 3, 8):
                    for sep in (True, False):
                        for max_len in (L, 0):
                            say(f"stale rows fill={fill:#06x} L={L} B={B} splits={n} "
                                f"separate={sep} max_len={max_len}")
                            ctx.set_decode_splits(n)
                            ctx.set_decode_merge(sep)
                            outs = []
                            for kcd, vcd in caches:
                                o1 = _decode(ctx, dev(q), kcd, vcd, pos, B, torch.float32,
                                             max_len=max_len)
                                o2 = torch.empty((B, H, D), dtype=torch.float32, device="cuda")
                                ctx.append_decode(dev(q), dev(kn), dev(vn), kcd.clone(), vcd.clone(),
                                                  pos, o2, B, max_len)
                                outs.append((o1, host(o2)))
                            assert np.all(np.isfinite(outs[0][0])) and np.all(np.isfinite(outs[0][1]))
                            key = (L, B, n, sep, max_len)
                            assert np.array_equal(outs[0][0], outs[1][0]), key
                            assert np.array_equal(outs[0][1], outs[1][1]), key
                assert ctx.device_status() == nw.NWD_OK
            want = oracle.sparse_attn_f32(f32(q[0]), f32(rows[0][0]), f32(rows[0][1]))
            assert max_abs(outs[1][0][0], want) < TOL, L


@pytest.mark.parametrize("L", [1, 2, 63, 64, 65, 127, 128, 129, 1000, 5000])
def test_split_invariance_small(L):
    say(f"split invariance L={L}")
    H, Hkv = 8, 2
    g = rng(50 + L)
    k, v = kv_rows(g, L, Hkv)
    q = normal_f16(g, (1, H, D))
    want = oracle.sparse_attn_f32(f32(q[0]), f32(k), f32(v))
    with nw.AttnContext(H, Hkv, L, o_dtype="f32") as ctx:
        kc, vc = dev(to_cache([k], Hkv, L)), dev(to_cache([v], Hkv, L))
        for n in (1, 2, 3, 7, 64, 256):
            for max_len in (0, L, max(1, L // 3)):
                for sep in (False, True):
                    ctx.set_decode_splits(n)
                    ctx.set_decode_merge(sep)
                    got = _decode(ctx, dev(q), kc, vc, pos_tensor([L - 1]), 1, torch.float32,
                                  max_len=max_len)[0]
                    assert max_abs(got, want) < TOL, (L, n, max_len, sep)


@pytest.mark.parametrize("G", [1, 4, 5, 8])
@pytest.mark.parametrize("src", ["f16", "f32"])
def test_append_decode_equals_two_launches(G, src):
    """nwd_append_decode == nwd_kv_append then nwd_decode_attn, for ragged
    batches, every split count and both source types; the cache rows it
    writes are bit-identical to kv_append's."""
    say(f"append_decode G={G} src={src}")
    Hkv, B = 2, 3
    H = G * Hkv
    past = [0, 127, 700]
    cap = 800
    g = rng(300 + G)
    rows = [kv_rows(g, p, Hkv) for p in past]
    new16 = normal_f16(g, (B, Hkv, D), scale=3.0)
    newv16 = normal_f16(g, (B, Hkv, D))
    newk = f32(new16) if src == "f32" else new16
    newv = f32(newv16) if src == "f32" else newv16
    if src == "f32":  # values that do not fit fp16 exactly: rounding must match
        newk = newk + np.float32(1e-4) * g.standard_normal(newk.shape).astype(np.float32)
    q = normal_f16(g, (B, H, D))
    with nw.AttnContext(H, Hkv, cap, max_batch=B, kv_dtype=src, o_dtype="f32") as ctx:
        base_k = to_cache([r[0] for r in rows], Hkv, cap)
        base_v = to_cache([r[1] for r in rows], Hkv, cap)
        pos = pos_tensor(past)
        kc1, vc1 = dev(base_k), dev(base_v)
        ctx.kv_append(dev(newk[:, None]), dev(newv[:, None]), kc1, vc1, pos, B, 1)
        want = _decode(ctx, dev(q), kc1, vc1, pos, B, torch.float32, max_len=cap)
        for n in (0, 1, 3, 256):
            ctx.set_decode_splits(n)
            kc2, vc2 = dev(base_k), dev(base_v)
            out = torch.empty((B, H, D), dtype=torch.float32, device="cuda")
            ctx.append_decode(dev(q), dev(newk), dev(newv), kc2, vc2, pos, out, B, max_len=cap)
            got = host(out)
            assert np.array_equal(host(kc2).view(np.uint16), host(kc1).view(np.uint16)), n
            assert np.array_equal(host(vc2).view(np.uint16), host(vc1).view(np.uint16)), n
            assert max_abs(got, want) < 1e-5, n
        assert ctx.device_status() == nw.NWD_OK
    for b in range(B):
        kk = f32(from_cache(host(kc1), b, past[b] + 1))
        vv = f32(from_cache(host(vc1), b, past[b] + 1))
        assert max_abs(want[b], oracle.sparse_attn_f32(f32(q[b]), kk, vv)) < TOL


@pytest.mark.parametrize("G", [2, 4, 5, 8])
def test_one_workgroup_per_query_head_same_bits(G):
    """A single-split decode of few sequences (batch x heads <= 256) runs one
    workgroup per query head; more sequences run one per KV head. Each
    sequence of a batch too large for the first form, run alone, must give
    the same bits (output and fused-append cache rows), and the oracle's
    result."""
    say(f"per-query-head form G={G}")
    Hkv, L = 8, 200
    H = G * Hkv
    B = 256 // H + 1
    g = rng(350 + G)
    rows = [kv_rows(g, L - 1, Hkv) for _ in range(B)]
    newk = normal_f16(g, (B, Hkv, D))
    newv = normal_f16(g, (B, Hkv, D))
    q = normal_f16(g, (B, H, D))
    with nw.AttnContext(H, Hkv, L, max_batch=B) as ctx:
        # both workgroup forms of the dot-product kernel (at G = 8 the batch
        # would otherwise take the matrix-core kernel)
        ctx.set_decode_kernel(0)
        base_k = to_cache([r[0] for r in rows], Hkv, L)
        base_v = to_cache([r[1] for r in rows], Hkv, L)
        assert ctx.decode_splits(B, L) == 1 and ctx.decode_splits(1, L) == 1
        kc, vc = dev(base_k), dev(base_v)
        out = torch.empty((B, H, D), dtype=torch.float16, device="cuda")
        ctx.append_decode(dev(q), dev(newk), dev(newv), kc, vc, pos_tensor([L - 1] * B), out, B)
        kc1, vc1 = dev(base_k), dev(base_v)
        for b in range(B):  # the same sequences one at a time
            o1 = torch.empty((1, H, D), dtype=torch.float16, device="cuda")
            ctx.append_decode(dev(q[b:b + 1]), dev(newk[b:b + 1]), dev(newv[b:b + 1]), kc1[b:b + 1],
                              vc1[b:b + 1], pos_tensor([L - 1]), o1, 1)
            assert torch.equal(o1[0], out[b]), b
        assert torch.equal(kc1, kc) and torch.equal(vc1, vc)
        assert ctx.device_status() == nw.NWD_OK
        got = out.float().cpu().numpy()
    for b in range(B):
        kk = f32(from_cache(host(kc), b, L))
        vv = f32(from_cache(host(vc), b, L))
        assert max_abs(got[b], oracle.sparse_attn_f32(f32(q[b]), kk, vv)) < TOL, b


@pytest.mark.parametrize("G,B,L", [(5, 3, 500), (4, 1, 1500), (8, 2, 450)])
def test_per_query_head_form_with_splits(G, B, L):
    """Few sequences run one workgroup per query head and split, with
    256 / (batch x heads) splits while they hold at most 256 keys each; both
    merge forms give the same bits, and the oracle's result."""
    say(f"per-query-head form with splits G={G} B={B} L={L}")
    Hkv = 8
    H = G * Hkv
    g = rng(400 + G)
    rows = [kv_rows(g, L - 29 * b, Hkv) for b in range(B)]
    q = normal_f16(g, (B, H, D))
    with nw.AttnContext(H, Hkv, L, max_batch=B, o_dtype="f32") as ctx:
        n = ctx.decode_splits(B, L)
        assert n == 256 // (B * H) and n > 1, n
        kc = dev(to_cache([r[0] for r in rows], Hkv, L))
        vc = dev(to_cache([r[1] for r in rows], Hkv, L))
        pos = pos_tensor([L - 1 - 29 * b for b in range(B)])
        outs = []
        for sep in (True, False):
            ctx.set_decode_merge(sep)
            outs.append(_decode(ctx, dev(q), kc, vc, pos, B, torch.float32))
        assert ctx.device_status() == nw.NWD_OK
    assert np.array_equal(outs[0], outs[1])
    for b in range(B):
        want = oracle.sparse_attn_f32(f32(q[b]), f32(rows[b][0]), f32(rows[b][1]))
        assert max_abs(outs[0][b], want) < TOL, b


def test_fused_merge_repeated_calls_and_batches():
    """Many back-to-back calls with changing inputs, batch sizes and split
    counts: the in-kernel merge (arrival tickets) must give the separate-kernel
    result every time."""
    say("fused merge repeated")
    H, Hkv, cap, B = 32, 8, 3000, 4
    g = rng(77)
    with nw.AttnContext(H, Hkv, cap, max_batch=B, o_dtype="f32") as ctx:
        kc = randn_f16((B, Hkv, cap, D), 70)
        vc = randn_f16((B, Hkv, cap, D), 71)
        for it in range(12):
            b = 1 + it % B
            q = randn_f16((b, H, D), 100 + it)
            pos = pos_tensor(g.integers(0, cap, size=b).tolist())
            ctx.set_decode_splits([0, 3, 16, 64][it % 4])
            outs = []
            for sep in (True, False):
                ctx.set_decode_merge(sep)
                o = torch.empty((b, H, D), dtype=torch.float32, device="cuda")
                ctx.decode(q, kc, vc, pos, o, b, cap)
                outs.append(host(o))
            assert np.array_equal(outs[0], outs[1]), it
        assert ctx.device_status() == nw.NWD_OK


def test_append_decode_bad_position_writes_nothing():
    say("append_decode bad position")
    H, Hkv, cap = 8, 2, 64
    with nw.AttnContext(H, Hkv, cap, o_dtype="f32") as ctx:
        kc = torch.zeros((1, Hkv, cap, D), dtype=torch.float16, device="cuda")
        vc = torch.zeros_like(kc)
        rows = torch.ones((1, Hkv, D), dtype=torch.float16, device="cuda")
        q = torch.ones((1, H, D), dtype=torch.float16, device="cuda")
        out = torch.empty((1, H, D), dtype=torch.float32, device="cuda")
        ctx.append_decode(q, rows, rows, kc, vc, pos_tensor([cap]), out, 1)
        assert ctx.device_status() == nw.NWD_ERR_DEVICE
        assert float(kc.abs().sum()) == 0.0 and float(vc.abs().sum()) == 0.0
        assert bool(torch.isfinite(out).all())


@pytest.mark.parametrize("G", [1, 2, 4, 5, 8])
@pytest.mark.parametrize("io", ["f16", "f32"])
def test_group_sizes_and_dtypes(G, io):
    say(f"group G={G} io={io}")
    Hkv, L, B = 2, 333, 2
    H = G * Hkv
    g = rng(60 + G)
    rows = [kv_rows(g, L - 17 * b, Hkv) for b in range(B)]
    q16 = normal_f16(g, (B, H, D))
    q = f32(q16) if io == "f32" else q16
    with nw.AttnContext(H, Hkv, L, max_batch=B, q_dtype=io, o_dtype=io) as ctx:
        kc = dev(to_cache([r[0] for r in rows], Hkv, L))
        vc = dev(to_cache([r[1] for r in rows], Hkv, L))
        got = _decode(ctx, dev(q), kc, vc, pos_tensor([L - 1 - 17 * b for b in range(B)]), B,
                      torch.float32 if io == "f32" else torch.float16)
    for b in range(B):
        want = oracle.sparse_attn_f32(f32(q16[b]), f32(rows[b][0]), f32(rows[b][1]))
        assert max_abs(got[b], want) < TOL, b


def test_scale_override():
    say("scale override")
    H, Hkv, L = 8, 2, 200
    g = rng(70)
    k, v = kv_rows(g, L, Hkv)
    q = normal_f16(g, (1, H, D))
    with nw.AttnContext(H, Hkv, L, o_dtype="f32", scale=0.05) as ctx:
        got = _decode(ctx, dev(q), dev(to_cache([k], Hkv, L)), dev(to_cache([v], Hkv, L)),
                      pos_tensor([L - 1]), 1, torch.float32)[0]
    assert max_abs(got, oracle.attn_f64(f32(q[0]), f32(k), f32(v), scale=0.05)) < TOL


def test_gqa_equal_queries_equal_outputs():
    say("gqa equal queries")
    H, Hkv, L = 32, 8, 500
    g = rng(71)
    k, v = kv_rows(g, L, Hkv)
    q = normal_f16(g, (1, H, D))
    q[0, 1:4] = q[0, 0]
    with nw.AttnContext(H, Hkv, L, o_dtype="f32") as ctx:
        got = _decode(ctx, dev(q), dev(to_cache([k], Hkv, L)), dev(to_cache([v], Hkv, L)),
                      pos_tensor([L - 1]), 1, torch.float32)[0]
    assert np.array_equal(got[0], got[1]) and np.array_equal(got[0], got[3])


def test_position_past_capacity_is_flagged():
    say("decode bad positions")
    H, Hkv, cap = 8, 2, 100
    g = rng(72)
    k, v = kv_rows(g, cap, Hkv)
    q = normal_f16(g, (2, H, D))
    with nw.AttnContext(H, Hkv, cap, max_batch=2, o_dtype="f32") as ctx:
        kc, vc = dev(to_cache([k, k], Hkv, cap)), dev(to_cache([v, v], Hkv, cap))
        got = _decode(ctx, dev(q), kc, vc, pos_tensor([cap, -3]), 2, torch.float32)
        assert ctx.device_status() == nw.NWD_ERR_DEVICE
        assert np.all(np.isfinite(got))
        # clamped to the capacity / to one key, as documented
        assert max_abs(got[0], oracle.sparse_attn_f32(f32(q[0]), f32(k), f32(v))) < TOL
        assert max_abs(got[1], oracle.sparse_attn_f32(f32(q[1]), f32(k[:1]), f32(v[:1]))) < TOL


def test_host_validation_rejects_before_launch():
    say("host validation")
    with nw.AttnContext(8, 2, 64, max_batch=2) as ctx:
        t = torch.zeros(1 << 16, dtype=torch.float16, device="cuda")
        p = pos_tensor([0, 0])
        with pytest.raises(nw.NwdError) as e:
            ctx.decode(t, t, t, p, t, 3)
        assert e.value.code == nw.NWD_ERR_CAPACITY
        with pytest.raises(nw.NwdError) as e:
            ctx.decode(t, t, t, p, t, 1, max_len=65)
        assert e.value.code == nw.NWD_ERR_CAPACITY
        with pytest.raises(nw.NwdError) as e:
            ctx.kv_append(t, t, t, t, p, 1, 65)
        assert e.value.code == nw.NWD_ERR_CAPACITY
        with pytest.raises(nw.NwdError) as e:
            ctx.decode(t, 0, t, p, t, 1)
        assert e.value.code == nw.NWD_ERR_INVALID


@pytest.mark.parametrize("merge_separate", [True, False])
def test_max_seq_last_position_fused_append(merge_separate):
    """The largest supported capacity, max_seq = 2^22, one KV head (a 1 GiB
    slab per cache): append a dominant key at position 2^22 - 1 and attend
    over all 2^22 keys. Every other key is zero (score 0) with V = 0.25, so
    the output is the appended V row up to a weight of 2^22 * exp(-40); the
    appended rows must land bit-exactly at the end of the slab. The automatic
    split count is at its maximum here, so the merge takes several passes."""
    say(f"max_seq 2^22: fused append + decode at the last position, separate merge={merge_separate}")
    cap = 1 << 22
    H, Hkv = 4, 1
    g = rng(4242)
    u = g.standard_normal(D)
    u /= np.linalg.norm(u)
    q = np.tile(u, (1, H, 1)).astype(np.float32)
    k_new = (40.0 * np.sqrt(D) * u).astype(np.float16)[None, None, :]     # score ~ 40 per query
    v_new = g.standard_normal((1, 1, D)).astype(np.float16)
    with nw.AttnContext(H, Hkv, cap, q_dtype="f32", o_dtype="f32") as ctx:
        ctx.set_decode_merge(merge_separate)
        kc = torch.zeros((1, Hkv, cap, D), dtype=torch.float16, device="cuda")
        vc = torch.full((1, Hkv, cap, D), 0.25, dtype=torch.float16, device="cuda")
        out = torch.empty((1, H, D), dtype=torch.float32, device="cuda")
        ctx.append_decode(dev(q), dev(k_new), dev(v_new), kc, vc, pos_tensor([cap - 1]), out, 1)
        assert ctx.device_status() == nw.NWD_OK
        o = host(out)
        np.testing.assert_array_equal(host(kc[0, 0, cap - 1]).view(np.uint16),
                                      k_new[0, 0].view(np.uint16))
        np.testing.assert_array_equal(host(vc[0, 0, cap - 1]).view(np.uint16),
                                      v_new[0, 0].view(np.uint16))
        assert host(kc[0, 0, cap - 2]).max() == 0 and host(vc[0, 0, cap - 2]).min() == np.float16(0.25)
    want = v_new[0, 0].astype(np.float32)
    for h in range(H):
        assert max_abs(o[0, h], want) < 1e-4, h


def test_split_count_keeps_small_batches_in_one_wave():
    """Past 2048 keys a launch of batch x 8 KV heads x splits workgroups
    stays within one wave of 256 while the sequences alone fill at most half
    of it (a partial second wave cost 37% at 64K keys), three quarters of it
    for one sequence with groups of 4+ query heads while the splits then hold
    1024-3072 keys; larger
    batches split by length (at most 2048 keys per split)."""
    cases = [  # (batch, max_len, expected splits)
        (1, 65600, 24), (1, 32832, 24), (1, 73728, 24), (1, 73729, 32), (1, 98305, 32),
        (1, 131136, 32), (1, 24576, 24), (1, 24575, 32), (2, 32832, 16), (3, 32832, 10),
        (4, 32832, 8),
        (16, 65600, 2), (20, 32832, 17), (64, 16448, 9), (1, 4160, 32),
    ]
    with nw.AttnContext(32, 8, 131136, max_batch=64) as ctx:
        for B, L, n in cases:
            assert ctx.decode_splits(B, L) == n, (B, L, ctx.decode_splits(B, L))
    # three quarters only for groups of 4+ query heads
    for heads, n in ((8, 32), (16, 32), (40, 24), (64, 24)):
        with nw.AttnContext(heads, 8, 32832) as ctx:
            assert ctx.decode_splits(1, 32832) == n, (heads, ctx.decode_splits(1, 32832))


@pytest.mark.parametrize("B,P,splits", [(1, 98304, 32), (1, 40000, 24), (2, 40000, 16)])
def test_long_context_default_launch(B, P, splits):
    """Long contexts on the launch's own choices: one wave of splits (32 at
    B = 1 past 72K keys, 16 at B = 2; three quarters of it, 24, for one
    sequence of 40K) on the matrix-core split kernel (G = 4, splits of 512+
    keys), fused append, against the oracle per sequence."""
    H, Hkv = 32, 8
    cap = P + 1
    say(f"long context B={B} past={P} splits={splits}")
    g = rng(7 + B)
    rows = [kv_rows(g, P + 1, Hkv, outlier_frac=0.01) for _ in range(B)]
    q = normal_f16(g, (B, H, D))
    with nw.AttnContext(H, Hkv, cap, max_batch=B) as ctx:
        assert ctx.decode_splits(B, cap) == splits
        kc = dev(to_cache([r[0][:P] for r in rows], Hkv, cap))
        vc = dev(to_cache([r[1][:P] for r in rows], Hkv, cap))
        kn = dev(np.stack([r[0][P] for r in rows]))
        vn = dev(np.stack([r[1][P] for r in rows]))
        out = torch.empty((B, H, D), dtype=torch.float16, device="cuda")
        ctx.append_decode(dev(q), kn, vn, kc, vc, pos_tensor([P] * B), out, B)
        assert ctx.device_status() == nw.NWD_OK
        got = out.float().cpu().numpy()
        # the default launch is the matrix-core kernel's, bit for bit
        ctx.set_decode_kernel(1)
        forced = torch.empty_like(out)
        ctx.decode(dev(q), kc, vc, pos_tensor([P] * B), forced, B)
        assert torch.equal(forced, out)
    for b in range(B):
        want = oracle.sparse_attn_f32(f32(q[b]), f32(rows[b][0]), f32(rows[b][1]), threads=0)
        assert max_abs(got[b], want) < TOL, b
