"""Parity of the general-shape path (csrc/nwd_general.hip and the append at
any head size) with the oracle, through the C ABI.

The reference's attention takes head_dim and both head counts as parameters
(kernels/sparse_attn.wgsl:12-17, :38-43), and kv_append its row width
(kernels/kv_append.wgsl:1-6, n = n_kv * hd). Shapes outside the specialised
kernels' set (head_dim 128 with a group up to 8, and the head sizes and
groups below) run the general kernels; these tests cover head sizes that
are and are not multiples of 8, above 256 (two runs per thread), down to 1,
and groups 3, 6, 7 and 12 (groups 3, 6 and 7 are built at head_dim 128 and
64, csrc/nwd_decode_groups.hip, and padded to 4 / 8 at the other multiples
of 8: test_group_3_6_7_*).
Decode at head sizes 64 (groups 1, 2, 4, 5, 8) and 256 (groups 1, 2, 4, 5)
runs the dot-product split kernel built for those sizes (csrc/nwd_decode_hd.hip),
and at the other multiples of 8 up to 256 its padded form;
test_head_size_split_decode covers its launch forms and knobs. Prefill at
head sizes below 128 that are multiples of 8 runs the MFMA prefill kernel on
rows padded to 128 dims (test_padded_head_prefill).

Bars, as for the specialised path: the append bit-exact (fp16 rows copied,
fp32 rows rounded to nearest even); attention max-abs <= 2e-3 against the
oracle's op-for-op f32 restatement of sparse_attn.wgsl (fp16 inputs widened
exactly); the chunked prefill equal, row by row, to that restatement over
keys 0..pos0+i (the reference's token-by-token prefill, runtime.js:640-643).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import nwd_attn as nw  # noqa: E402
import oracle  # noqa: E402
from attn_cases import f32, from_cache, max_abs, rng, to_cache  # noqa: E402
from gpu_util import dev, host, pos_tensor, say  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 2e-3

# (head_dim, n_heads, n_kv_heads) and the route each takes
SHAPES = [
    (64, 8, 2),     # G 4: the split kernel built for head size 64
    (96, 6, 2),     # G 3 padded to 4, on the head-128 split kernel's padded form
    (80, 12, 1),    # G 12 padded to 16 (two groups of 8), padded head form
    (100, 3, 3),    # the general kernels, single-value runs (100 % 8 != 0)
    (256, 4, 1),    # G 4: the split kernel built for head size 256
    (256, 8, 1),    # G 8 at 256 (not built there): two groups of 4 per KV head
    (320, 2, 2),    # the general kernels, 40 runs: 6 key groups, 16 threads idle in P.V
    (300, 2, 1),    # the general kernels, single values, 300 > 256 threads: two runs per thread
    (512, 2, 1),    # the general kernels at the largest head size
    (128, 6, 2),    # D 128 with group 3, built for it
    (128, 7, 1),    # D 128 with group 7, built for it
    (1, 4, 2),      # the general kernels, one dim
]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    nw.load_library()


def _rows(g, L, n_kv, D, scale=1.0):
    k = (g.standard_normal((L, n_kv, D), dtype=np.float32) * np.float32(scale)).astype(np.float16)
    v = g.standard_normal((L, n_kv, D), dtype=np.float32).astype(np.float16)
    return k, v


def _tdtype(name):
    return torch.float16 if name == "f16" else torch.float32


def _q(g, shape, dtype):
    x = g.standard_normal(shape, dtype=np.float32)
    return x.astype(np.float16) if dtype == "f16" else x


@pytest.mark.parametrize("D,H,Hkv", SHAPES)
def test_general_decode_matches_oracle(D, H, Hkv):
    """Two sequences of different lengths (1..3 tiles per split and beyond),
    f16 and f32 queries/outputs, against the oracle per sequence."""
    for qd, od, lens in (("f16", "f16", [700, 65]), ("f32", "f32", [1, 3000])):
        say(f"general decode D={D} H={H} Hkv={Hkv} q={qd} o={od} L={lens}")
        g = rng(700 + D + H)
        cap = max(lens) + 7
        rows = [_rows(g, L, Hkv, D) for L in lens]
        q = _q(g, (len(lens), H, D), qd)
        with nw.AttnContext(H, Hkv, cap, head_dim=D, max_batch=len(lens), q_dtype=qd,
                            o_dtype=od) as ctx:
            kc = dev(to_cache([r[0] for r in rows], Hkv, cap))
            vc = dev(to_cache([r[1] for r in rows], Hkv, cap))
            out = torch.empty((len(lens), H, D), dtype=_tdtype(od), device="cuda")
            ctx.decode(dev(q), kc, vc, pos_tensor([L - 1 for L in lens]), out, len(lens), max(lens))
            torch.cuda.synchronize()
            assert ctx.device_status() == nw.NWD_OK
            say(f"  splits {ctx.decode_splits(len(lens), max(lens))}")
            got = host(out).astype(np.float32)
        for b, (k, v) in enumerate(rows):
            want = oracle.sparse_attn_f32(q[b].astype(np.float32), f32(k), f32(v))
            err = max_abs(got[b], want)
            assert err < TOL, (b, err)


@pytest.mark.parametrize("D,H,Hkv", [(64, 8, 8), (64, 16, 8), (64, 32, 8), (64, 40, 8),
                                     (64, 64, 8), (256, 8, 8), (256, 16, 8), (256, 32, 8),
                                     (256, 20, 4),
                                     # the padded form at other multiples of 8
                                     (96, 32, 32), (96, 32, 8), (80, 16, 8), (40, 64, 8),
                                     (192, 16, 8), (136, 40, 8), (120, 64, 8), (248, 8, 8)])
@pytest.mark.parametrize("io", ["f16", "f32"])
def test_head_size_split_decode(D, H, Hkv, io):
    """Head sizes 64 and 256 on the dot-product split kernel built for them,
    other multiples of 8 on its padded form (rows of 40 dims on the head-64
    kernel, 80-120 on the head-128 one, 136-248 on the head-256 one): a batch of one
    at 3000 keys (one workgroup per query head when batch x heads x splits
    fits 256 workgroups, else one per KV head) and a ragged batch of three,
    against the oracle; forced split counts 1, 7 and 64, the in-kernel merge
    and both key layouts (and at head size 64 the matrix-core kernel) within
    fp32 rounding of the default; the fused append bit-identical to append +
    decode in the caches."""
    g = rng(820 + D + H)
    lens = [3000, 40, 1333]
    cap = max(lens) + 2
    rows = [_rows(g, L, Hkv, D) for L in lens]
    q = _q(g, (3, H, D), io)
    kn = g.standard_normal((3, Hkv, D), dtype=np.float32).astype(np.float16)
    vn = g.standard_normal((3, Hkv, D), dtype=np.float32).astype(np.float16)
    rt = 2e-3 if io == "f16" else 2e-5
    with nw.AttnContext(H, Hkv, cap, head_dim=D, max_batch=3, q_dtype=io, o_dtype=io) as ctx:
        kc = dev(to_cache([r[0] for r in rows], Hkv, cap))
        vc = dev(to_cache([r[1] for r in rows], Hkv, cap))
        for batch in (1, 3):
            say(f"head size {D} {H}q/{Hkv}kv io={io} batch={batch} "
                f"splits {ctx.decode_splits(batch, max(lens[:batch]))}")
            pos = pos_tensor([L - 1 for L in lens[:batch]])
            outs = []
            runs = [(0, None, None, None), (1, None, None, None), (7, None, None, None),
                    (64, None, None, None), (0, 0, None, None), (7, 0, None, None),
                    (7, None, 1, None), (7, None, 0, None)]
            if D == 64:  # the matrix-core kernel built for head size 64
                runs += [(0, None, None, 1), (7, None, None, 1), (7, 0, None, 1), (64, None, 1, 1)]
            for n, merge, layout, kern in runs:
                ctx.set_decode_splits(n)
                ctx.set_decode_merge(merge)
                ctx.set_decode_layout(layout)
                ctx.set_decode_kernel(kern)
                out = torch.empty((batch, H, D), dtype=_tdtype(io), device="cuda")
                ctx.decode(dev(q[:batch]), kc, vc, pos, out, batch, max(lens[:batch]))
                outs.append(host(out).astype(np.float32))
            assert ctx.device_status() == nw.NWD_OK
            for b in range(batch):
                k, v = rows[b]
                want = oracle.sparse_attn_f32(q[b].astype(np.float32), f32(k), f32(v))
                assert max_abs(outs[0][b], want) < TOL, (batch, b)
            for i, o in enumerate(outs[1:]):
                assert max_abs(o, outs[0]) < rt, (batch, i)
        ctx.set_decode_splits(0)
        ctx.set_decode_merge(None)
        ctx.set_decode_layout(None)
        ctx.set_decode_kernel(None)
        res = []
        for fused in (True, False):
            kc2, vc2 = kc.clone(), vc.clone()
            out = torch.empty((3, H, D), dtype=_tdtype(io), device="cuda")
            p2 = pos_tensor(lens)
            if fused:
                ctx.append_decode(dev(q), dev(kn), dev(vn), kc2, vc2, p2, out, 3, cap)
            else:
                ctx.kv_append(dev(kn[:, None]), dev(vn[:, None]), kc2, vc2, p2, 3, 1)
                ctx.decode(dev(q), kc2, vc2, p2, out, 3, cap)
            assert ctx.device_status() == nw.NWD_OK
            res.append((host(out).astype(np.float32), host(kc2).view(np.uint16),
                        host(vc2).view(np.uint16)))
        assert np.array_equal(res[0][1], res[1][1]) and np.array_equal(res[0][2], res[1][2])
        assert max_abs(res[0][0], res[1][0]) < rt
        for b, L in enumerate(lens):
            k_all = np.concatenate([rows[b][0], kn[b][None]], axis=0)
            v_all = np.concatenate([rows[b][1], vn[b][None]], axis=0)
            want = oracle.sparse_attn_f32(q[b].astype(np.float32), f32(k_all), f32(v_all))
            assert max_abs(res[0][0][b], want) < TOL, b


@pytest.mark.parametrize("D,H,Hkv", [(128, 128, 8), (128, 96, 8), (64, 48, 1), (128, 71, 1),
                                     (96, 20, 2), (256, 16, 2), (192, 14, 2), (128, 9, 1)])
@pytest.mark.parametrize("io", ["f16", "f32"])
def test_large_group_decode_and_prefill(D, H, Hkv, io):
    """Groups the kernels are not built for run as several built groups per
    KV head (16 = 2 x 8, 48 = 6 x 8, 10 = 2 x 5, 8 at head size 256 =
    2 x 4) or padded to such groups (12 -> 16 = 2 x 8, 71 -> 72 = 9 x 8,
    9 -> 16, 7 at 192 -> 8 = 2 x 4): decode of a ragged pair (2000 and 37 keys) and
    forced split counts against the oracle, the fused append bit-identical
    to append + decode in the caches, and a prefill chunk row by row."""
    say(f"large group D={D} {H}q/{Hkv}kv io={io}")
    g = rng(900 + D + H)
    lens = [2000, 37]
    cap = 2050
    rows = [_rows(g, L, Hkv, D, scale=0.5) for L in lens]
    q = _q(g, (2, H, D), io)
    kn = g.standard_normal((2, Hkv, D), dtype=np.float32).astype(np.float16)
    vn = g.standard_normal((2, Hkv, D), dtype=np.float32).astype(np.float16)
    rt = 2e-3 if io == "f16" else 2e-5
    with nw.AttnContext(H, Hkv, cap, head_dim=D, max_batch=2, q_dtype=io, o_dtype=io) as ctx:
        kc = dev(to_cache([r[0] for r in rows], Hkv, cap))
        vc = dev(to_cache([r[1] for r in rows], Hkv, cap))
        pos = pos_tensor([L - 1 for L in lens])
        outs = []
        for n in (0, 1, 9):
            ctx.set_decode_splits(n)
            out = torch.empty((2, H, D), dtype=_tdtype(io), device="cuda")
            ctx.decode(dev(q), kc, vc, pos, out, 2, max(lens))
            outs.append(host(out).astype(np.float32))
        ctx.set_decode_splits(0)
        assert ctx.device_status() == nw.NWD_OK
        for b, (k, v) in enumerate(rows):
            want = oracle.sparse_attn_f32(q[b].astype(np.float32), f32(k), f32(v))
            assert max_abs(outs[0][b], want) < TOL, b
        for o in outs[1:]:
            assert max_abs(o, outs[0]) < rt
        res = []
        for fused in (True, False):
            kc2, vc2 = kc.clone(), vc.clone()
            out = torch.empty((2, H, D), dtype=_tdtype(io), device="cuda")
            p2 = pos_tensor(lens)
            if fused:
                ctx.append_decode(dev(q), dev(kn), dev(vn), kc2, vc2, p2, out, 2, cap)
            else:
                ctx.kv_append(dev(kn[:, None]), dev(vn[:, None]), kc2, vc2, p2, 2, 1)
                ctx.decode(dev(q), kc2, vc2, p2, out, 2, cap)
            assert ctx.device_status() == nw.NWD_OK
            res.append((host(out).astype(np.float32), host(kc2).view(np.uint16),
                        host(vc2).view(np.uint16)))
        assert np.array_equal(res[0][1], res[1][1]) and np.array_equal(res[0][2], res[1][2])
        assert max_abs(res[0][0], res[1][0]) < rt
        if D <= 256:
            n_new, p0 = 21, [1500, 2]
            qp = _q(g, (2, n_new, H, D), io)
            out = torch.empty((2, n_new, H, D), dtype=_tdtype(io), device="cuda")
            ctx.prefill(dev(qp), kc, vc, pos_tensor(p0), out, 2, n_new, max(p0) + n_new)
            assert ctx.device_status() == nw.NWD_OK
            got = host(out).astype(np.float32)
            kh, vh = host(kc), host(vc)
            worst = 0.0
            for b in range(2):
                for i in range(n_new):
                    L = p0[b] + i + 1
                    want = oracle.sparse_attn_f32(qp[b, i].astype(np.float32),
                                                  f32(from_cache(kh, b, L)), f32(from_cache(vh, b, L)))
                    worst = max(worst, max_abs(got[b, i], want))
            say(f"  prefill max-abs {worst:.2e}")
            assert worst < TOL


@pytest.mark.parametrize("D,H,Hkv", [(96, 6, 2), (100, 3, 3), (300, 2, 1)])
def test_general_split_count_does_not_change_results(D, H, Hkv):
    """Forced split counts 1, 3, 17 and 64 (the last leaves splits with no
    keys, whose records weigh nothing in the merge) agree within fp32
    rounding and with the oracle."""
    g = rng(710 + D)
    L, cap = 1500, 1600
    k, v = _rows(g, L, Hkv, D)
    q = _q(g, (1, H, D), "f32")
    outs = []
    with nw.AttnContext(H, Hkv, cap, head_dim=D, q_dtype="f32", o_dtype="f32") as ctx:
        kc, vc = dev(to_cache([k], Hkv, cap)), dev(to_cache([v], Hkv, cap))
        for n in (1, 3, 17, 64):
            ctx.set_decode_splits(n)
            assert ctx.decode_splits(1, L) == n
            out = torch.empty((1, H, D), device="cuda")
            ctx.decode(dev(q), kc, vc, pos_tensor([L - 1]), out, 1, 256)  # bound below L: the last split runs on
            outs.append(host(out)[0])
        assert ctx.device_status() == nw.NWD_OK
    want = oracle.sparse_attn_f32(q[0], f32(k), f32(v))
    for n, o in zip((1, 3, 17, 64), outs):
        assert max_abs(o, outs[0]) < 1e-5, n
        assert max_abs(o, want) < TOL, n


@pytest.mark.parametrize("D", [64, 100, 3, 512])
@pytest.mark.parametrize("kv", ["f16", "f32"])
def test_general_append_bit_exact(D, kv):
    """Rows of any width land bit for bit (fp16) or rounded to nearest even
    (fp32) at pos[b] + j, canaries untouched, for 2 sequences x 3 tokens."""
    say(f"general append D={D} kv={kv}")
    B, n_tok, n_kv, cap = 2, 3, 3, 16
    g = rng(720 + D)
    if kv == "f16":
        src = g.integers(0, 65536, size=(2, B, n_tok, n_kv, D), dtype=np.uint32).astype(np.uint16)
        want_rows = src
        tsrc = [dev(src[i].view(np.int16)) for i in range(2)]
    else:
        x = (g.standard_normal((2, B, n_tok, n_kv, D)) * np.exp2(g.uniform(-20, 15, (2, B, n_tok, n_kv, D)))
             ).astype(np.float32)
        want_rows = np.stack([oracle.f32_to_f16(x[i].reshape(-1, D)).reshape(B, n_tok, n_kv, D)
                              for i in range(2)])
        tsrc = [dev(x[i]) for i in range(2)]
    canary = 0x7E5A
    pos = [2, cap - n_tok]
    with nw.AttnContext(6, n_kv, cap, head_dim=D, max_batch=B, kv_dtype=kv) as ctx:
        caches = [torch.full((B, n_kv, cap, D), canary, dtype=torch.int16, device="cuda") for _ in range(2)]
        ctx.kv_append(tsrc[0], tsrc[1], caches[0], caches[1], pos_tensor(pos), B, n_tok)
        assert ctx.device_status() == nw.NWD_OK
        assert ctx.cache_offset(1, 5, 2, D - 1) == ((1 * n_kv + 2) * cap + 5) * D + D - 1
        for which in range(2):
            want = np.full((B, n_kv, cap, D), canary, np.uint16)
            for b in range(B):
                for j in range(n_tok):
                    want[b, :, pos[b] + j, :] = want_rows[which, b, j]
            assert np.array_equal(host(caches[which]).view(np.uint16), want)


@pytest.mark.parametrize("D,H,Hkv", [(64, 8, 2), (100, 3, 3), (128, 6, 2)])
def test_general_append_decode_matches_two_calls(D, H, Hkv):
    """nwd_append_decode on a general shape gives the bits of nwd_kv_append
    followed by nwd_decode_attn, caches included."""
    g = rng(730 + D)
    B, cap = 2, 512
    past = [300, 17]
    rows = [_rows(g, p + 1, Hkv, D) for p in past]
    q = _q(g, (B, H, D), "f16")
    new_k = np.stack([r[0][p] for r, p in zip(rows, past)])[:, None]
    new_v = np.stack([r[1][p] for r, p in zip(rows, past)])[:, None]
    res = []
    with nw.AttnContext(H, Hkv, cap, head_dim=D, max_batch=B) as ctx:
        for fused in (True, False):
            kc = dev(to_cache([r[0][:p] for r, p in zip(rows, past)], Hkv, cap))
            vc = dev(to_cache([r[1][:p] for r, p in zip(rows, past)], Hkv, cap))
            out = torch.empty((B, H, D), dtype=torch.float16, device="cuda")
            pos = pos_tensor(past)
            if fused:
                ctx.append_decode(dev(q), dev(new_k), dev(new_v), kc, vc, pos, out, B, max(past) + 1)
            else:
                ctx.kv_append(dev(new_k), dev(new_v), kc, vc, pos, B, 1)
                ctx.decode(dev(q), kc, vc, pos, out, B, max(past) + 1)
            assert ctx.device_status() == nw.NWD_OK
            res.append((host(out).view(np.uint16), host(kc).view(np.uint16), host(vc).view(np.uint16)))
    for a, b in zip(*res):
        assert np.array_equal(a, b)
    for b, (k, v) in enumerate(rows):
        want = oracle.sparse_attn_f32(f32(q[b]), f32(k), f32(v))
        assert max_abs(res[0][0][b].view(np.float16).astype(np.float32), want) < TOL


@pytest.mark.parametrize("D,H,Hkv", [(64, 6, 2), (100, 3, 3), (128, 12, 1)])
@pytest.mark.parametrize("splits", [0, 5])
def test_general_prefill_matches_token_by_token(D, H, Hkv, splits):
    """A chunk of 37 queries appended at pos0 (two sequences, pos0 90 and
    0): query i equals the oracle's decode over keys 0..pos0+i. With 5 forced
    splits the early rows have splits with no keys."""
    say(f"general prefill D={D} H={H} Hkv={Hkv} splits={splits}")
    g = rng(740 + D + splits)
    n_new, pos0 = 37, [90, 0]
    B, cap = 2, 140
    rows = [_rows(g, p + n_new, Hkv, D, scale=0.5) for p in pos0]
    q = _q(g, (B, n_new, H, D), "f32")
    with nw.AttnContext(H, Hkv, cap, head_dim=D, max_batch=B, q_dtype="f32", o_dtype="f32") as ctx:
        if splits:
            ctx.set_decode_splits(splits)
        kc = dev(to_cache([r[0] for r in rows], Hkv, cap))
        vc = dev(to_cache([r[1] for r in rows], Hkv, cap))
        out = torch.empty((B, n_new, H, D), device="cuda")
        ctx.prefill(dev(q), kc, vc, pos_tensor(pos0), out, B, n_new, max(pos0) + n_new)
        assert ctx.device_status() == nw.NWD_OK
        got = host(out)
    worst = 0.0
    for b, (k, v) in enumerate(rows):
        for i in range(n_new):
            L = pos0[b] + i + 1
            want = oracle.sparse_attn_f32(q[b, i], f32(k[:L]), f32(v[:L]))
            worst = max(worst, max_abs(got[b, i], want))
    say(f"  max-abs {worst:.2e}")
    assert worst < TOL


@pytest.mark.parametrize("D,H,Hkv", [(64, 32, 8), (64, 8, 8), (96, 10, 2), (32, 16, 2),
                                     (120, 4, 2), (64, 6, 2), (96, 7, 1),
                                     # the head-256 prefill, as it is and padded
                                     (256, 16, 8), (256, 8, 8), (256, 20, 4), (200, 8, 4),
                                     (136, 6, 2), (256, 14, 2)])
@pytest.mark.parametrize("io", ["f16", "f32"])
def test_padded_head_prefill(D, H, Hkv, io):
    """Head sizes below 128 (multiples of 8) prefill on the MFMA prefill
    kernel with rows padded to 128 dims, head sizes 136 to 256 on the head-256
    MFMA prefill (padded below 256); groups 3 and 7 also through padded
    query rows: two sequences, pos0 1500 (several key tiles, split over
    workgroups and merged) and 3, 40 new tokens; every row against the
    oracle's decode over keys 0..pos0+i."""
    say(f"padded-head prefill D={D} H={H} Hkv={Hkv} io={io}")
    g = rng(860 + D + H)
    n_new, pos0 = 40, [1500, 3]
    B, cap = 2, 1600
    rows = [_rows(g, p + n_new, Hkv, D, scale=0.5) for p in pos0]
    q = _q(g, (B, n_new, H, D), io)
    with nw.AttnContext(H, Hkv, cap, head_dim=D, max_batch=B, q_dtype=io, o_dtype=io) as ctx:
        kc = dev(to_cache([r[0] for r in rows], Hkv, cap))
        vc = dev(to_cache([r[1] for r in rows], Hkv, cap))
        out = torch.empty((B, n_new, H, D), dtype=_tdtype(io), device="cuda")
        ctx.prefill(dev(q), kc, vc, pos_tensor(pos0), out, B, n_new, max(pos0) + n_new)
        assert ctx.device_status() == nw.NWD_OK
        got = host(out).astype(np.float32)
    worst = 0.0
    for b, (k, v) in enumerate(rows):
        for i in range(n_new):
            L = pos0[b] + i + 1
            want = oracle.sparse_attn_f32(q[b, i].astype(np.float32), f32(k[:L]), f32(v[:L]))
            worst = max(worst, max_abs(got[b, i], want))
    say(f"  max-abs {worst:.2e}")
    assert worst < TOL


def test_general_bad_positions_flagged():
    """A decode position at the capacity and a prefill chunk that would run
    past it are flagged in the status word, as on the specialised path; the
    decode then attends the whole cache (clamped)."""
    D, H, Hkv, cap = 96, 6, 2, 40
    g = rng(750)
    k, v = _rows(g, cap, Hkv, D)
    q = _q(g, (1, H, D), "f32")
    with nw.AttnContext(H, Hkv, cap, head_dim=D, q_dtype="f32", o_dtype="f32") as ctx:
        kc, vc = dev(to_cache([k], Hkv, cap)), dev(to_cache([v], Hkv, cap))
        out = torch.empty((1, H, D), device="cuda")
        ctx.decode(dev(q), kc, vc, pos_tensor([cap]), out, 1, cap)
        assert ctx.device_status() == nw.NWD_ERR_DEVICE
        assert "position" in ctx.last_error()
        want = oracle.sparse_attn_f32(q[0], f32(k), f32(v))
        assert max_abs(host(out)[0], want) < TOL
        pout = torch.empty((1, 8, H, D), device="cuda")
        ctx.prefill(dev(_q(g, (1, 8, H, D), "f32")), kc, vc, pos_tensor([cap - 4]), pout, 1, 8, cap)
        assert ctx.device_status() == nw.NWD_ERR_DEVICE
        assert ctx.device_status() == nw.NWD_OK


def test_general_cache_rows_read_back():
    """from_cache of what the general append wrote gives the rows back (the
    layout helper and the library agree at head_dim 80)."""
    D, Hkv, cap = 80, 3, 12
    g = rng(760)
    k, v = _rows(g, 5, Hkv, D)
    with nw.AttnContext(6, Hkv, cap, head_dim=D) as ctx:
        kc = torch.zeros((1, Hkv, cap, D), dtype=torch.float16, device="cuda")
        vc = torch.zeros_like(kc)
        ctx.kv_append(dev(k[None]), dev(v[None]), kc, vc, pos_tensor([4]), 1, 5)
        assert ctx.device_status() == nw.NWD_OK
        assert np.array_equal(from_cache(host(kc), 0, 9)[4:].view(np.uint16), k.view(np.uint16))
        assert np.array_equal(from_cache(host(vc), 0, 9)[4:].view(np.uint16), v.view(np.uint16))


# ----------------------------------------------------- groups 3, 6, 7 ---

@pytest.mark.parametrize("D,H,Hkv", [(128, 12, 4), (128, 6, 1), (128, 28, 4), (128, 14, 2),
                                     (64, 28, 4), (64, 12, 4), (96, 12, 4), (80, 28, 4),
                                     (256, 12, 4), (256, 12, 2)])
@pytest.mark.parametrize("io", ["f16", "f32"])
def test_group_3_6_7_decode(D, H, Hkv, io):
    """Groups 3, 6 and 7 run decode kernels built for them at head_dim 128
    and 64 (group 3 at 256, and 6 as two groups of 3), and at other head
    sizes the kernels of groups 4 and 8 on padded query rows: against the oracle at 5000 and 1100 keys, with two key bounds
    (different split partitions) within fp32 rounding of each other, and the
    fused append bit-identical to append + decode in the caches."""
    cap = 5010
    lens = [5000, 1100]
    say(f"group 3/6/7 decode {H}q/{Hkv}kv/d{D} io={io}")
    g = rng(780 + H)
    rows = [_rows(g, L, Hkv, D) for L in lens]
    q = _q(g, (2, H, D), io)
    kn = g.standard_normal((2, Hkv, D), dtype=np.float32).astype(np.float16)
    vn = g.standard_normal((2, Hkv, D), dtype=np.float32).astype(np.float16)
    with nw.AttnContext(H, Hkv, cap, head_dim=D, max_batch=2, q_dtype=io, o_dtype=io) as ctx:
        kc = dev(to_cache([r[0] for r in rows], Hkv, cap))
        vc = dev(to_cache([r[1] for r in rows], Hkv, cap))
        pos = pos_tensor([L - 1 for L in lens])
        outs = {}
        for bound in (cap, 1000):
            out = torch.empty((2, H, D), dtype=_tdtype(io), device="cuda")
            ctx.decode(dev(q), kc, vc, pos, out, 2, bound)
            outs[bound] = host(out).astype(np.float32)
        assert ctx.device_status() == nw.NWD_OK
        for b, (k, v) in enumerate(rows):
            want = oracle.sparse_attn_f32(q[b].astype(np.float32), f32(k), f32(v))
            assert max_abs(outs[cap][b], want) < TOL, b
        assert max_abs(outs[cap], outs[1000]) < (2e-3 if io == "f16" else 2e-5)  # other splits
        # fused append + attend
        res = []
        for fused in (True, False):
            kc2, vc2 = kc.clone(), vc.clone()
            out = torch.empty((2, H, D), dtype=_tdtype(io), device="cuda")
            p2 = pos_tensor(lens)  # the new rows go at L, attended over L + 1 keys
            if fused:
                ctx.append_decode(dev(q), dev(kn), dev(vn), kc2, vc2, p2, out, 2, cap)
            else:
                ctx.kv_append(dev(kn[:, None]), dev(vn[:, None]), kc2, vc2, p2, 2, 1)
                ctx.decode(dev(q), kc2, vc2, p2, out, 2, cap)
            assert ctx.device_status() == nw.NWD_OK
            res.append((host(out), host(kc2).view(np.uint16), host(vc2).view(np.uint16)))
        assert np.array_equal(res[0][1], res[1][1]) and np.array_equal(res[0][2], res[1][2])
        assert max_abs(res[0][0].astype(np.float32), res[1][0].astype(np.float32)) < (
            1e-3 if io == "f16" else 1e-5)
        for b, L in enumerate(lens):
            k_all = np.concatenate([rows[b][0], kn[b][None]], axis=0)
            v_all = np.concatenate([rows[b][1], vn[b][None]], axis=0)
            want = oracle.sparse_attn_f32(q[b].astype(np.float32), f32(k_all), f32(v_all))
            assert max_abs(res[0][0][b].astype(np.float32), want) < TOL, b


@pytest.mark.parametrize("H,Hkv,D", [(14, 2, 128), (6, 2, 128), (14, 2, 64), (14, 2, 96)])
def test_group_3_6_7_knobs(H, Hkv, D):
    """The decode knobs apply to groups 3, 6 and 7, built (head_dim 128 and
    64) or padded (96): forced split counts and both split kernels give the
    same results within fp32 rounding."""
    L = 3000
    say(f"group 3/6/7 knobs {H}q/{Hkv}kv/d{D}")
    g = rng(790 + H + D)
    k, v = _rows(g, L, Hkv, D)
    q = _q(g, (1, H, D), "f32")
    outs = []
    with nw.AttnContext(H, Hkv, L, head_dim=D, q_dtype="f32", o_dtype="f32") as ctx:
        kc, vc = dev(to_cache([k], Hkv, L)), dev(to_cache([v], Hkv, L))
        for n, kern in ((0, None), (3, None), (40, None), (0, 0), (0, 1)):
            ctx.set_decode_splits(n)
            ctx.set_decode_kernel(kern)
            out = torch.empty((1, H, D), device="cuda")
            ctx.decode(dev(q), kc, vc, pos_tensor([L - 1]), out, 1, L)
            outs.append(host(out)[0])
        assert ctx.device_status() == nw.NWD_OK
    want = oracle.sparse_attn_f32(q[0], f32(k), f32(v))
    for o in outs:
        assert max_abs(o, want) < TOL
        assert max_abs(o, outs[0]) < 1e-5


@pytest.mark.parametrize("D,H,Hkv", [(128, 12, 4), (128, 7, 1), (128, 12, 2), (64, 7, 1),
                                     (96, 12, 4), (80, 7, 1), (256, 12, 4), (256, 12, 2)])
@pytest.mark.parametrize("max_batch", [2, 2048])
@pytest.mark.parametrize("io", ["f16", "f32"])
def test_group_3_6_7_prefill(D, H, Hkv, max_batch, io):
    """Groups 3, 6 and 7 prefill on the fp16 MFMA prefill kernel built for
    them at head_dim 128 and 64 (and group 3 at 256, 6 as two groups of 3),
    and at other head sizes on the kernels of groups 4 and 8 through padded
    query rows: 37 queries onto pos0 90 and 0, row by
    row against the oracle's decode over keys 0..pos0+i. With max_batch 2048
    the padded route's buffers hold a few tokens, so the chunk runs in
    several sub-chunks."""
    n_new, pos0, cap = 37, [90, 0], 140
    say(f"group 3/6/7 prefill {H}q/{Hkv}kv/d{D} max_batch={max_batch} io={io}")
    g = rng(800 + H)
    rows = [_rows(g, p + n_new, Hkv, D, scale=0.5) for p in pos0]
    q = _q(g, (2, n_new, H, D), io)
    with nw.AttnContext(H, Hkv, cap, head_dim=D, max_batch=max_batch, q_dtype=io,
                        o_dtype="f32") as ctx:
        kc = dev(to_cache([r[0] for r in rows], Hkv, cap))
        vc = dev(to_cache([r[1] for r in rows], Hkv, cap))
        out = torch.empty((2, n_new, H, D), device="cuda")
        ctx.prefill(dev(q), kc, vc, pos_tensor(pos0), out, 2, n_new, max(pos0) + n_new)
        assert ctx.device_status() == nw.NWD_OK
        got = host(out)
        # a chunk past the capacity is flagged once and run at the last fitting pos0
        ctx.prefill(dev(q), kc, vc, pos_tensor([cap - 10, 0]), out, 2, n_new, cap)
        assert ctx.device_status() == nw.NWD_ERR_DEVICE
        assert ctx.device_status() == nw.NWD_OK
    worst = 0.0
    for b, (k, v) in enumerate(rows):
        for i in range(n_new):
            L = pos0[b] + i + 1
            want = oracle.sparse_attn_f32(q[b, i].astype(np.float32), f32(k[:L]), f32(v[:L]))
            worst = max(worst, max_abs(got[b, i], want))
    say(f"  max-abs {worst:.2e}")
    assert worst < TOL
