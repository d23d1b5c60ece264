"""The allocation-free entry point nwd_append_decode_noalloc against the
context entry point nwd_append_decode it varies: same descriptor, same
inputs, bit-identical outputs and cache rows, on two calls in a row (the
second with a smaller input) through the C ABI; a call whose split records
exceed the static scratch is rejected before any launch; an out-of-range
position is reported through the caller's status word."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import nwd_attn as nw  # noqa: E402
import oracle  # noqa: E402
from attn_cases import f32, from_cache, kv_rows, max_abs, normal_f16, rng, to_cache  # noqa: E402
from gpu_util import dev, host, pos_tensor, say  # noqa: E402

pytestmark = pytest.mark.gpu

D = 128


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    nw.load_library()


def _case(g, H, Hkv, B, past, cap):
    rows = [kv_rows(g, p, Hkv) for p in past]
    return dict(kc=to_cache([r[0] for r in rows], Hkv, cap), vc=to_cache([r[1] for r in rows], Hkv, cap),
                q=normal_f16(g, (B, H, D)), kn=normal_f16(g, (B, Hkv, D)),
                vn=normal_f16(g, (B, Hkv, D)), pos=list(past))


def test_noalloc_matches_context_entry_point():
    H, Hkv, cap = 32, 8, 6000
    g = rng(900)
    # first call: 32 splits (records in the scratch); second, smaller: one
    # split, then a smaller batch with 8 splits of a shorter bound
    cases = [(1, [5000], 0), (1, [300], 300), (3, [1200, 17, 900], 1300)]
    with nw.AttnContext(H, Hkv, cap, max_batch=3) as ctx:
        desc = ctx.desc
        stream = torch.cuda.Stream()
        status = torch.zeros(1, dtype=torch.int32, device="cuda")
        datas = [_case(g, H, Hkv, B, past, cap) for B, past, _ in cases]
        outs, caches = [], []
        for (B, past, max_len), d in zip(cases, datas):  # calls in a row on one stream
            say(f"noalloc B={B} past={past} max_len={max_len} splits={ctx.decode_splits(B, max_len)}")
            kc, vc = dev(d["kc"]), dev(d["vc"])
            out = torch.empty((B, H, D), dtype=torch.float16, device="cuda")
            nw.append_decode_noalloc(desc, dev(d["q"]), dev(d["kn"]), dev(d["vn"]), kc, vc,
                                     pos_tensor(d["pos"]), out, B, max_len, status, stream)
            outs.append(out)
            caches.append((kc, vc))
        torch.cuda.synchronize()
        assert int(status.item()) == 0
        for (B, past, max_len), d, out, (kc, vc) in zip(cases, datas, outs, caches):
            kc1, vc1 = dev(d["kc"]), dev(d["vc"])
            want = torch.empty((B, H, D), dtype=torch.float16, device="cuda")
            ctx.append_decode(dev(d["q"]), dev(d["kn"]), dev(d["vn"]), kc1, vc1,
                              pos_tensor(d["pos"]), want, B, max_len)
            torch.cuda.synchronize()
            assert torch.equal(out, want), (B, past)
            assert torch.equal(kc, kc1) and torch.equal(vc, vc1), (B, past)
            got = host(out).astype(np.float32)
            for b in range(B):
                L = past[b] + 1
                kk = f32(from_cache(host(kc), b, L))
                vv = f32(from_cache(host(vc), b, L))
                assert max_abs(got[b], oracle.sparse_attn_f32(f32(d["q"][b]), kk, vv)) < 2e-3, b
        assert ctx.device_status() == nw.NWD_OK



@pytest.mark.parametrize("H,Hkv,Dg", [(9, 3, 100), (8, 2, 96), (16, 4, 64), (10, 2, 256),
                                      (14, 2, 128), (14, 2, 64)])
def test_noalloc_general_shape_matches_context_entry_point(H, Hkv, Dg):
    """The same at other shapes: the general kernels (head_dim 100, group
    3), the split kernel's padded form (head_dim 96), the split kernel built
    for head sizes 64 and 256, and group 7 at head_dim 128 and 64, their
    records in the scratch, two calls in a row (the second smaller),
    bit-identical to nwd_append_decode. (Groups 3, 6 and 7 that the context
    decodes as padded groups, at head sizes other than 128 and 64, take the
    general kernels here, which have no padded buffers: not the same
    bits.)"""
    cap = 4096
    g = rng(910 + Dg)
    cases = [(2, [4000, 1500], 0), (1, [200], 256)]
    with nw.AttnContext(H, Hkv, cap, head_dim=Dg, max_batch=2) as ctx:
        desc = ctx.desc
        status = torch.zeros(1, dtype=torch.int32, device="cuda")
        for B, past, max_len in cases:
            say(f"noalloc general B={B} past={past} splits={ctx.decode_splits(B, max_len)}")
            rows = [[g.standard_normal((p, Hkv, Dg), dtype=np.float32).astype(np.float16)
                     for _ in range(2)] for p in past]
            q = g.standard_normal((B, H, Dg), dtype=np.float32).astype(np.float16)
            kn, vn = (g.standard_normal((B, Hkv, Dg), dtype=np.float32).astype(np.float16)
                      for _ in range(2))
            res = []
            for noalloc in (True, False):
                kc = dev(to_cache([r[0] for r in rows], Hkv, cap))
                vc = dev(to_cache([r[1] for r in rows], Hkv, cap))
                out = torch.empty((B, H, Dg), dtype=torch.float16, device="cuda")
                if noalloc:
                    nw.append_decode_noalloc(desc, dev(q), dev(kn), dev(vn), kc, vc, pos_tensor(past),
                                             out, B, max_len, status)
                else:
                    ctx.append_decode(dev(q), dev(kn), dev(vn), kc, vc, pos_tensor(past), out, B,
                                      max_len)
                torch.cuda.synchronize()
                res.append((out, kc, vc))
            assert int(status.item()) == 0
            for a, b in zip(*res):
                assert torch.equal(a, b), (B, past)
            got = host(res[0][0]).astype(np.float32)
            for b in range(B):
                L = past[b] + 1
                kk = f32(from_cache(host(res[0][1]), b, L))
                vv = f32(from_cache(host(res[0][2]), b, L))
                assert max_abs(got[b], oracle.sparse_attn_f32(f32(q[b]), kk, vv)) < 2e-3, b
        assert ctx.device_status() == nw.NWD_OK

def test_noalloc_rejects_calls_beyond_the_scratch():
    say("noalloc capacity check")
    H, Hkv, cap, B = 32, 8, 16384, 128
    desc = nw.NwdDesc(H, Hkv, D, cap, B, nw.NWD_F16, nw.NWD_F16, nw.NWD_F16, 0.0)
    t = torch.zeros(16, dtype=torch.float16, device="cuda")
    pos = torch.zeros(B, dtype=torch.int32, device="cuda")
    # 128 sequences x 32 heads x 8 splits = 32768 records > 32262: rejected
    # on the host, nothing launched (the tiny buffers are never touched)
    with pytest.raises(nw.NwdError) as e:
        nw.append_decode_noalloc(desc, t, t, t, t, t, pos, t, B, cap)
    assert e.value.code == nw.NWD_ERR_CAPACITY
    assert "scratch" in e.value.message
    with pytest.raises(nw.NwdError) as e:
        nw.append_decode_noalloc(desc, t, t, t, t, t, pos, t, B + 1, cap)
    assert e.value.code == nw.NWD_ERR_CAPACITY


def test_noalloc_bad_position_reported_in_status():
    say("noalloc bad position")
    H, Hkv, cap = 8, 2, 64
    desc = nw.NwdDesc(H, Hkv, D, cap, 1, nw.NWD_F16, nw.NWD_F32, nw.NWD_F16, 0.0)
    kc = torch.zeros((1, Hkv, cap, D), dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    rows = torch.ones((1, Hkv, D), dtype=torch.float16, device="cuda")
    q = torch.ones((1, H, D), dtype=torch.float16, device="cuda")
    out = torch.empty((1, H, D), dtype=torch.float32, device="cuda")
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    nw.append_decode_noalloc(desc, q, rows, rows, kc, vc, pos_tensor([cap]), out, 1, 0, status)
    torch.cuda.synchronize()
    assert int(status.item()) == 1
    assert float(kc.abs().sum()) == 0.0 and float(vc.abs().sum()) == 0.0
    assert bool(torch.isfinite(out).all())
