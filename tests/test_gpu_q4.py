"""Parity of the HIP 4-bit GEMV (nwd_q4_gemv) and the fused q/k/v projection
+ kv_append (nwd_qkv_append) with the oracle's restatement of
kernels/matmul_nbits_sg.wgsl, through the C ABI.

Bars:
  * projections: |y - y64| <= 1e-6 * sum_k |w_k a_k| against the float64
    dequantise-and-multiply (the oracle meets the same bound, pinned in
    test_q4_oracle.py);
  * epilogues: relu2 and accumulate are exact functions of the plain result
    (bit-exact);
  * cache rows written by nwd_qkv_append: within one fp16 ulp of the
    float64 projection rounded to fp16, canary rows untouched;
  * qkv_append then decode: max-abs <= 2e-3 against the oracle chain
    (q4 GEMV -> fp16 cache -> sparse_attn restatement).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import nwd_attn as nw  # noqa: E402
import oracle  # noqa: E402
from attn_cases import max_abs  # noqa: E402
from gpu_util import dev, host, pos_tensor, say  # noqa: E402
from q4_cases import HIDDEN, gemv_f64, random_q4, rng  # noqa: E402

pytestmark = pytest.mark.gpu

TOL_REL = 1e-6
D = 128


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    nw.load_library()


class DevQ4:
    """One projection's weights on the device plus its host copy."""

    def __init__(self, g, n, n_blocks, scale=0.02):
        self.quant, self.scales, self.zp = random_q4(g, n, n_blocks, scale)
        self.n, self.n_blocks = n, n_blocks
        self.t = (dev(self.quant), dev(self.scales), dev(self.zp))
        self.w = nw.q4_weight(*self.t, n, n_blocks)

    def f64(self, a):
        return gemv_f64(a, self.quant, self.scales, self.zp)


def _ctx(H=32, Hkv=8, cap=64, B=1, q="f32", Dh=D):
    return nw.AttnContext(H, Hkv, cap, head_dim=Dh, max_batch=B, q_dtype=q, o_dtype="f32",
                          kv_dtype="f32")


@pytest.mark.parametrize("n,n_blocks,batch", [
    (5120, 98, 1),    # q_proj of the Nano-4B attention layer
    (1024, 98, 1),    # k_proj / v_proj
    (3136, 160, 1),   # o_proj
    (37, 3, 2),       # ragged column tail, one slot
    (20, 256, 3),     # K = 8192, four slots
    (64, 65, 1),      # 65 blocks: lane 0 holds two
    (53, 70, 1),      # K split over 2 wavefronts, ragged column tail
    (37, 130, 2),     # K split over 4 wavefronts (33 + 33 + 33 + 31 blocks), ragged tail
    (24, 64, 1),      # 2 parts of exactly 32 blocks
])
def test_gemv_matches_float64(n, n_blocks, batch):
    say(f"q4_gemv n={n} n_blocks={n_blocks} batch={batch}")
    g = rng(200 + n + n_blocks)
    w = DevQ4(g, n, n_blocks)
    a = g.standard_normal((batch, 32 * n_blocks)).astype(np.float32)
    y = torch.full((batch, n), float("nan"), dtype=torch.float32, device="cuda")
    with _ctx() as ctx:
        ctx.q4_gemv(dev(a), w.w, y, batch)
        got = host(y)
    for b in range(batch):
        y64, bound = w.f64(a[b])
        assert np.all(np.abs(got[b] - y64) <= TOL_REL * bound), b
        ref = oracle.q4_gemv_f32(a[b], w.quant, w.scales, w.zp)
        assert np.all(np.abs(got[b] - ref) <= 2 * TOL_REL * bound), b


def test_gemv_epilogues_exact():
    say("q4_gemv epilogues relu2 / accumulate")
    g = rng(301)
    n, nb, batch = 300, 98, 2
    w = DevQ4(g, n, nb)
    a = dev(g.standard_normal((batch, 32 * nb)).astype(np.float32))
    prev = g.standard_normal((batch, n)).astype(np.float32)
    with _ctx() as ctx:
        plain = torch.empty((batch, n), dtype=torch.float32, device="cuda")
        ctx.q4_gemv(a, w.w, plain, batch, nw.NWD_Q4_PLAIN)
        relu = torch.empty_like(plain)
        ctx.q4_gemv(a, w.w, relu, batch, nw.NWD_Q4_RELU2)
        acc = dev(prev)
        ctx.q4_gemv(a, w.w, acc, batch, nw.NWD_Q4_ACCUMULATE)
        p, r, s = host(plain), host(relu), host(acc)
    t = np.maximum(p, np.float32(0))
    np.testing.assert_array_equal(r, t * t)
    np.testing.assert_array_equal(s, prev + p)


def _ulp_f16(x: np.ndarray) -> np.ndarray:
    h = x.astype(np.float16)
    return np.abs((np.nextafter(h, np.float16(np.inf)) - h).astype(np.float64))


@pytest.mark.parametrize("H,Hkv,q,Dh", [(40, 8, "f32", 128), (32, 8, "f16", 128), (16, 4, "f32", 128),
                                        (12, 4, "f32", 64), (6, 2, "f16", 96)])
def test_qkv_append_matches_float64(H, Hkv, q, Dh):
    """Also at head sizes 64 and 96 (groups 3), the cache rows placed with
    the context's head size."""
    say(f"qkv_append H={H} Hkv={Hkv} q={q} D={Dh}")
    g = rng(400 + H)
    B, cap, nb = 2, 48, HIDDEN // 32
    wq, wk, wv = DevQ4(g, H * Dh, nb), DevQ4(g, Hkv * Dh, nb), DevQ4(g, Hkv * Dh, nb)
    x = g.standard_normal((B, HIDDEN)).astype(np.float32)
    pos = [5, cap - 1]
    canary = -7.5
    with _ctx(H, Hkv, cap, B, q, Dh) as ctx:
        kc = torch.full((B, Hkv, cap, Dh), canary, dtype=torch.float16, device="cuda")
        vc = kc.clone()
        q_out = torch.empty((B, H, Dh), dtype=torch.float32 if q == "f32" else torch.float16,
                            device="cuda")
        ctx.qkv_append(dev(x), wq.w, wk.w, wv.w, q_out, kc, vc, pos_tensor(pos), B)
        assert ctx.device_status() == nw.NWD_OK
        qo, kh, vh = host(q_out).astype(np.float32), host(kc), host(vc)
    for b in range(B):
        y64, bound = wq.f64(x[b])
        got = qo[b].reshape(-1)
        if q == "f32":
            assert np.all(np.abs(got - y64) <= TOL_REL * bound)
        else:
            assert np.all(np.abs(got - y64) <= TOL_REL * bound + _ulp_f16(y64))
        for wm, cache in ((wk, kh), (wv, vh)):
            y64, bound = wm.f64(x[b])
            row = cache[b, :, pos[b], :].astype(np.float64).reshape(-1)
            assert np.all(np.abs(row - y64) <= TOL_REL * bound + _ulp_f16(y64))
            others = np.delete(cache[b], pos[b], axis=1)
            assert np.all(others == np.float16(canary))


def test_qkv_append_bad_position_writes_no_row():
    say("qkv_append bad position")
    g = rng(402)
    H, Hkv, cap, nb = 32, 8, 16, 4
    wq, wk, wv = DevQ4(g, H * D, nb), DevQ4(g, Hkv * D, nb), DevQ4(g, Hkv * D, nb)
    x = dev(g.standard_normal((1, 32 * nb)).astype(np.float32))
    with _ctx(H, Hkv, cap) as ctx:
        kc = torch.zeros((1, Hkv, cap, D), dtype=torch.float16, device="cuda")
        vc = kc.clone()
        q_out = torch.empty((1, H, D), dtype=torch.float32, device="cuda")
        for p in (cap, -1):
            ctx.qkv_append(x, wq.w, wk.w, wv.w, q_out, kc, vc, pos_tensor([p]), 1)
            assert ctx.device_status() == nw.NWD_ERR_DEVICE
            assert int(torch.count_nonzero(kc)) == 0 and int(torch.count_nonzero(vc)) == 0
        assert ctx.device_status() == nw.NWD_OK


def test_qkv_append_then_decode_matches_oracle_chain():
    """The attention layer from the hidden state: projections, cache write,
    attention — against q4 GEMV oracle -> fp16 cache -> sparse_attn oracle."""
    say("qkv_append + decode vs oracle chain, H=40 Hkv=8 past=100")
    g = rng(403)
    H, Hkv, cap, nb, past = 40, 8, 128, HIDDEN // 32, 100
    wq, wk, wv = DevQ4(g, H * D, nb), DevQ4(g, Hkv * D, nb), DevQ4(g, Hkv * D, nb)
    x = g.standard_normal((1, HIDDEN)).astype(np.float32)
    k_past = g.standard_normal((past, Hkv, D)).astype(np.float16)
    v_past = g.standard_normal((past, Hkv, D)).astype(np.float16)
    with _ctx(H, Hkv, cap) as ctx:
        kc = torch.zeros((1, Hkv, cap, D), dtype=torch.float16, device="cuda")
        vc = kc.clone()
        kc[0, :, :past, :] = dev(k_past).permute(1, 0, 2)
        vc[0, :, :past, :] = dev(v_past).permute(1, 0, 2)
        q_out = torch.empty((1, H, D), dtype=torch.float32, device="cuda")
        out = torch.empty((1, H, D), dtype=torch.float32, device="cuda")
        pos = pos_tensor([past])
        ctx.qkv_append(dev(x), wq.w, wk.w, wv.w, q_out, kc, vc, pos, 1)
        ctx.decode(q_out, kc, vc, pos, out, 1, past + 1)
        assert ctx.device_status() == nw.NWD_OK
        got = host(out)[0]
    q_ref = oracle.q4_gemv_f32(x[0], wq.quant, wq.scales, wq.zp).reshape(H, D)
    k_new = oracle.q4_gemv_f32(x[0], wk.quant, wk.scales, wk.zp).reshape(Hkv, D)
    v_new = oracle.q4_gemv_f32(x[0], wv.quant, wv.scales, wv.zp).reshape(Hkv, D)
    k_all = np.concatenate([k_past.astype(np.float32),
                            oracle.f16_to_f32(oracle.f32_to_f16(k_new))[None]], axis=0)
    v_all = np.concatenate([v_past.astype(np.float32),
                            oracle.f16_to_f32(oracle.f32_to_f16(v_new))[None]], axis=0)
    ref = oracle.sparse_attn_f32(q_ref, k_all, v_all)
    assert max_abs(got, ref) <= 2e-3


def test_q4_host_validation():
    say("q4 host validation (no launch)")
    g = rng(404)
    with _ctx(32, 8, 16) as ctx:
        wq, wk = DevQ4(g, 32 * D, 4), DevQ4(g, 8 * D, 4)
        wk5 = DevQ4(g, 8 * D, 5)
        x = torch.zeros((1, 128), dtype=torch.float32, device="cuda")
        buf = torch.zeros((1, 32, D), dtype=torch.float32, device="cuda")
        kc = torch.zeros((1, 8, 16, D), dtype=torch.float16, device="cuda")
        pos = pos_tensor([0])
        cases = [
            (lambda: ctx.qkv_append(x, wk.w, wk.w, wk.w, buf, kc, kc, pos, 1), nw.NWD_ERR_INVALID),
            (lambda: ctx.qkv_append(x, wq.w, wq.w, wk.w, buf, kc, kc, pos, 1), nw.NWD_ERR_INVALID),
            (lambda: ctx.qkv_append(x, wq.w, wk.w, wk5.w, buf, kc, kc, pos, 1), nw.NWD_ERR_INVALID),
            (lambda: ctx.qkv_append(x, wq.w, wk.w, wk.w, buf, kc, kc, pos, 2), nw.NWD_ERR_CAPACITY),
            (lambda: ctx.qkv_append(x.data_ptr() + 4, wq.w, wk.w, wk.w, buf, kc, kc, pos, 1),
             nw.NWD_ERR_INVALID),
            (lambda: ctx.q4_gemv(x, wk.w, buf, 1, 7), nw.NWD_ERR_INVALID),
            (lambda: ctx.q4_gemv(x, nw.q4_weight(wk.t[0].data_ptr() + 8, wk.t[1], wk.t[2], 8 * D, 4),
                                 buf, 1), nw.NWD_ERR_INVALID),
            (lambda: ctx.q4_gemv(x, nw.q4_weight(*wk.t, 8 * D, 257), buf, 1), nw.NWD_ERR_UNSUPPORTED),
            (lambda: ctx.q4_gemv(x, nw.q4_weight(*wk.t, 0, 4), buf, 1), nw.NWD_ERR_INVALID),
            (lambda: ctx.q4_gemv(x, wk.w, buf, 0), nw.NWD_ERR_INVALID),
        ]
        for i, (call, code) in enumerate(cases):
            with pytest.raises(nw.NwdError) as e:
                call()
            assert e.value.code == code, (i, e.value)
        assert ctx.device_status() == nw.NWD_OK
    # head size 100 with 2 KV heads: 200 k columns do not split into whole
    # 16-column workgroups, so the fused projection refuses the shape
    with _ctx(4, 2, 16, Dh=100) as ctx:
        wq, wk = DevQ4(g, 400, 4), DevQ4(g, 200, 4)
        buf = torch.zeros((1, 400), dtype=torch.float32, device="cuda")
        kc = torch.zeros((1, 2, 16, 100), dtype=torch.float16, device="cuda")
        x = torch.zeros((1, 128), dtype=torch.float32, device="cuda")
        with pytest.raises(nw.NwdError) as e:
            ctx.qkv_append(x, wq.w, wk.w, wk.w, buf, kc, kc, pos_tensor([0]), 1)
        assert e.value.code == nw.NWD_ERR_UNSUPPORTED and "multiples of 16" in str(e.value)
