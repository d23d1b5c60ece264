"""Parity of the greedy pick (nwd_argmax) and of lm_head + pick
(nwd_lm_head_argmax) with the oracle's op-for-op restatement of
kernels/argmax_partial.wgsl + argmax_merge.wgsl, through the C ABI.

Bars: the index is bit-exact against the oracle on the same logits,
including the reference's tie order, NaN, -inf and -3.402823466e38; the
lm_head logits are within 1e-6 of sum |w a| of the float64 projection, and
the picked token equals the oracle's pick on the oracle's own logits unless
the top two logits are closer than that tolerance.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import nwd_attn as nw  # noqa: E402
import oracle  # noqa: E402
from argmax_cases import NEG_FLT_MAX, tie_heavy  # noqa: E402
from gpu_util import dev, host, say  # noqa: E402
from q4_cases import HIDDEN, gemv_f64, random_q4, rng  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    nw.load_library()


def _ctx():
    return nw.AttnContext(32, 8, 64, q_dtype="f32", o_dtype="f32", kv_dtype="f32")


def _pick(ctx, x: np.ndarray) -> np.ndarray:
    batch, n = x.shape
    out = torch.full((batch,), 0xDEAD, dtype=torch.int32, device="cuda")
    ctx.argmax(dev(x), n, out, batch)
    return host(out).astype(np.uint32)


@pytest.mark.parametrize("n", [1, 7, 256, 4096, 4097, 131072, 200003])
def test_argmax_random_and_ties(n):
    say(f"argmax n={n}")
    g = rng(500 + n)
    rows = [g.standard_normal(n).astype(np.float32), tie_heavy(g, n), tie_heavy(g, n)]
    x = np.stack(rows)
    with _ctx() as ctx:
        got = _pick(ctx, x)
    for b in range(len(rows)):
        assert got[b] == oracle.argmax_ref(x[b]), (n, b)


def test_argmax_special_values():
    say("argmax special values")
    n = 5000
    rows = []
    r = np.full(n, np.nan, np.float32); rows.append(r)
    r = np.full(n, -np.inf, np.float32); rows.append(r)
    r = np.full(n, NEG_FLT_MAX, np.float32); rows.append(r)
    r = np.zeros(n, np.float32); r[::3] = -0.0; rows.append(r)            # signed zeros tie
    r = np.zeros(n, np.float32); r[::7] = -0.0; r[4000] = np.float32(1e-45); rows.append(r)
    r = np.full(n, NEG_FLT_MAX, np.float32); r[1234] = np.nextafter(NEG_FLT_MAX, np.float32(0)); rows.append(r)
    r = np.zeros(n, np.float32); r[17] = np.inf; r[18] = np.nan; rows.append(r)
    x = np.stack(rows)
    with _ctx() as ctx:
        got = _pick(ctx, x)
    for b in range(len(rows)):
        assert got[b] == oracle.argmax_ref(x[b]), b


@pytest.mark.parametrize("vocab,batch", [(8191, 2), (131072, 1), (20001, 3)])
def test_lm_head_argmax(vocab, batch):
    """8191: the per-slot GEMV form; 131072 and 20001 (>= 16384 columns) the
    wide form, 20001 with a ragged last workgroup and three rows."""
    say(f"lm_head_argmax vocab={vocab} batch={batch}")
    g = rng(600 + vocab)
    nb = HIDDEN // 32
    quant, scales, zp = random_q4(g, vocab, nb)
    h = g.standard_normal((batch, HIDDEN)).astype(np.float32)
    with _ctx() as ctx:
        t = (dev(quant), dev(scales), dev(zp))
        w = nw.q4_weight(*t, vocab, nb)
        logits = torch.empty((batch, vocab), dtype=torch.float32, device="cuda")
        out = torch.zeros((batch,), dtype=torch.int32, device="cuda")
        ctx.lm_head_argmax(dev(h), w, out, logits, batch)
        out_nolog = torch.zeros((batch,), dtype=torch.int32, device="cuda")
        ctx.lm_head_argmax(dev(h), w, out_nolog, None, batch)
        lg, idx, idx2 = host(logits), host(out).astype(np.uint32), host(out_nolog).astype(np.uint32)
    np.testing.assert_array_equal(idx, idx2)
    for b in range(batch):
        y64, bound = gemv_f64(h[b], quant, scales, zp)
        assert np.all(np.abs(lg[b] - y64) <= 1e-6 * bound)
        assert idx[b] == oracle.argmax_ref(lg[b])  # bit-exact on the same logits
        ref_logits = oracle.q4_gemv_f32(h[b], quant, scales, zp, threads=oracle.max_threads())
        ref = oracle.argmax_ref(ref_logits)
        top2 = np.sort(y64)[-2:]
        if top2[1] - top2[0] > 2e-6 * bound.max():
            assert idx[b] == ref


def test_argmax_host_validation():
    say("argmax host validation (no launch)")
    g = rng(700)
    with _ctx() as ctx:
        x = torch.zeros((1, 16), dtype=torch.float32, device="cuda")
        out = torch.zeros((1,), dtype=torch.int32, device="cuda")
        quant, scales, zp = random_q4(g, 16, 4)
        t = (dev(quant), dev(scales), dev(zp))
        cases = [
            (lambda: ctx.argmax(x, 0, out, 1), nw.NWD_ERR_INVALID),
            (lambda: ctx.argmax(x, 16, out, 0), nw.NWD_ERR_INVALID),
            (lambda: ctx.argmax(None, 16, out, 1), nw.NWD_ERR_INVALID),
            (lambda: ctx.lm_head_argmax(x.data_ptr() + 4, nw.q4_weight(*t, 16, 4), out), nw.NWD_ERR_INVALID),
            # 65 rows of a 131072-token vocabulary need more partial records than the workspace
            (lambda: ctx.lm_head_argmax(x, nw.q4_weight(*t, 131072, 4), out, None, 65),
             nw.NWD_ERR_CAPACITY),
        ]
        for i, (call, code) in enumerate(cases):
            with pytest.raises(nw.NwdError) as e:
                call()
            assert e.value.code == code, (i, e.value)
        assert ctx.device_status() == nw.NWD_OK
