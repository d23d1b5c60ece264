"""Parity of the causal chunked prefill (nwd_prefill_attn, fp16 MFMA) with the
oracle. The reference's prefill is token-by-token decode
(engine/runtime.js:640-643), so query i of a chunk appended at pos0 must equal
decode attention over keys 0..pos0+i; the oracle's sparse_attn restatement is
run with seq = pos0 + i + 1 for each checked query."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import nwd_attn as nw  # noqa: E402
import oracle  # noqa: E402
from attn_cases import f32, kv_rows, max_abs, normal_f16, rng, to_cache  # noqa: E402
from gpu_util import cache_rows_f32, dev, pos_tensor, randn_f16, say  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 2e-3
D = 128


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    nw.load_library()


def _run_prefill(H, Hkv, pos0s, n_new, seed, io="f16"):
    """Appends n_new rows per sequence with nwd_kv_append, then prefills.
    Returns (out [B][n_new][H][D] f32, q f16, per-seq token-major k, v)."""
    B = len(pos0s)
    g = rng(seed)
    cap = max(pos0s) + n_new + 5
    rows = [kv_rows(g, p + n_new, Hkv) for p in pos0s]
    q16 = normal_f16(g, (B, n_new, H, D))
    with nw.AttnContext(H, Hkv, cap, max_batch=B, q_dtype=io, o_dtype=io, kv_dtype="f16") as ctx:
        kc = dev(to_cache([r[0][:p] for r, p in zip(rows, pos0s)], Hkv, cap))
        vc = dev(to_cache([r[1][:p] for r, p in zip(rows, pos0s)], Hkv, cap))
        pos = pos_tensor(pos0s)
        knew = np.stack([r[0][p:] for r, p in zip(rows, pos0s)])
        vnew = np.stack([r[1][p:] for r, p in zip(rows, pos0s)])
        ctx.kv_append(dev(knew), dev(vnew), kc, vc, pos, B, n_new)
        q = dev(f32(q16) if io == "f32" else q16)
        out = torch.empty((B, n_new, H, D), dtype=q.dtype, device="cuda")
        ctx.prefill(q, kc, vc, pos, out, B, n_new, max_len=cap)
        assert ctx.device_status() == nw.NWD_OK
        return out.float().cpu().numpy(), q16, rows


def _check_rows(out, q16, rows, pos0s, queries):
    worst = 0.0
    for b, p in enumerate(pos0s):
        kf, vf = f32(rows[b][0]), f32(rows[b][1])
        for i in queries:
            want = oracle.sparse_attn_f32(f32(q16[b, i]), kf[:p + i + 1], vf[:p + i + 1], threads=0)
            worst = max(worst, max_abs(out[b, i], want))
    return worst


@pytest.mark.parametrize("G", [1, 2, 4, 5, 8])
def test_prefill_small_all_queries(G):
    Hkv = 2
    say(f"prefill small G={G}")
    pos0s, n_new = [100], 37
    out, q16, rows = _run_prefill(G * Hkv, Hkv, pos0s, n_new, 80 + G)
    assert _check_rows(out, q16, rows, pos0s, range(n_new)) < TOL


@pytest.mark.parametrize("G", [4, 5])
def test_prefill_short_prompt_one_split(G):
    """A prompt of 60 tokens from an empty cache: every row tile has one
    key tile, so its keys are not split and the output is written directly."""
    say(f"prefill short prompt G={G}")
    Hkv = 8
    out, q16, rows = _run_prefill(G * Hkv, Hkv, [0], 60, 95 + G)
    assert _check_rows(out, q16, rows, [0], range(60)) < TOL


def test_prefill_batch_ragged_f32_io():
    say("prefill batch=3 f32 io")
    pos0s, n_new = [0, 65, 300], 70
    out, q16, rows = _run_prefill(32, 8, pos0s, n_new, 90, io="f32")
    assert _check_rows(out, q16, rows, pos0s, range(0, n_new, 3)) < TOL


@pytest.mark.parametrize("sigma", [1.0, 4.0])
def test_prefill_config5_offgrid_f32_queries(sigma):
    """Config 5's shape (32q/8kv, 512 new tokens onto 8192) with fp32 queries
    off the fp16 grid, as the engine's q projection produces them
    (engine/runtime.js:120, kernels/sparse_attn.wgsl:19 reads f32 Q): every
    query against the oracle run on the same fp32 query rows. sigma 4 gives
    scores four times sharper than N(0, 1) rows, where a query rounded to
    fp16 misses the bar."""
    H, Hkv, P, n_new = 32, 8, 8192, 512
    cap = P + n_new
    say(f"config5 prefill fp32 off-grid queries sigma={sigma}")
    g = rng(777 + int(sigma))
    k, v = kv_rows(g, cap, Hkv)
    q = (g.standard_normal((1, n_new, H, D)) * sigma).astype(np.float32)
    assert not np.array_equal(q, f32(q.astype(np.float16)))
    with nw.AttnContext(H, Hkv, cap, q_dtype="f32", o_dtype="f32") as ctx:
        kc = dev(to_cache([k], Hkv, cap))
        vc = dev(to_cache([v], Hkv, cap))
        out = torch.empty((1, n_new, H, D), dtype=torch.float32, device="cuda")
        ctx.prefill(dev(q), kc, vc, pos_tensor([P]), out, 1, n_new, max_len=cap)
        assert ctx.device_status() == nw.NWD_OK
        got = out.cpu().numpy()[0]
    kf, vf = f32(k), f32(v)
    worst = 0.0
    for i in range(n_new):
        if i % 128 == 0:
            say(f"  oracle queries {i}..{i + 127}")
        want = oracle.sparse_attn_f32(q[0, i], kf[:P + i + 1], vf[:P + i + 1], threads=0)
        worst = max(worst, max_abs(got[i], want))
    say(f"  worst {worst:.2e}")
    assert worst < TOL, worst


@pytest.mark.parametrize("io", ["f16", "f32"])
def test_prefill_scaled_matches_sequential_decode(io):
    """A non-default softmax scale (0.3, factor scale * log2 e = 0.43): the
    prefill chunk against the token-by-token decode on the GPU and against
    the float64 definition with that scale. fp16 queries are rounded once
    more after the scaling in the prefill (the decode keeps them exact); the
    bar is the same 2e-3."""
    say(f"prefill scale 0.3 io={io} == sequential decode")
    H, Hkv, P, n_new, scale = 32, 8, 300, 40, 0.3
    cap = P + n_new
    g = rng(94)
    k, v = kv_rows(g, cap, Hkv)
    q16 = normal_f16(g, (1, n_new, H, D))
    qh = f32(q16) if io == "f32" else q16
    if io == "f32":  # off the fp16 grid
        qh = (qh + g.standard_normal(qh.shape).astype(np.float32) * 1e-3).astype(np.float32)
    with nw.AttnContext(H, Hkv, cap, o_dtype="f32", q_dtype=io, scale=scale) as ctx:
        kc, vc = dev(to_cache([k[:P]], Hkv, cap)), dev(to_cache([v[:P]], Hkv, cap))
        seq = []
        for i in range(n_new):
            pos = pos_tensor([P + i])
            ctx.kv_append(dev(k[P + i:P + i + 1][None]), dev(v[P + i:P + i + 1][None]), kc, vc, pos, 1, 1)
            o = torch.empty((1, H, D), dtype=torch.float32, device="cuda")
            ctx.decode(dev(qh[:, i]), kc, vc, pos, o, 1)
            seq.append(o)
        out = torch.empty((1, n_new, H, D), dtype=torch.float32, device="cuda")
        ctx.prefill(dev(qh), kc, vc, pos_tensor([P]), out, 1, n_new)
        assert ctx.device_status() == nw.NWD_OK
        torch.cuda.synchronize()
    got = out.cpu().numpy()
    vs_decode = max_abs(got, torch.stack(seq, dim=1).cpu().numpy())
    assert vs_decode < TOL, vs_decode
    kf, vf, qf = f32(k), f32(v), np.asarray(qh, np.float32)
    worst = 0.0
    for i in (0, 7, 39):
        want = oracle.attn_f64(qf[0, i], kf[:P + i + 1], vf[:P + i + 1], scale=scale)
        worst = max(worst, max_abs(got[0, i], want))
    assert worst < TOL, worst


def test_prefill_query_range_flagged():
    """An fp32 query whose scaled value leaves the fp16 range of the MFMA
    operand (scale 8: factor 11.5, |q| = 8000) is reported by
    nwd_device_status as NWD_ERR_DEVICE instead of passing silently; the
    next call is clean. fp16 queries enter the MFMAs unscaled and are never
    flagged."""
    say("prefill query range flag")
    H, Hkv, P, n_new = 8, 2, 64, 16
    cap = P + n_new
    g = rng(95)
    k, v = kv_rows(g, cap, Hkv)
    q = f32(normal_f16(g, (1, n_new, H, D)))
    with nw.AttnContext(H, Hkv, cap, scale=8.0, q_dtype="f32", o_dtype="f32") as ctx:
        kc, vc = dev(to_cache([k], Hkv, cap)), dev(to_cache([v], Hkv, cap))
        out = torch.empty((1, n_new, H, D), dtype=torch.float32, device="cuda")
        ctx.prefill(dev(q), kc, vc, pos_tensor([P]), out, 1, n_new)
        assert ctx.device_status() == nw.NWD_OK
        big = q.copy()
        big[0, 3, 5, 17] = np.float32(8000.0)
        ctx.prefill(dev(big), kc, vc, pos_tensor([P]), out, 1, n_new)
        assert ctx.device_status() == nw.NWD_ERR_DEVICE
        assert "fp16 range" in ctx.last_error()
        ctx.prefill(dev(q), kc, vc, pos_tensor([P]), out, 1, n_new)
        assert ctx.device_status() == nw.NWD_OK


def test_prefill_from_empty_cache_is_causal():
    """pos0 = 0: query 0 sees only itself, so O = V[0] up to fp16 P rounding."""
    say("prefill from empty cache")
    out, q16, rows = _run_prefill(8, 2, [0], 129, 91)
    assert max_abs(out[0, 0], np.repeat(f32(rows[0][1][0]), 4, axis=0)) < 1e-3
    assert _check_rows(out, q16, rows, [0], range(129)) < TOL


def test_config5_chunk512_onto_8192():
    """32q/8kv/d128: 512 new tokens appended at 8192, causal within the chunk.
    Every query against the oracle and against a torch fp32 reference of the
    same masked softmax."""
    H, Hkv, P, n_new = 32, 8, 8192, 512
    cap = P + n_new
    say("config5 prefill 512 onto 8192")
    kc = randn_f16((1, Hkv, cap, D), 500)
    vc = randn_f16((1, Hkv, cap, D), 501)
    q = randn_f16((1, n_new, H, D), 502)
    with nw.AttnContext(H, Hkv, cap) as ctx:
        out = torch.empty_like(q)
        ctx.prefill(q, kc, vc, pos_tensor([P]), out, 1, n_new, max_len=cap)
        assert ctx.device_status() == nw.NWD_OK
    got = out.float()
    # torch fp32 reference, one kv head at a time
    G = H // Hkv
    worst_t = 0.0
    keys = torch.arange(cap, device="cuda")
    lim = P + torch.arange(n_new, device="cuda")
    mask = keys[None, :] > lim[:, None]
    for h in range(Hkv):
        kf = kc[0, h].float()
        vf = vc[0, h].float()
        for g in range(G):
            qf = q[0, :, h * G + g, :].float()
            s = (qf @ kf.t()) / np.sqrt(D)
            s = s.masked_fill(mask, float("-inf"))
            ref = torch.softmax(s, dim=-1) @ vf
            worst_t = max(worst_t, float((ref - got[0, :, h * G + g, :]).abs().max()))
    assert worst_t < TOL, worst_t
    # the oracle on every query: the caches once, token-major, then key prefixes
    qh = q.float().cpu().numpy()
    oh = got.cpu().numpy()
    kk = cache_rows_f32(kc, 0, cap)
    vv = cache_rows_f32(vc, 0, cap)
    worst = 0.0
    for i in range(n_new):
        if i % 128 == 0:
            say(f"config5 oracle queries {i}..{i + 127}")
        L = P + i + 1
        want = oracle.sparse_attn_f32(qh[0, i], kk[:L], vv[:L], threads=0)
        worst = max(worst, max_abs(oh[0, i], want))
    assert worst < TOL, worst


def test_prefill_matches_sequential_decode():
    """The chunk equals the reference's token-by-token loop run on the GPU
    decode path (append one token, attend, repeat)."""
    say("prefill == sequential decode")
    H, Hkv, P, n_new = 32, 8, 40, 20
    cap = P + n_new
    g = rng(93)
    k, v = kv_rows(g, cap, Hkv)
    q = normal_f16(g, (1, n_new, H, D))
    with nw.AttnContext(H, Hkv, cap, o_dtype="f32", q_dtype="f16") as ctx:
        kc, vc = dev(to_cache([k[:P]], Hkv, cap)), dev(to_cache([v[:P]], Hkv, cap))
        seq = []
        for i in range(n_new):
            pos = pos_tensor([P + i])
            ctx.kv_append(dev(k[P + i:P + i + 1][None]), dev(v[P + i:P + i + 1][None]), kc, vc, pos, 1, 1)
            o = torch.empty((1, H, D), dtype=torch.float32, device="cuda")
            ctx.decode(dev(q[:, i]), kc, vc, pos, o, 1)
            seq.append(o)
        out = torch.empty((1, n_new, H, D), dtype=torch.float32, device="cuda")
        ctx.prefill(dev(q), kc, vc, pos_tensor([P]), out, 1, n_new)
        torch.cuda.synchronize()
    stepwise = torch.stack(seq, dim=1).cpu().numpy()
    assert max_abs(out.cpu().numpy(), stepwise) < TOL


def test_prefill_at_max_seq():
    """A 64-token chunk appended at the end of the largest capacity (max_seq =
    2^22, one KV head, 1 GiB slabs): each query attends ~2^22 keys, so every
    row tile's key range is split (and merged) over several workgroups. Old
    keys are zero (score 0) with V = 0.25; the new keys are a dominant
    direction u (score 40 against every query), so query i averages the new
    V rows 0..i up to a weight of 2^22 * exp(-40)."""
    say("prefill 64 new tokens at the end of max_seq = 2^22")
    cap, n_new, H, Hkv = 1 << 22, 64, 4, 1
    p0 = cap - n_new
    g = rng(4343)
    u = g.standard_normal(D)
    u /= np.linalg.norm(u)
    q = np.tile(u, (1, n_new, H, 1)).astype(np.float16)
    knew = np.tile((40.0 * np.sqrt(D) * u).astype(np.float16), (1, n_new, Hkv, 1))
    vnew = g.standard_normal((1, n_new, Hkv, D)).astype(np.float16)
    with nw.AttnContext(H, Hkv, cap) as ctx:
        kc = torch.zeros((1, Hkv, cap, D), dtype=torch.float16, device="cuda")
        vc = torch.full((1, Hkv, cap, D), 0.25, dtype=torch.float16, device="cuda")
        pos = pos_tensor([p0])
        ctx.kv_append(dev(knew), dev(vnew), kc, vc, pos, 1, n_new)
        out = torch.empty((1, n_new, H, D), dtype=torch.float16, device="cuda")
        ctx.prefill(dev(q), kc, vc, pos, out, 1, n_new)
        assert ctx.device_status() == nw.NWD_OK
        o = out.float().cpu().numpy()
    v = vnew[0, :, 0].astype(np.float64)
    for i in range(n_new):
        want = v[:i + 1].mean(axis=0)
        for h in range(H):
            assert max_abs(o[0, i, h], want) < 2e-3, (i, h)


@pytest.mark.parametrize("offset", [0.0, -60.0])
def test_prefill_rising_and_negative_scores(offset):
    """Scores that climb ~33 log2 units across the keys make the weights of
    later tiles overflow fp16 against the reference point a wavefront took
    from its first keys, so the kernel's overflow path (row maximum, rescale,
    weights again) runs many times per row; offset -60 puts every score near
    -60 / ln 2 log2 units, where weights taken without a row maximum would
    underflow. Checked against a float64 softmax of the same fp16 inputs."""
    say(f"prefill rising scores offset={offset}")
    H, Hkv, P, n_new = 8, 2, 1200, 100
    cap = P + n_new
    g = rng(4411)
    u = g.standard_normal(D)
    u /= np.linalg.norm(u)
    # q = 4u, k_j = (0.05 j + offset * sqrt(D) / 4) u + noise: the scaled
    # score is 0.2 j / sqrt(D) + offset (3.3 log2 units more per 128 keys).
    q = (np.tile(4.0 * u, (1, n_new, H, 1)) + 0.05 * g.standard_normal((1, n_new, H, D))).astype(np.float16)
    j = np.arange(cap, dtype=np.float64)[:, None]
    base = (0.05 * j + offset * np.sqrt(D) / 4.0) * u[None, :]
    k = np.stack([base + 0.05 * g.standard_normal((cap, D)) for _ in range(Hkv)], axis=1).astype(np.float16)
    v = g.standard_normal((cap, Hkv, D)).astype(np.float16)
    with nw.AttnContext(H, Hkv, cap, o_dtype="f32") as ctx:
        kc = dev(np.ascontiguousarray(k.transpose(1, 0, 2))[None])
        vc = dev(np.ascontiguousarray(v.transpose(1, 0, 2))[None])
        out = torch.empty((1, n_new, H, D), dtype=torch.float32, device="cuda")
        ctx.prefill(dev(q), kc, vc, pos_tensor([P]), out, 1, n_new)
        assert ctx.device_status() == nw.NWD_OK
        got = out.cpu().numpy()[0]
    G = H // Hkv
    kf, vf, qf = k.astype(np.float64), v.astype(np.float64), q[0].astype(np.float64)
    worst = 0.0
    for i in (0, 1, 37, 63, 64, 99):
        L = P + i + 1
        for h in range(H):
            s = kf[:L, h // G] @ qf[i, h] / np.sqrt(D)
            w = np.exp(s - s.max())
            want = (w[:, None] * vf[:L, h // G]).sum(axis=0) / w.sum()
            worst = max(worst, float(np.abs(got[i, h] - want).max()))
    assert worst < TOL, worst
