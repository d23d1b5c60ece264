"""Seeded random sweep over the whole call surface against the oracle.

The reference's attention takes any head size and group
(kernels/sparse_attn.wgsl:12-17, :38-43) and kv_append any row width
(kernels/kv_append.wgsl:1-6). The library routes a shape to one of several
kernels by head size, group, batch, length and split count (the specialised
split kernels at head sizes 64/128/256, the padded-group and padded-head
routes, the MFMA prefill, the general kernels). Each case here draws a
shape, dtypes, a ragged batch, an operation (decode, fused append + decode,
two-call append + decode, chunked prefill) and a split count, and checks
every output row against the oracle's op-for-op f32 restatement of
sparse_attn.wgsl (max-abs 2e-3, fp16 inputs widened exactly) and the
appended cache rows bit for bit (fp16 rows copied, fp32 rows rounded to
nearest even). The draw is fixed by the case number, so a failure names a
case that can be rerun. A second sweep draws only head sizes 64 and 128 with
groups 3, 6, 7 and the larger groups that divide into them (12, 14, 21),
which run kernels built for those groups there.
"""
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import nwd_attn as nw  # noqa: E402
import oracle  # noqa: E402
from attn_cases import f32, from_cache, max_abs, rng, to_cache  # noqa: E402
from gpu_util import dev, host, pos_tensor, say  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 2e-3
# Case counts and the first seed can be raised for a longer sweep, e.g.
# NWD_RANDOM_CASES=2000 NWD_RANDOM_BASE=20000 NWD_RANDOM_BUILT_CASES=500.
N_CASES = int(os.environ.get("NWD_RANDOM_CASES", "200"))
BASE = int(os.environ.get("NWD_RANDOM_BASE", "5000"))
N_BUILT = int(os.environ.get("NWD_RANDOM_BUILT_CASES", "40"))
HEAD_DIMS = [1, 3, 8, 16, 24, 32, 40, 48, 64, 64, 72, 80, 96, 96, 100, 112, 120, 128, 128, 128,
             136, 160, 192, 200, 256, 256, 320, 512]
GROUPS = [1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 12, 16, 24, 25, 40]
# bound on B * H * L * D of a case, which keeps the oracle to a fraction of a second
WORK = 60_000_000


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    nw.load_library()


def _draw(i: int, dims=HEAD_DIMS, groups=GROUPS, base: int = 5000) -> dict:
    g = rng(base + i)
    D = int(g.choice(dims))
    G = int(g.choice(groups))
    Hkv = int(g.choice([1, 2, 4, 8]))
    H = Hkv * G
    B = int(g.integers(1, 5))
    op = str(g.choice(["decode", "append_decode", "append_then_decode", "prefill"]))
    n_new = int(g.integers(1, 48)) if op == "prefill" else 1
    max_len = max(1, WORK // (B * H * D * (n_new if op == "prefill" else 1)))
    max_len = int(min(max_len, 4000))
    past = [int(g.integers(0, max(1, max_len - n_new))) for _ in range(B)]
    return {"D": D, "H": H, "Hkv": Hkv, "B": B, "op": op, "n_new": n_new, "past": past,
            "io": str(g.choice(["f16", "f32"])), "kv": str(g.choice(["f16", "f32"])),
            "splits": int(g.choice([0, 0, 1, 3, 17])), "seed": base + 1000 + i}


def _tdtype(name):
    return torch.float16 if name == "f16" else torch.float32


def _rows(g, n, Hkv, D, dtype="f16"):
    x = g.standard_normal((n, Hkv, D), dtype=np.float32)
    return x.astype(np.float16) if dtype == "f16" else x


@pytest.mark.parametrize("case", range(N_CASES))
def test_random_shape_matches_oracle(case):
    _check(_draw(case, base=BASE), case)


# Groups 3, 6 and 7 (and the larger groups that divide into them) at the
# head sizes where kernels are built for them, 64 and 128.
@pytest.mark.parametrize("case", range(N_BUILT))
def test_random_built_group_matches_oracle(case):
    _check(_draw(case, dims=[64, 128], groups=[3, 6, 7, 12, 14, 21], base=BASE + 3000), case)


def _check(c: dict, case: int):
    say(f"random case {case}: {c}")
    g = rng(c["seed"])
    D, H, Hkv, B, n_new, past = c["D"], c["H"], c["Hkv"], c["B"], c["n_new"], c["past"]
    cap = max(past) + n_new + int(g.integers(0, 9))
    # cached rows 0 .. past-1, scaled keys so that the scores stay moderate at every D
    old = [(_rows(g, p, Hkv, D) * np.float16(0.5), _rows(g, p, Hkv, D)) for p in past]
    new = [(_rows(g, n_new, Hkv, D, c["kv"]), _rows(g, n_new, Hkv, D, c["kv"])) for _ in past]
    qshape = (B, n_new, H, D) if c["op"] == "prefill" else (B, H, D)
    q = g.standard_normal(qshape, dtype=np.float32)
    if c["io"] == "f16":
        q = q.astype(np.float16)

    def padded(rows, p):  # [cap][Hkv][D] fp16 with rows 0..p-1
        full = np.zeros((max(p, 1), Hkv, D), np.float16)
        full[:p] = rows[:p]
        return full

    with nw.AttnContext(H, Hkv, cap, head_dim=D, max_batch=B, q_dtype=c["io"], o_dtype=c["io"],
                        kv_dtype=c["kv"]) as ctx:
        if c["splits"]:
            ctx.set_decode_splits(c["splits"])
        kc = dev(to_cache([padded(k, p) for (k, _), p in zip(old, past)], Hkv, cap))
        vc = dev(to_cache([padded(v, p) for (_, v), p in zip(old, past)], Hkv, cap))
        kn = dev(np.stack([k for k, _ in new]))  # [B][n_new][Hkv][D]
        vn = dev(np.stack([v for _, v in new]))
        pos = pos_tensor(past)
        out = torch.empty(qshape, dtype=_tdtype(c["io"]), device="cuda")
        bound = max(past) + n_new
        if c["op"] == "decode":
            ctx.kv_append(kn, vn, kc, vc, pos, B, 1)
            ctx.decode(dev(q), kc, vc, pos, out, B, bound)
        elif c["op"] == "append_decode":
            ctx.append_decode(dev(q), kn[:, 0], vn[:, 0], kc, vc, pos, out, B, bound)
        elif c["op"] == "append_then_decode":
            ctx.kv_append(kn, vn, kc, vc, pos, B, 1)
            ctx.decode(dev(q), kc, vc, pos, out, B, 0)
        else:
            ctx.kv_append(kn, vn, kc, vc, pos, B, n_new)
            ctx.prefill(dev(q), kc, vc, pos, out, B, n_new, bound)
        assert ctx.device_status() == nw.NWD_OK
        got = host(out).astype(np.float32)
        kc_h, vc_h = host(kc), host(vc)

    worst = 0.0
    for b in range(B):
        L = past[b] + n_new
        kk, vv = from_cache(kc_h, b, L), from_cache(vc_h, b, L)
        # the appended rows, bit for bit (fp32 rows rounded to nearest even)
        for src, cache in ((new[b][0], kk), (new[b][1], vv)):
            want = np.asarray(src, np.float32).astype(np.float16)
            assert np.array_equal(cache[past[b]:L].view(np.uint16), want.view(np.uint16)), b
        assert np.array_equal(kk[:past[b]].view(np.uint16), old[b][0].view(np.uint16)), b
        if c["op"] == "prefill":
            for i in range(n_new):
                want = oracle.sparse_attn_f32(q[b, i].astype(np.float32), f32(kk[:past[b] + i + 1]),
                                              f32(vv[:past[b] + i + 1]))
                worst = max(worst, max_abs(got[b, i], want))
        else:
            want = oracle.sparse_attn_f32(q[b].astype(np.float32), f32(kk), f32(vv))
            worst = max(worst, max_abs(got[b], want))
    say(f"  max-abs {worst:.2e}")
    assert worst < TOL, (case, worst)
