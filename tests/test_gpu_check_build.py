"""The debug builds of the library (nemotron-webgpu-decode_amd/build.py
--variants) on the GPU.

lib/check/libnwd_attn.so is built with -DNWD_CHECK: every kernel store
compares its address with the size of the buffer it writes and, when
outside, drops the store and sets a status bit that nwd_device_status
reports. Each entry point is run here on both builds with the same inputs:
the checked build must flag nothing and give the product build's bits.

lib/asan/nwd_abi_asan drives the C ABI through the AddressSanitizer build of
the host code, one context per query-head group through every entry point;
it is run as a child process (the ASan runtime is linked into it).
"""
import os
import subprocess

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import nwd_attn as nw  # noqa: E402
from gpu_util import dev, pos_tensor, randn_f16, say  # noqa: E402
from q4_cases import random_q4, rng  # noqa: E402

pytestmark = pytest.mark.gpu

D = 128
ASAN_DRIVER = nw.PKG_DIR / "lib" / "asan" / "nwd_abi_asan"


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    nw.load_library()
    if not nw.CHECK_LIB_PATH.exists():
        pytest.fail(f"{nw.CHECK_LIB_PATH} is missing: python nemotron-webgpu-decode_amd/build.py "
                    "--variants")


def _pair(*args, **kw):
    return nw.AttnContext(*args, **kw), nw.AttnContext(*args, lib_path=nw.CHECK_LIB_PATH, **kw)


def _bits(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.detach().contiguous().cpu().numpy().view(np.uint8)


def _same(run, prod, chk, outputs):
    """run(ctx, *outputs_copy) on both builds, each on its own copy of the
    outputs (which may be read too, as caches and accumulators are); checks
    the status words and compares every output bit for bit."""
    mine = [o.clone() for o in outputs]
    theirs = [o.clone() for o in outputs]
    run(prod, *mine)
    run(chk, *theirs)
    assert prod.device_status() == nw.NWD_OK, prod.last_error()
    assert chk.device_status() == nw.NWD_OK, chk.last_error()
    for i, (a, b) in enumerate(zip(mine, theirs)):
        assert np.array_equal(_bits(a), _bits(b)), f"output {i} differs"


@pytest.mark.parametrize("H,Hkv,lens,o_dtype,splits,separate", [
    (32, 8, (300, 4000), "f16", 0, None),
    (32, 8, (300, 4000), "f32", 7, True),
    (32, 8, (300, 4000), "f16", 7, False),
    (8, 8, (1000,), "f16", 0, None),
    (64, 8, (17, 2500), "f32", 0, None),
    (40, 8, (153,), "f16", 0, None),
    (40, 8, (3000, 3900), "f32", 0, None),  # the matrix-core split kernel
])
def test_decode_checked_build_matches(H, Hkv, lens, o_dtype, splits, separate):
    say("check build decode", H, Hkv, lens, o_dtype, splits, separate)
    B, cap = len(lens), 4096
    prod, chk = _pair(H, Hkv, cap, max_batch=B, o_dtype=o_dtype)
    with prod, chk:
        for c in (prod, chk):
            c.set_decode_splits(splits)
            c.set_decode_merge(separate)
        q = randn_f16((B, H, D), 1)
        kc = randn_f16((B, Hkv, cap, D), 2)
        vc = randn_f16((B, Hkv, cap, D), 3)
        kn = randn_f16((B, Hkv, D), 4)
        vn = randn_f16((B, Hkv, D), 5)
        pos = pos_tensor([L - 1 for L in lens])
        odt = torch.float16 if o_dtype == "f16" else torch.float32
        out = torch.zeros((B, H, D), dtype=odt, device="cuda")
        _same(lambda c, o: c.decode(q, kc, vc, pos, o, B), prod, chk, [out])
        _same(lambda c, o, k, v: c.append_decode(q, kn, vn, k, v, pos, o, B), prod, chk,
              [out, kc, vc])


@pytest.mark.parametrize("kernel,layout", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_decode_checked_build_full_workspace(kernel, layout):
    """A context whose split-K workspace is filled exactly by one call: 8
    query heads, max_seq 64, batch 1 give 2048 records, and 256 forced splits
    use all of them (most splits hold no key). Every record store is in
    bounds, so the checked build flags nothing and gives the product's bits,
    with either merge form, both split kernels and both key layouts."""
    say("check build full workspace", kernel, layout)
    H, Hkv, cap = 8, 8, 64
    prod, chk = _pair(H, Hkv, cap, o_dtype="f32")
    with prod, chk:
        assert prod.decode_splits(1, cap) >= 1
        q = randn_f16((1, H, D), 21)
        kc = randn_f16((1, Hkv, cap, D), 22)
        vc = randn_f16((1, Hkv, cap, D), 23)
        kn = randn_f16((1, Hkv, D), 24)
        vn = randn_f16((1, Hkv, D), 25)
        pos = pos_tensor([cap - 1])
        out = torch.zeros((1, H, D), dtype=torch.float32, device="cuda")
        for c in (prod, chk):
            c.set_decode_splits(256)
            c.set_decode_kernel(kernel)
            c.set_decode_layout(layout)
        assert prod.decode_splits(1, cap) == 256
        for separate in (True, False):
            for c in (prod, chk):
                c.set_decode_merge(separate)
            _same(lambda c, o: c.decode(q, kc, vc, pos, o, 1), prod, chk, [out])
            _same(lambda c, o, k, v: c.append_decode(q, kn, vn, k, v, pos, o, 1), prod, chk,
                  [out, kc, vc])


def test_kv_append_checked_build_matches():
    say("check build kv_append")
    B, n_tok, cap, Hkv = 3, 5, 64, 8
    prod, chk = _pair(32, Hkv, cap, max_batch=B)
    with prod, chk:
        kn = randn_f16((B, n_tok, Hkv, D), 6)
        vn = randn_f16((B, n_tok, Hkv, D), 7)
        kc = torch.zeros((B, Hkv, cap, D), dtype=torch.float16, device="cuda")
        pos = pos_tensor([0, 17, cap - n_tok])
        _same(lambda c, k, v: c.kv_append(kn, vn, k, v, pos, B, n_tok), prod, chk,
              [kc, kc.clone()])


@pytest.mark.parametrize("H,Hkv,pos0,n_new,o_dtype", [
    (32, 8, (0, 700), 200, "f16"),
    (32, 8, (0, 700), 200, "f32"),
    (40, 8, (1000,), 513, "f16"),
    (8, 8, (5,), 64, "f32"),
])
def test_prefill_checked_build_matches(H, Hkv, pos0, n_new, o_dtype):
    say("check build prefill", H, Hkv, pos0, n_new, o_dtype)
    B, cap = len(pos0), 2048
    prod, chk = _pair(H, Hkv, cap, max_batch=B, o_dtype=o_dtype)
    with prod, chk:
        q = randn_f16((B, n_new, H, D), 8)
        kc = randn_f16((B, Hkv, cap, D), 9)
        vc = randn_f16((B, Hkv, cap, D), 10)
        odt = torch.float16 if o_dtype == "f16" else torch.float32
        out = torch.zeros((B, n_new, H, D), dtype=odt, device="cuda")
        _same(lambda c, o: c.prefill(q, kc, vc, pos_tensor(pos0), o, B, n_new), prod, chk, [out])


def _q4(g, n, n_blocks):
    t = tuple(dev(a) for a in random_q4(g, n, n_blocks))
    return t, nw.q4_weight(*t, n, n_blocks)


def test_q4_checked_build_matches():
    say("check build q4 gemv / qkv_append / lm_head_argmax")
    g = rng(11)
    B, H, Hkv, cap, nb = 2, 32, 8, 64, 98
    prod, chk = _pair(H, Hkv, cap, max_batch=B, q_dtype="f32", o_dtype="f32", kv_dtype="f32")
    with prod, chk:
        x = dev(g.standard_normal((B, nb * 32)).astype(np.float32))
        keep = []
        t, w = _q4(g, 1024, nb)
        keep.append(t)
        y = dev(g.standard_normal((B, 1024)).astype(np.float32))
        for ep in (nw.NWD_Q4_PLAIN, nw.NWD_Q4_RELU2, nw.NWD_Q4_ACCUMULATE):
            _same(lambda c, o: c.q4_gemv(x, w, o, B, ep), prod, chk, [y])
        (tq, wq), (tk, wk), (tv, wv) = _q4(g, H * D, nb), _q4(g, Hkv * D, nb), _q4(g, Hkv * D, nb)
        keep += [tq, tk, tv]
        qo = torch.zeros((B, H * D), dtype=torch.float32, device="cuda")
        kc = torch.zeros((B, Hkv, cap, D), dtype=torch.float16, device="cuda")
        pos = pos_tensor([3, cap - 1])
        _same(lambda c, o, k, v: c.qkv_append(x, wq, wk, wv, o, k, v, pos, B), prod, chk,
              [qo, kc, kc.clone()])
        t, wl = _q4(g, 50000, nb)
        keep.append(t)
        logits = torch.zeros((B, 50000), dtype=torch.float32, device="cuda")
        ids = torch.zeros((B,), dtype=torch.int32, device="cuda")
        _same(lambda c, lg, i: c.lm_head_argmax(x, wl, i, logits=lg, batch=B), prod, chk,
              [logits, ids])
        _same(lambda c, i: c.argmax(logits, 50000, i, B), prod, chk, [ids])



@pytest.mark.parametrize("Dh,H,Hkv", [(96, 6, 2), (100, 3, 3), (300, 2, 1), (128, 7, 1), (128, 12, 4),
                                      (64, 8, 2), (256, 10, 2), (128, 32, 2), (96, 18, 2),
                                      (200, 16, 8), (64, 14, 2), (128, 12, 2), (80, 14, 2),
                                      (256, 6, 2)])
def test_general_checked_build_matches(Dh, H, Hkv):
    """The general-shape kernels in the checked build: append, decode with
    the workspace filled exactly (max_seq 64 gives H * 256 records, and 256
    forced splits use them all, most with no key), append + decode, and a
    split prefill; nothing flagged, the product build's bits. Groups 3, 6
    and 7 run the kernels built for them at head_dim 128 and 64 and the
    padded-group route at 96 and 80 (the group-4 / group-8 kernels on padded
    rows, decode and prefill); head sizes 64 and 256 the split kernel built
    for them (decode) and the MFMA prefills."""
    say("check build general", Dh, H, Hkv)
    cap, B = 64, 1
    prod, chk = _pair(H, Hkv, cap, head_dim=Dh, o_dtype="f32")
    with prod, chk:
        q = randn_f16((B, H, Dh), 31)
        kc = randn_f16((B, Hkv, cap, Dh), 32)
        vc = randn_f16((B, Hkv, cap, Dh), 33)
        kn = randn_f16((B, 3, Hkv, Dh), 34)
        vn = randn_f16((B, 3, Hkv, Dh), 35)
        pos = pos_tensor([cap - 3])
        out = torch.zeros((B, H, Dh), dtype=torch.float32, device="cuda")
        _same(lambda c, k, v: c.kv_append(kn, vn, k, v, pos, B, 3), prod, chk, [kc, vc])
        for c in (prod, chk):
            c.set_decode_splits(256)
        # 256, or what the workspace holds for padded groups' heads (H * 256
        # records over Hkv * padded group heads)
        G = H // Hkv  # padded: 9 -> 16; 3, 6, 7 where not built (3 and 6 = 2 x 3 are at 256)
        padded = G == 9 or (G in (3, 6, 7) and Dh not in (64, 128) and not (Dh == 256 and G != 7))
        if not padded:
            assert prod.decode_splits(B, cap) == 256
        assert prod.decode_splits(B, cap) > 64
        _same(lambda c, o: c.decode(q, kc, vc, pos, o, B), prod, chk, [out])
        _same(lambda c, o, k, v: c.append_decode(q, kn[:, 0], vn[:, 0], k, v, pos, o, B), prod, chk,
              [out, kc, vc])
        for c in (prod, chk):
            c.set_decode_splits(4)
        n_new = 9
        qp = randn_f16((B, n_new, H, Dh), 36)
        op = torch.zeros((B, n_new, H, Dh), dtype=torch.float32, device="cuda")
        _same(lambda c, o: c.prefill(qp, kc, vc, pos_tensor([20]), o, B, n_new), prod, chk, [op])

def test_asan_host_driver_on_gpu():
    """Host code under AddressSanitizer, with the kernels running: one
    context per group (and two general shapes) through every entry point,
    then released. Leak
    checking is off here: the HIP runtime keeps allocations until exit."""
    if not ASAN_DRIVER.exists():
        pytest.fail(f"{ASAN_DRIVER} is missing: python nemotron-webgpu-decode_amd/build.py "
                    "--variants")
    say("asan host driver: gpu mode")
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1")
    res = subprocess.run([str(ASAN_DRIVER), "gpu"], capture_output=True, text=True, timeout=100,
                         env=env)
    print(res.stdout[-2000:], res.stderr[-4000:], flush=True)
    assert res.returncode == 0, res.stderr[-4000:]
    assert "AddressSanitizer" not in res.stderr
    assert "gpu cycle group 8 head_dim 128" in res.stdout
    assert "gpu cycle group 3 head_dim 96" in res.stdout  # the padded-group route
    assert "gpu cycle group 7 head_dim 80" in res.stdout
    assert "gpu cycle group 7 head_dim 64" in res.stdout  # groups 3, 6, 7 built at 64
    assert "gpu cycle group 2 head_dim 100" in res.stdout  # the general kernels' host paths
    assert "gpu cycle group 7 head_dim 128" in res.stdout  # groups 3, 6, 7 built at 128
    assert "gpu cycle group 6 head_dim 128" in res.stdout
    assert "gpu cycle group 4 head_dim 64" in res.stdout  # the split kernel at other head sizes
    assert "gpu cycle group 5 head_dim 256" in res.stdout
    assert "gpu cycle group 12 head_dim 96" in res.stdout  # padded to 16: two groups of 8
    assert "0 failed so far" in res.stdout.splitlines()[-1]
