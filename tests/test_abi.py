"""The C ABI library loads and exports what include/nwd_attn.h declares, and
its host-side validation rejects bad arguments before touching the GPU.
No kernel is launched here (these run without a GPU)."""
import ctypes

import pytest

import nwd_attn as nw


@pytest.fixture(scope="module")
def lib():
    return nw.load_library()


def test_exports_every_declared_function(lib):
    names = nw.header_functions()
    assert len(names) >= 11
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_header_declares_every_bound_function():
    # the ctypes binding covers the whole header and nothing beyond it
    import inspect
    src = inspect.getsource(nw.load_library)
    for n in nw.header_functions():
        assert f'"{n}"' in src, n


def _desc(**kw):
    d = dict(n_heads=32, n_kv_heads=8, head_dim=128, max_seq=4096, max_batch=1,
             q_dtype=nw.NWD_F16, o_dtype=nw.NWD_F16, kv_dtype=nw.NWD_F16, scale=0.0)
    d.update(kw)
    return nw.NwdDesc(**d)


@pytest.mark.parametrize("kw,code", [
    (dict(n_heads=0), nw.NWD_ERR_INVALID),
    (dict(n_kv_heads=-1), nw.NWD_ERR_INVALID),
    (dict(n_heads=30), nw.NWD_ERR_INVALID),          # not a multiple of 8
    (dict(head_dim=0), nw.NWD_ERR_INVALID),
    (dict(head_dim=513), nw.NWD_ERR_UNSUPPORTED),    # past the general kernels' 512
    (dict(max_seq=0), nw.NWD_ERR_INVALID),
    (dict(max_seq=(1 << 22) + 1), nw.NWD_ERR_UNSUPPORTED),  # slab byte offsets need 31 bits
    (dict(max_batch=0), nw.NWD_ERR_INVALID),
    (dict(q_dtype=7), nw.NWD_ERR_INVALID),
    (dict(scale=-1.0), nw.NWD_ERR_INVALID),
    (dict(scale=float("nan")), nw.NWD_ERR_INVALID),
])
def test_create_rejects_bad_descriptors(lib, kw, code):
    h = ctypes.c_void_p(1234)
    rc = lib.nwd_create(ctypes.byref(_desc(**kw)), ctypes.byref(h))
    assert rc == code
    assert h.value is None
    assert lib.nwd_last_error(None).decode().startswith("nwd_create")


def test_null_arguments(lib):
    assert lib.nwd_create(None, None) == nw.NWD_ERR_INVALID
    h = ctypes.c_void_p()
    assert lib.nwd_create(None, ctypes.byref(h)) == nw.NWD_ERR_INVALID
    assert lib.nwd_kv_append(None, None, None, None, None, None, 1, 1, None) == nw.NWD_ERR_INVALID
    assert lib.nwd_decode_attn(None, None, None, None, None, None, 1, 0, None) == nw.NWD_ERR_INVALID
    assert lib.nwd_prefill_attn(None, None, None, None, None, None, 1, 1, 0, None) == nw.NWD_ERR_INVALID
    assert lib.nwd_device_status(None, None) == nw.NWD_ERR_INVALID
    assert lib.nwd_set_decode_splits(None, 3) == nw.NWD_ERR_INVALID
    assert lib.nwd_cache_bytes(None) == 0
    assert lib.nwd_cache_offset(None, 0, 0, 0, 0) == -1
    assert lib.nwd_decode_splits(None, 1, 100) == 0
    lib.nwd_destroy(None)
    assert isinstance(lib.nwd_last_error(None), bytes)


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="build the HIP library"):
        nw.load_library(tmp_path / "libnwd_attn.so")


def test_library_matches_the_sources_on_disk(lib):
    """nwd_source_hash() of the built library equals the hash of csrc/ and
    include/nwd_attn.h as they are now, so the tested library is the one these
    sources build (build.py embeds it at compile time)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("nwd_build_for_hash", nw.PKG_DIR / "build.py")
    build = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(build)
    assert nw.source_hash(lib) == build.source_hash(), "rebuild: python nemotron-webgpu-decode_amd/build.py"
    assert len(nw.source_hash(lib)) == 64


@pytest.mark.parametrize("kw", [dict(n_heads=24), dict(n_heads=96), dict(head_dim=64),
                                dict(head_dim=100), dict(head_dim=512), dict(n_heads=8, n_kv_heads=8,
                                                                              head_dim=1)])
def test_general_shapes_pass_validation(lib, kw):
    """Any group (24/8 = 3, 96/8 = 12) and any head size up to 512 pass the
    descriptor checks (the reference's Params take both,
    kernels/sparse_attn.wgsl:12-17). nwd_create then gets as far as the
    device: without a GPU it fails there, not on the shape."""
    h = ctypes.c_void_p(1234)
    rc = lib.nwd_create(ctypes.byref(_desc(**kw)), ctypes.byref(h))
    assert rc not in (nw.NWD_ERR_INVALID, nw.NWD_ERR_UNSUPPORTED), lib.nwd_last_error(None)


def test_noalloc_accepts_general_shapes(lib):
    """The allocation-free entry point takes the general shapes too: its split
    records (at most ~2048 of head_dim floats for them) always fit the 16 MiB
    scratch, even at head_dim 512, so the call gets past every host check to
    the device (which this container lacks)."""
    p = ctypes.c_void_p(8)
    for kw in (dict(head_dim=512, n_heads=64, n_kv_heads=8, max_batch=64),
               dict(head_dim=64, n_heads=6, n_kv_heads=2, max_batch=1)):
        d = _desc(max_seq=32768, **kw)
        rc = lib.nwd_append_decode_noalloc(ctypes.byref(d), p, p, p, p, p, p, p, d.max_batch, 32768,
                                           None, None)
        assert rc not in (nw.NWD_ERR_INVALID, nw.NWD_ERR_UNSUPPORTED, nw.NWD_ERR_CAPACITY), \
            lib.nwd_last_error(None)
