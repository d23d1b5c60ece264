"""ctypes binding of libnwd_attn.so (the C ABI in include/nwd_attn.h).

Used by the tests and by bench.py to drive the HIP library from Python; the
engine-facing host is the Node.js module in js/. Buffers are passed as device
addresses (ints) or as objects with a ``data_ptr()`` method (torch tensors),
so this module itself needs no torch.

The library is required: there is no fallback path. ``load_library`` raises
if lib/libnwd_attn.so has not been built (``python build.py``).
"""
from __future__ import annotations

import ctypes
import os
import re
from pathlib import Path
from typing import Optional

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "lib" / "libnwd_attn.so"
# debug build of the same sources with -DNWD_CHECK (build.py --variants):
# every kernel store checks its address and flags NWD_ERR_DEVICE if outside
CHECK_LIB_PATH = PKG_DIR / "lib" / "check" / "libnwd_attn.so"
HEADER_PATH = PKG_DIR.parent / "include" / "nwd_attn.h"

NWD_OK = 0
NWD_ERR_INVALID = 1
NWD_ERR_UNSUPPORTED = 2
NWD_ERR_CAPACITY = 3
NWD_ERR_HIP = 4
NWD_ERR_DEVICE = 5

NWD_F32 = 0
NWD_F16 = 1
_DTYPES = {"f32": NWD_F32, "float32": NWD_F32, "f16": NWD_F16, "float16": NWD_F16}


class NwdDesc(ctypes.Structure):
    _fields_ = [
        ("n_heads", ctypes.c_int32),
        ("n_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("max_seq", ctypes.c_int32),
        ("max_batch", ctypes.c_int32),
        ("q_dtype", ctypes.c_int32),
        ("o_dtype", ctypes.c_int32),
        ("kv_dtype", ctypes.c_int32),
        ("scale", ctypes.c_float),
    ]


NWD_Q4_PLAIN = 0
NWD_Q4_RELU2 = 1
NWD_Q4_ACCUMULATE = 2


class NwdQ4Weight(ctypes.Structure):
    """nwd_q4_weight: one 4-bit projection [K -> n] in the reference's
    MatMulNBits format (engine/weights.js:99-104)."""
    _fields_ = [
        ("quant", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("zp", ctypes.c_void_p),
        ("n", ctypes.c_int32),
        ("n_blocks", ctypes.c_int32),
    ]


def q4_weight(quant, scales, zp, n: int, n_blocks: int) -> NwdQ4Weight:
    """Descriptor of device buffers (addresses or tensors)."""
    return NwdQ4Weight(_ptr(quant), _ptr(scales), _ptr(zp), n, n_blocks)


class NwdError(RuntimeError):
    """A non-zero status from the C ABI, with the library's message."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[nwd status {code}] {message}")
        self.code = code
        self.message = message


_lib: Optional[ctypes.CDLL] = None


def header_functions() -> list[str]:
    """Names of the functions include/nwd_attn.h declares."""
    text = HEADER_PATH.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nwd_[a-z_0-9]+)\s*\(", text)))


def load_library(path: Optional[os.PathLike] = None) -> ctypes.CDLL:
    """Loads libnwd_attn.so (once) and declares the C signatures."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"{p} is missing: build the HIP library first "
            "(python nemotron-webgpu-decode_amd/build.py)")
    lib = ctypes.CDLL(str(p))
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    sig = {
        "nwd_create": (ctypes.c_int, [ctypes.POINTER(NwdDesc), ctypes.POINTER(vp)]),
        "nwd_destroy": (None, [vp]),
        "nwd_last_error": (ctypes.c_char_p, [vp]),
        "nwd_source_hash": (ctypes.c_char_p, []),
        "nwd_cache_bytes": (ctypes.c_size_t, [vp]),
        "nwd_cache_offset": (i64, [vp, i32, i32, i32, i32]),
        "nwd_kv_append": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, i32, i32, vp]),
        "nwd_decode_attn": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, i32, i32, vp]),
        "nwd_append_decode": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, vp]),
        "nwd_append_decode_noalloc": (ctypes.c_int, [ctypes.POINTER(NwdDesc), vp, vp, vp, vp, vp,
                                                     vp, vp, i32, i32, vp, vp]),
        "nwd_prefill_attn": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, i32, i32, i32, vp]),
        "nwd_device_status": (ctypes.c_int, [vp, vp]),
        "nwd_decode_splits": (i32, [vp, i32, i32]),
        "nwd_set_decode_splits": (ctypes.c_int, [vp, i32]),
        "nwd_set_decode_merge": (ctypes.c_int, [vp, i32]),
        "nwd_set_decode_kernel": (ctypes.c_int, [vp, i32]),
        "nwd_set_decode_layout": (ctypes.c_int, [vp, i32]),
        "nwd_set_kernel_events": (ctypes.c_int, [vp, vp, vp]),
        "nwd_q4_gemv": (ctypes.c_int, [vp, vp, ctypes.POINTER(NwdQ4Weight), vp, i32, i32, vp]),
        "nwd_qkv_append": (ctypes.c_int, [vp, vp, ctypes.POINTER(NwdQ4Weight),
                                          ctypes.POINTER(NwdQ4Weight), ctypes.POINTER(NwdQ4Weight),
                                          vp, vp, vp, vp, i32, vp]),
        "nwd_argmax": (ctypes.c_int, [vp, vp, i32, vp, i32, vp]),
        "nwd_lm_head_argmax": (ctypes.c_int, [vp, vp, ctypes.POINTER(NwdQ4Weight), vp, vp, i32,
                                              vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def source_hash(lib: Optional[ctypes.CDLL] = None) -> str:
    """nwd_source_hash() of the loaded library (the hash of the sources it
    was built from; build.source_hash() gives that of the sources on disk)."""
    return (lib or load_library()).nwd_source_hash().decode()


_others: dict = {}


def _load_other(path: os.PathLike) -> ctypes.CDLL:
    """A second build of the library, loaded once per path beside the first
    (ctypes loads it with local symbol binding, so the builds stay apart)."""
    key = str(Path(path).resolve())
    if key not in _others:
        _others[key] = load_library(path)
    return _others[key]


def _ptr(x) -> Optional[int]:
    if x is None:
        return None
    if isinstance(x, int):
        return x
    dp = getattr(x, "data_ptr", None)
    if dp is not None:
        return int(dp())
    raise TypeError(f"expected a device address or a tensor, got {type(x).__name__}")


def _stream(s) -> Optional[int]:
    if s is None or s == 0:
        return None
    if isinstance(s, int):
        return s
    handle = getattr(s, "cuda_stream", None)  # torch.cuda.Stream
    if handle is not None:
        return int(handle)
    raise TypeError("stream must be an int handle or a torch.cuda.Stream")


def append_decode_noalloc(desc: NwdDesc, q, k_new, v_new, k_cache, v_cache, pos, out,
                          batch: int, max_len: int = 0, status=None, stream=None):
    """nwd_append_decode_noalloc: nwd_append_decode without a context, its
    split-K records in the library's static device scratch (no allocation)."""
    lib = load_library()
    rc = lib.nwd_append_decode_noalloc(ctypes.byref(desc), _ptr(q), _ptr(k_new), _ptr(v_new),
                                       _ptr(k_cache), _ptr(v_cache), _ptr(pos), _ptr(out), batch,
                                       max_len, _ptr(status), _stream(stream))
    if rc != NWD_OK:
        raise NwdError(rc, lib.nwd_last_error(None).decode())


class AttnContext:
    """One nwd_ctx: shapes, dtypes and the split-K workspace.

    Mirrors the attention slice of the reference engine: the descriptor is
    the Params uniform {n_heads, n_kv_heads, head_dim, seq}
    (kernels/sparse_attn.wgsl:12-17) plus allocation sizes
    (engine/runtime.js:170-173,182-183).
    """

    def __init__(self, n_heads: int, n_kv_heads: int, max_seq: int, *, head_dim: int = 128,
                 max_batch: int = 1, q_dtype: str = "f16", o_dtype: str = "f16",
                 kv_dtype: str = "f16", scale: float = 0.0,
                 lib_path: Optional[os.PathLike] = None):
        # lib_path: another build of the library (e.g. CHECK_LIB_PATH)
        self.lib = load_library() if lib_path is None else _load_other(lib_path)
        self.desc = NwdDesc(n_heads, n_kv_heads, head_dim, max_seq, max_batch,
                            _DTYPES[q_dtype], _DTYPES[o_dtype], _DTYPES[kv_dtype], scale)
        h = ctypes.c_void_p()
        rc = self.lib.nwd_create(ctypes.byref(self.desc), ctypes.byref(h))
        if rc != NWD_OK:
            raise NwdError(rc, self.lib.nwd_last_error(None).decode())
        self.handle = h

    # ---------------------------------------------------------------- helpers
    def _check(self, rc: int):
        if rc != NWD_OK:
            raise NwdError(rc, self.lib.nwd_last_error(self.handle).decode())

    def close(self):
        if getattr(self, "handle", None):
            self.lib.nwd_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def cache_bytes(self) -> int:
        return int(self.lib.nwd_cache_bytes(self.handle))

    def cache_offset(self, b: int, t: int, h: int, d: int) -> int:
        return int(self.lib.nwd_cache_offset(self.handle, b, t, h, d))

    def decode_splits(self, batch: int, max_len: int) -> int:
        return int(self.lib.nwd_decode_splits(self.handle, batch, max_len))

    def set_decode_splits(self, n: int):
        self._check(self.lib.nwd_set_decode_splits(self.handle, n))

    def set_decode_merge(self, separate_kernel):
        """True: merge split-K records in a second kernel; False: in the split
        kernel's last workgroup; None: the default (the separate kernel)."""
        v = -1 if separate_kernel is None else int(bool(separate_kernel))
        self._check(self.lib.nwd_set_decode_merge(self.handle, v))

    def set_decode_kernel(self, kernel):
        """0: the dot-product (VALU) split kernel; 1: the matrix-core (MFMA)
        one; None: the default choice (by group size and keys per split)."""
        self._check(self.lib.nwd_set_decode_kernel(self.handle, -1 if kernel is None else int(kernel)))

    def set_decode_layout(self, layout):
        """0: each split owns one contiguous key range; 1: split s owns the
        key blocks s, s + n_splits, ...; None: the default choice."""
        self._check(self.lib.nwd_set_decode_layout(self.handle, -1 if layout is None else int(layout)))

    def set_kernel_events(self, start, stop):
        """hipEvent_t handles (ints) recorded around every later decode call's
        split kernel; None, None turns it off."""
        self._check(self.lib.nwd_set_kernel_events(self.handle, start, stop))

    # ------------------------------------------------------------ operations
    def kv_append(self, k_new, v_new, k_cache, v_cache, pos, batch: int, n_tokens: int = 1,
                  stream=None):
        """kernels/kv_append.wgsl:12-18 for K and V in one launch."""
        self._check(self.lib.nwd_kv_append(self.handle, _ptr(k_new), _ptr(v_new), _ptr(k_cache),
                                           _ptr(v_cache), _ptr(pos), batch, n_tokens,
                                           _stream(stream)))

    def decode(self, q, k_cache, v_cache, pos, out, batch: int, max_len: int = 0, stream=None):
        """kernels/sparse_attn.wgsl:31-114 with L_b = pos[b] + 1 keys."""
        self._check(self.lib.nwd_decode_attn(self.handle, _ptr(q), _ptr(k_cache), _ptr(v_cache),
                                             _ptr(pos), _ptr(out), batch, max_len,
                                             _stream(stream)))

    def append_decode(self, q, k_new, v_new, k_cache, v_cache, pos, out, batch: int,
                      max_len: int = 0, stream=None):
        """kv_append (K, V) + sparse_attn of engine/runtime.js:389-391, fused."""
        self._check(self.lib.nwd_append_decode(self.handle, _ptr(q), _ptr(k_new), _ptr(v_new),
                                               _ptr(k_cache), _ptr(v_cache), _ptr(pos), _ptr(out),
                                               batch, max_len, _stream(stream)))

    def prefill(self, q, k_cache, v_cache, pos0, out, batch: int, n_new: int, max_len: int = 0,
                stream=None):
        """Token-by-token prefill of engine/runtime.js:640-643 as one causal chunk."""
        self._check(self.lib.nwd_prefill_attn(self.handle, _ptr(q), _ptr(k_cache), _ptr(v_cache),
                                              _ptr(pos0), _ptr(out), batch, n_new, max_len,
                                              _stream(stream)))

    def q4_gemv(self, a, w: NwdQ4Weight, y, batch: int = 1, epilogue: int = NWD_Q4_PLAIN,
                stream=None):
        """kernels/matmul_nbits_sg.wgsl:81-137 for `batch` rows; epilogue
        NWD_Q4_RELU2 (its epilogue 1) or NWD_Q4_ACCUMULATE (y += W.a, the
        residual add of kernels/add.wgsl fused)."""
        self._check(self.lib.nwd_q4_gemv(self.handle, _ptr(a), ctypes.byref(w), _ptr(y), batch,
                                         epilogue, _stream(stream)))

    def qkv_append(self, x, wq: NwdQ4Weight, wk: NwdQ4Weight, wv: NwdQ4Weight, q_out, k_cache,
                   v_cache, pos, batch: int = 1, stream=None):
        """The q/k/v projections and kv_append of engine/runtime.js:386-390 in one launch."""
        self._check(self.lib.nwd_qkv_append(self.handle, _ptr(x), ctypes.byref(wq),
                                            ctypes.byref(wk), ctypes.byref(wv), _ptr(q_out),
                                            _ptr(k_cache), _ptr(v_cache), _ptr(pos), batch,
                                            _stream(stream)))

    def argmax(self, x, n: int, out, batch: int = 1, stream=None):
        """kernels/argmax_partial.wgsl + argmax_merge.wgsl (engine/runtime.js:398-399)."""
        self._check(self.lib.nwd_argmax(self.handle, _ptr(x), n, _ptr(out), batch, _stream(stream)))

    def lm_head_argmax(self, h, w: NwdQ4Weight, out, logits=None, batch: int = 1, stream=None):
        """lm-head + argmax0 + argmax1 of engine/runtime.js:397-399 in two launches."""
        self._check(self.lib.nwd_lm_head_argmax(self.handle, _ptr(h), ctypes.byref(w),
                                                _ptr(logits), _ptr(out), batch, _stream(stream)))

    def device_status(self, stream=None) -> int:
        """Synchronises and returns the status code (raises nothing)."""
        return int(self.lib.nwd_device_status(self.handle, _stream(stream)))

    def last_error(self) -> str:
        return self.lib.nwd_last_error(self.handle).decode()
