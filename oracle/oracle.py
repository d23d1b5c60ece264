"""ctypes binding of oracle/liboracle.so — TEST INFRASTRUCTURE ONLY.

The oracle is what the HIP library's results are checked against. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this module.
Each wrapped function cites the reference file:line its C code restates (see
attn_oracle.c). Inputs are numpy arrays in the reference's layouts:
Q/O [n_heads][head_dim] and K/V token-major [seq][n_kv_heads][head_dim];
4-bit weights as quant uint8 [N][n_blocks][16], scales float32 [N][n_blocks]
and packed zero points uint8 [ceil(N * n_blocks / 2)] (q4_oracle.c).
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"

_lib = None


def build() -> Path:
    """Compiles liboracle.so with oracle/Makefile."""
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    return LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    P = np.ctypeslib.ndpointer
    f32 = P(dtype=np.float32, flags="C_CONTIGUOUS")
    f64 = P(dtype=np.float64, flags="C_CONTIGUOUS")
    u16 = P(dtype=np.uint16, flags="C_CONTIGUOUS")
    u32, i64 = ctypes.c_uint32, ctypes.c_int64
    lib.oracle_f16_to_f32.argtypes = [u16, f32, i64]
    lib.oracle_f16_to_f32.restype = None
    lib.oracle_f32_to_f16.argtypes = [f32, u16, i64]
    lib.oracle_f32_to_f16.restype = None
    lib.oracle_kv_append_f32.argtypes = [f32, f32, u32, u32, u32]
    lib.oracle_kv_append_f32.restype = None
    lib.oracle_sparse_attn_f32.argtypes = [f32, f32, f32, f32, u32, u32, u32, u32]
    lib.oracle_sparse_attn_f32.restype = ctypes.c_int
    lib.oracle_sparse_attn_f32_mt.argtypes = [f32, f32, f32, f32, u32, u32, u32, u32, ctypes.c_int]
    lib.oracle_sparse_attn_f32_mt.restype = ctypes.c_int
    lib.oracle_attn_f64.argtypes = [f32, f32, f32, f64, u32, u32, u32, u32, ctypes.c_double]
    lib.oracle_attn_f64.restype = ctypes.c_int
    lib.oracle_max_threads.argtypes = []
    lib.oracle_max_threads.restype = ctypes.c_int
    u8 = P(dtype=np.uint8, flags="C_CONTIGUOUS")
    lib.oracle_q4_gemv_f32.argtypes = [f32, u8, f32, u8, f32, u32, u32, u32, u32, ctypes.c_int]
    lib.oracle_q4_gemv_f32.restype = ctypes.c_int
    lib.oracle_q4_dequant.argtypes = [u8, f32, u8, f32, u32, u32]
    lib.oracle_q4_dequant.restype = None
    lib.oracle_argmax_ref.argtypes = [f32, u32]
    lib.oracle_argmax_ref.restype = ctypes.c_uint32
    _lib = lib
    return lib


def max_threads() -> int:
    return int(_load().oracle_max_threads())


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    """binary16 bit patterns -> float32 (exact). attn_oracle.c half_to_float."""
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    _load().oracle_f16_to_f32(b.reshape(-1), out.reshape(-1), b.size)
    return out


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    """float32 -> binary16 bit patterns, round to nearest even."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(a.shape, np.uint16)
    _load().oracle_f32_to_f16(a.reshape(-1), out.reshape(-1), a.size)
    return out


def kv_append_f32(src: np.ndarray, cache: np.ndarray, seq: int, n_kv: int, hd: int) -> None:
    """kernels/kv_append.wgsl:12-18 on a flat f32 cache, in place."""
    assert cache.dtype == np.float32 and cache.flags.c_contiguous
    assert (seq + 1) * n_kv * hd <= cache.size
    _load().oracle_kv_append_f32(np.ascontiguousarray(src, np.float32).reshape(-1),
                                 cache.reshape(-1), seq, n_kv, hd)


def sparse_attn_f32(q: np.ndarray, k: np.ndarray, v: np.ndarray, threads: int = 1) -> np.ndarray:
    """kernels/sparse_attn.wgsl:31-114 op for op in f32 (no 256-key cap).

    q [H][D], k/v [L][Hkv][D] -> O [H][D] float32. threads > 1 (or 0 = all)
    spreads the per-head workgroups over OpenMP threads; same result."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    H, D = q.shape
    L, Hkv, Dk = k.shape
    assert Dk == D and v.shape == k.shape
    o = np.empty((H, D), np.float32)
    lib = _load()
    if threads == 1:
        rc = lib.oracle_sparse_attn_f32(q, k, v, o, H, Hkv, D, L)
    else:
        rc = lib.oracle_sparse_attn_f32_mt(q, k, v, o, H, Hkv, D, L, threads)
    if rc != 0:
        raise ValueError("oracle_sparse_attn_f32: seq == 0 or heads do not divide")
    return o


def attn_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float = 0.0) -> np.ndarray:
    """Double-precision softmax(q.K^T*scale).V, same layouts; scale 0 = 1/sqrt(D)."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    H, D = q.shape
    L, Hkv, _ = k.shape
    o = np.empty((H, D), np.float64)
    rc = _load().oracle_attn_f64(q, k, v, o, H, Hkv, D, L, float(scale))
    if rc != 0:
        raise ValueError("oracle_attn_f64: seq == 0 or heads do not divide")
    return o


def q4_gemv_f32(a: np.ndarray, quant: np.ndarray, scales: np.ndarray, zp: np.ndarray,
                epilogue: int = 0, threads: int = 1) -> np.ndarray:
    """kernels/matmul_nbits_sg.wgsl:81-137 op for op in f32: Y[N] =
    epilogue(dequant(W) . a). a [K] float32, K = 32 * n_blocks; epilogue 1 =
    relu2. threads > 1 spreads the workgroups over OpenMP threads (same
    result)."""
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    quant = np.ascontiguousarray(quant, np.uint8)
    scales = np.ascontiguousarray(scales, np.float32)
    zp = np.ascontiguousarray(zp, np.uint8).reshape(-1)
    N, n_blocks = scales.shape
    assert quant.shape == (N, n_blocks, 16) and a.size == 32 * n_blocks
    assert zp.size * 2 >= N * n_blocks
    y = np.empty(N, np.float32)
    rc = _load().oracle_q4_gemv_f32(a, quant.reshape(-1), scales.reshape(-1), zp, y, a.size, N,
                                    n_blocks, epilogue, threads)
    if rc != 0:
        raise ValueError("oracle_q4_gemv_f32: K != 32 * n_blocks")
    return y


def q4_dequant(quant: np.ndarray, scales: np.ndarray, zp: np.ndarray) -> np.ndarray:
    """(nib - zp) * scale of every weight, [N][K] float32, as dequant_dot forms it."""
    quant = np.ascontiguousarray(quant, np.uint8)
    scales = np.ascontiguousarray(scales, np.float32)
    zp = np.ascontiguousarray(zp, np.uint8).reshape(-1)
    N, n_blocks = scales.shape
    assert quant.shape == (N, n_blocks, 16) and zp.size * 2 >= N * n_blocks
    w = np.empty((N, 32 * n_blocks), np.float32)
    _load().oracle_q4_dequant(quant.reshape(-1), scales.reshape(-1), zp, w, N, n_blocks)
    return w


def argmax_ref(x: np.ndarray) -> int:
    """kernels/argmax_partial.wgsl:16-52 (256 workgroups over ceil(n / 256)
    slices) then kernels/argmax_merge.wgsl:8-42, op for op: the token index
    the reference picks from logits x [n]."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    assert x.size >= 1
    return int(_load().oracle_argmax_ref(x, x.size))
