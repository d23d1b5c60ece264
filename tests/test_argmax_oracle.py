"""Pins the greedy-pick oracle (oracle/argmax_oracle.c, a restatement of
kernels/argmax_partial.wgsl + kernels/argmax_merge.wgsl as dispatched at
engine/runtime.js:398-399) against two statements that do not share its
code: a pure-Python emulation of the two WGSL kernels (small n), and the
closed-form rule in argmax_cases.py (any n). CPU only."""
import numpy as np
import pytest

import oracle
from argmax_cases import NEG_FLT_MAX, reference_rule, tie_heavy

F32 = np.float32


def _emulate_wgsl(x):
    """The two WGSL kernels as written, in plain Python (small n only)."""
    n = len(x)
    WG, N_WG = 256, 256
    n_slice = (n + N_WG - 1) // N_WG
    neg = F32(NEG_FLT_MAX)
    parts = []
    for wg in range(N_WG):
        start = wg * n_slice
        end = min(start + n_slice, n)
        bv, bi = [neg] * WG, [start] * WG
        for tid in range(WG):
            i = start + tid
            while i < end:
                if x[i] > bv[tid]:
                    bv[tid], bi[tid] = x[i], i
                i += WG
        stride = WG // 2
        while stride:
            for tid in range(stride):
                if bv[tid + stride] > bv[tid]:
                    bv[tid], bi[tid] = bv[tid + stride], bi[tid + stride]
            stride //= 2
        parts.append((bv[0], bi[0]))
    bv, bi = [neg] * WG, [0] * WG
    for tid in range(WG):
        if parts[tid][0] > bv[tid]:
            bv[tid], bi[tid] = parts[tid]
    stride = WG // 2
    while stride:
        for tid in range(stride):
            if bv[tid + stride] > bv[tid]:
                bv[tid], bi[tid] = bv[tid + stride], bi[tid + stride]
        stride //= 2
    return bi[0]


@pytest.mark.parametrize("n", [1, 2, 7, 255, 256, 257, 600, 1000])
def test_matches_python_emulation(n):
    g = np.random.Generator(np.random.PCG64(n))
    for trial in range(4):
        x = tie_heavy(g, n) if trial % 2 else g.standard_normal(n).astype(F32)
        assert oracle.argmax_ref(x) == _emulate_wgsl(list(x)), (n, trial)


@pytest.mark.parametrize("n", [1, 300, 4097, 131072])
def test_matches_closed_form_rule(n):
    g = np.random.Generator(np.random.PCG64(7 + n))
    for trial in range(6):
        x = tie_heavy(g, n) if trial % 2 else g.standard_normal(n).astype(F32)
        assert oracle.argmax_ref(x) == reference_rule(x), (n, trial)


def test_unique_maximum_is_numpy_argmax():
    g = np.random.Generator(np.random.PCG64(3))
    x = g.standard_normal(131072).astype(F32)
    assert oracle.argmax_ref(x) == int(np.argmax(x))


def test_special_values():
    x = np.full(1000, np.nan, F32)
    assert oracle.argmax_ref(x) == 0                      # nothing qualifies
    x[:] = -np.inf
    assert oracle.argmax_ref(x) == 0
    x[:] = F32(NEG_FLT_MAX)
    assert oracle.argmax_ref(x) == 0                      # must be strictly above
    x[123] = np.nextafter(F32(NEG_FLT_MAX), F32(0))
    assert oracle.argmax_ref(x) == 123
    x[500] = np.inf
    x[7] = np.nan
    assert oracle.argmax_ref(x) == 500


def test_tie_order_is_the_trees_not_the_lowest_index():
    """n = 131072: slices of 512, thread tid visits start + tid and
    start + 256 + tid. A tie between index 256 (thread 0, second step) and
    index 1 (thread 1, first step) goes to 256; between slice 0 and slice 1
    to slice 0; between slice 6 and slice 128 to slice 128 (bit-reversed 1 <
    96). A lowest-index rule would say 1, 1 and slice 6."""
    x = np.zeros(131072, F32)
    x[1] = x[256] = 5.0
    assert oracle.argmax_ref(x) == 256 == reference_rule(x)
    assert int(np.argmax(x)) == 1
    x[512 + 3] = 5.0
    assert oracle.argmax_ref(x) == 256 == reference_rule(x)
    y = np.zeros(131072, F32)
    y[6 * 512 + 10] = y[128 * 512 + 20] = 1.0
    assert oracle.argmax_ref(y) == 128 * 512 + 20 == reference_rule(y)
