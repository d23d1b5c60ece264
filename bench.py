"""Benchmark of the decode-attention path on one MI355X.

One "step" is one attention-layer step of the reference engine
(engine/runtime.js:389-391: kv_append for K, for V, then sparse_attn): here
one nwd_append_decode call that writes the new token's K and V rows and
attends over pos+1 keys.

The headline (the JSON line's `value`, `ms_per_step`, `roofline`,
`cpu_baseline`) is the decode-32k workload: batch 1, 32 query heads, 8 KV
heads, head_dim 128, fp16 cache, 32768 cached tokens with 1% of K/V entries
at +-8, one token appended and attended per step. To keep the 256 MB
Infinity Cache from serving the KV reads, step s uses layer cache s % 4 of 4
distinct caches (537 MB), the way a model walks its layers, and token
(s // 4) % 64 of a 64-token window. The other four workloads of the
benchmark specification (decode-153, decode-4k, ragged-64, prefill-512) and
the read ceiling of the same access pattern (stream-read) are measured in the
same run and reported under `configs` and `stream_read`, each with its own
roofline block.

Inputs are resident in HBM before timing starts and steps are replayed from
HIP graphs (captured once), timed with hipEvents on the stream the kernels
run on. Prints ONE JSON line.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]
       python bench.py --workload NAME    (one workload, for profiling)
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "nemotron-webgpu-decode_amd"))

METRIC = "µs/attention-layer step + achieved KV-read GB/s (% of HBM peak), 1×MI355X"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
H, HKV, D = 32, 8, 128
BENCH_LIB = ROOT / "nemotron-webgpu-decode_amd" / "lib" / "libnwd_bench.so"


def kv_bytes(L: int) -> int:
    """Algorithmic KV-read bytes of one decode over L keys: L*Hkv*D*(K+V)*2 B."""
    return L * HKV * D * 2 * 2


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Hip:
    """The few HIP runtime calls bench.py makes directly (events around the
    split kernel, see nwd_set_kernel_events)."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so")
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.lib.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                 ctypes.c_void_p]

    def event(self) -> int:
        e = ctypes.c_void_p()
        if self.lib.hipEventCreate(ctypes.byref(e)) != 0:
            raise RuntimeError("hipEventCreate failed")
        return e.value

    def elapsed_ms(self, a: int, b: int) -> float:
        if self.lib.hipEventSynchronize(b) != 0:
            raise RuntimeError("hipEventSynchronize failed")
        ms = ctypes.c_float()
        if self.lib.hipEventElapsedTime(ctypes.byref(ms), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def destroy(self, e: int):
        self.lib.hipEventDestroy(e)


class DecodeWorkload:
    """`layers` distinct caches of `past` random tokens plus `window` tokens
    of new rows and queries, all on the device. K/V are N(0,1), times a
    per-KV-head scale drawn U[0.5, 2] (`dist="head-scale"`), or with 1% of
    entries replaced by +-8 (`dist="outliers"`)."""

    def __init__(self, torch, nw, past: int, window: int, layers: int, seed: int,
                 dist: str = "normal", heads: int = H):
        self.torch, self.past, self.window, self.layers = torch, past, window, layers
        self.heads = heads
        self.cap = past + window
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        f16 = torch.float16

        def rnd(*shape):
            return torch.randn(*shape, generator=g, device="cuda", dtype=torch.float32).to(f16)

        # one scale per KV head for K and one for V (caches and new rows alike)
        hs_k = torch.rand(HKV, generator=g, device="cuda") * 1.5 + 0.5
        hs_v = torch.rand(HKV, generator=g, device="cuda") * 1.5 + 0.5

        def kv(shape, hs, head_axis):
            x = torch.randn(*shape, generator=g, device="cuda", dtype=torch.float32)
            if dist == "head-scale":
                x *= hs.view(HKV, *([1] * (len(shape) - head_axis - 1)))
            elif dist == "outliers":
                hit = torch.rand(*shape, generator=g, device="cuda") < 0.01
                sign = torch.randint(0, 2, shape, generator=g, device="cuda") * 2 - 1
                x = torch.where(hit, 8.0 * sign, x)
            return x.to(f16)

        self.kc = [kv((1, HKV, self.cap, D), hs_k, 1) for _ in range(layers)]
        self.vc = [kv((1, HKV, self.cap, D), hs_v, 1) for _ in range(layers)]
        self.knew = kv((window, 1, HKV, D), hs_k, 2)
        self.vnew = kv((window, 1, HKV, D), hs_v, 2)
        self.q = rnd(window, 1, heads, D)
        self.out = torch.empty(1, heads, D, dtype=f16, device="cuda")
        self.pos = torch.arange(past, past + window, dtype=torch.int32, device="cuda")
        self.ctx = nw.AttnContext(heads, HKV, self.cap)

    def pos_ptr(self, i: int) -> int:
        return self.pos.data_ptr() + 4 * i

    def step(self, s: int, stream, append=True):
        layer, i = s % self.layers, (s // self.layers) % self.window
        if append:
            self.ctx.append_decode(self.q[i], self.knew[i], self.vnew[i], self.kc[layer],
                                   self.vc[layer], self.pos_ptr(i), self.out, 1, self.cap, stream)
        else:
            self.ctx.decode(self.q[i], self.kc[layer], self.vc[layer], self.pos_ptr(i), self.out,
                            1, self.cap, stream)

    def mean_kv_bytes(self, steps: int) -> float:
        tot = 0
        for s in range(steps):
            tot += kv_bytes(self.past + (s // self.layers) % self.window + 1)
        return tot / steps


class RaggedWorkload:
    """64 independent sequences, past lengths U{512..16384} from a seed, one
    query per sequence per step; step s appends token s % window of every
    sequence at past_b + token and attends (one nwd_append_decode call)."""

    def __init__(self, torch, nw, batch: int = 64, window: int = 64, seed: int = 4):
        import numpy as np

        g = np.random.Generator(np.random.PCG64(seed))
        self.past = g.integers(512, 16385, size=batch)
        self.batch, self.window = batch, window
        self.cap = int(self.past.max()) + window
        tg = torch.Generator(device="cuda")
        tg.manual_seed(seed)

        def rnd(*shape):
            return torch.randn(*shape, generator=tg, device="cuda", dtype=torch.float32).half()

        self.kc = rnd(batch, HKV, self.cap, D)
        self.vc = rnd(batch, HKV, self.cap, D)
        self.q = rnd(window, batch, H, D)
        self.knew = rnd(window, batch, HKV, D)
        self.vnew = rnd(window, batch, HKV, D)
        pos = self.past[None, :] + np.arange(window)[:, None]
        self.pos = torch.tensor(pos, dtype=torch.int32, device="cuda")
        self.out = torch.empty(batch, H, D, dtype=torch.float16, device="cuda")
        self.ctx = nw.AttnContext(H, HKV, self.cap, max_batch=batch)

    def step(self, s: int, stream, append=True):
        i = s % self.window
        if append:
            self.ctx.append_decode(self.q[i], self.knew[i], self.vnew[i], self.kc, self.vc,
                                   self.pos[i], self.out, self.batch, self.cap, stream)
        else:
            self.ctx.decode(self.q[i], self.kc, self.vc, self.pos[i], self.out, self.batch,
                            self.cap, stream)

    def mean_kv_bytes(self, steps: int) -> float:
        tot = 0
        for s in range(steps):
            tot += sum(kv_bytes(int(p) + s % self.window + 1) for p in self.past)
        return tot / steps


class PrefillWorkload:
    """Causal chunked prefill: 512 new tokens appended at 8192 (one
    nwd_kv_append of 512 rows) then nwd_prefill_attn over them. q_dtype
    "f32" gives fp32 queries and outputs (the engine's activations,
    engine/runtime.js:120-123), the query rows off the fp16 grid."""

    def __init__(self, torch, nw, past: int = 8192, n_new: int = 512, seed: int = 5,
                 q_dtype: str = "f16"):
        self.past, self.n_new, self.cap = past, n_new, past + n_new
        tg = torch.Generator(device="cuda")
        tg.manual_seed(seed)

        def rnd(*shape):
            return torch.randn(*shape, generator=tg, device="cuda", dtype=torch.float32).half()

        self.kc = rnd(1, HKV, self.cap, D)
        self.vc = rnd(1, HKV, self.cap, D)
        self.q = rnd(1, n_new, H, D)
        if q_dtype == "f32":
            self.q = self.q.float() + 1e-3 * torch.randn(self.q.shape, generator=tg, device="cuda")
        self.knew = rnd(1, n_new, HKV, D)
        self.vnew = rnd(1, n_new, HKV, D)
        self.out = torch.empty_like(self.q)
        self.pos0 = torch.tensor([past], dtype=torch.int32, device="cuda")
        self.ctx = nw.AttnContext(H, HKV, self.cap, q_dtype=q_dtype, o_dtype=q_dtype)

    def step(self, s: int, stream, append=True):
        if append:
            self.ctx.kv_append(self.knew, self.vnew, self.kc, self.vc, self.pos0, 1, self.n_new,
                               stream)
        self.ctx.prefill(self.q, self.kc, self.vc, self.pos0, self.out, 1, self.n_new, self.cap,
                         stream)

    def flops(self) -> float:
        """4*H*D*sum_i L_i: QK^T and PV, 2 flops per multiply-add each."""
        return 4.0 * H * D * sum(self.past + i + 1 for i in range(self.n_new))

    def mean_kv_bytes(self, steps: int) -> float:
        return float(kv_bytes(self.cap))


class Q4LayerWorkload:
    """The attention layer's 4-bit projections at the Nano-4B shapes
    (engine/config.js:2-26): `qkv-append` runs nwd_qkv_append (K = 3136 to
    q 5120 + k 1024 + v 1024 columns, k/v rounded into the fp16 caches at
    pos), `o-proj` runs nwd_q4_gemv with the residual accumulate (K = 5120
    to 3136). `layers` distinct random weight sets are rotated so the weights
    (14.4 MB / 8.3 MB per layer) come from HBM, not the 256 MB MALL."""

    HIDDEN, HEADS, KV_HEADS, VOCAB = 3136, 40, 8, 131072

    def __init__(self, torch, nw, kind: str, layers: int = 32, seed: int = 6):
        if kind == "lm-head":
            layers = 2  # 2 x 263 MB of weights already exceed the 256 MB MALL
        self.kind, self.layers, self.nw = kind, layers, nw
        tg = torch.Generator(device="cuda")
        tg.manual_seed(seed)
        if kind == "qkv-append":
            shapes = [(self.HEADS * D, self.HIDDEN // 32), (self.KV_HEADS * D, self.HIDDEN // 32),
                      (self.KV_HEADS * D, self.HIDDEN // 32)]
            k_in = self.HIDDEN
        elif kind == "lm-head":
            shapes = [(self.VOCAB, self.HIDDEN // 32)]
            k_in = self.HIDDEN
        else:
            shapes = [(self.HIDDEN, self.HEADS * D // 32)]
            k_in = self.HEADS * D

        def q4(n, nb):
            quant = torch.randint(0, 256, (n, nb, 16), generator=tg, device="cuda", dtype=torch.uint8)
            scales = torch.rand((n, nb), generator=tg, device="cuda") * 0.02 + 0.01
            zp = torch.randint(0, 256, ((n * nb + 1) // 2,), generator=tg, device="cuda",
                               dtype=torch.uint8)
            return (quant, scales, zp), nw.q4_weight(quant, scales, zp, n, nb)

        self.sets = [[q4(n, nb) for n, nb in shapes] for _ in range(layers)]
        self.weight_bytes = sum(n * nb * 16 + n * nb * 4 + (n * nb + 1) // 2 for n, nb in shapes)
        self.x = torch.randn((1, k_in), generator=tg, device="cuda")
        self.io_bytes = k_in * 4
        self.cap = 64
        self.ctx = nw.AttnContext(self.HEADS, self.KV_HEADS, self.cap, q_dtype="f32")
        if kind == "qkv-append":
            self.q_out = torch.empty((1, self.HEADS, D), device="cuda")
            self.kc = torch.zeros((1, self.KV_HEADS, self.cap, D), dtype=torch.float16, device="cuda")
            self.vc = torch.zeros_like(self.kc)
            self.pos = torch.arange(self.cap, dtype=torch.int32, device="cuda")
            self.io_bytes += self.HEADS * D * 4 + 2 * self.KV_HEADS * D * 2
        elif kind == "lm-head":
            self.token = torch.zeros((1,), dtype=torch.int32, device="cuda")
            self.io_bytes += 4
        else:
            self.h = torch.zeros((1, self.HIDDEN), device="cuda")
            self.io_bytes += 2 * self.HIDDEN * 4

    def step(self, s: int, stream, append=True):
        ws = [w for _, w in self.sets[s % self.layers]]
        if self.kind == "qkv-append":
            pos = self.pos.data_ptr() + 4 * ((s // self.layers) % self.cap)
            self.ctx.qkv_append(self.x, ws[0], ws[1], ws[2], self.q_out, self.kc, self.vc, pos, 1,
                                stream)
        elif self.kind == "lm-head":
            self.ctx.lm_head_argmax(self.x, ws[0], self.token, None, 1, stream)
        else:
            self.ctx.q4_gemv(self.x, ws[0], self.h, 1, self.nw.NWD_Q4_ACCUMULATE, stream)

    def bytes_per_step(self) -> int:
        return self.weight_bytes + self.io_bytes


class GeneralWorkload:
    """Decode-only calls on a head layout other than the benchmark's:
    `layers` caches of `past` random fp16 tokens (rotated so the K/V reads
    come from HBM), one fp16 query per call attending all `past` keys."""

    def __init__(self, torch, nw, heads: int, kv_heads: int, head_dim: int, past: int,
                 layers: int = 8, seed: int = 7):
        self.heads, self.kv_heads, self.head_dim, self.past = heads, kv_heads, head_dim, past
        self.layers = layers
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)

        def rnd(*shape):
            return torch.randn(*shape, generator=g, device="cuda", dtype=torch.float32).to(torch.float16)

        self.kc = [rnd(1, kv_heads, past, head_dim) for _ in range(layers)]
        self.vc = [rnd(1, kv_heads, past, head_dim) for _ in range(layers)]
        self.q = rnd(1, heads, head_dim)
        self.out = torch.empty(1, heads, head_dim, dtype=torch.float16, device="cuda")
        self.pos = torch.tensor([past - 1], dtype=torch.int32, device="cuda")
        self.ctx = nw.AttnContext(heads, kv_heads, past, head_dim=head_dim)

    def step(self, s: int, stream, append=False):
        layer = s % self.layers
        self.ctx.decode(self.q, self.kc[layer], self.vc[layer], self.pos, self.out, 1, self.past,
                        stream)

    def kv_bytes(self) -> int:
        return self.past * self.kv_heads * self.head_dim * 2 * 2


class GeneralPrefillWorkload:
    """Prefill-only calls on a head layout other than the benchmark's: n_new
    fp16 queries onto `past` cached tokens (the cache already holds the new
    rows)."""

    def __init__(self, torch, nw, heads: int, kv_heads: int, head_dim: int, past: int,
                 n_new: int, seed: int = 9):
        self.heads, self.head_dim, self.past, self.n_new = heads, head_dim, past, n_new
        cap = past + n_new
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)

        def rnd(*shape):
            return torch.randn(*shape, generator=g, device="cuda", dtype=torch.float32).to(torch.float16)

        self.kc, self.vc = rnd(1, kv_heads, cap, head_dim), rnd(1, kv_heads, cap, head_dim)
        self.q = rnd(1, n_new, heads, head_dim)
        self.out = torch.empty_like(self.q)
        self.pos0 = torch.tensor([past], dtype=torch.int32, device="cuda")
        self.cap = cap
        self.ctx = nw.AttnContext(heads, kv_heads, cap, head_dim=head_dim)

    def step(self, s: int, stream, append=False):
        self.ctx.prefill(self.q, self.kc, self.vc, self.pos0, self.out, 1, self.n_new, self.cap,
                         stream)

    def flops(self) -> float:
        """QK^T and PV over the real head dims, 2 flops per multiply-add."""
        return 4.0 * self.heads * self.head_dim * sum(self.past + i + 1 for i in range(self.n_new))


def run_general(torch, nw, steps: int = 128, warmup: int = 8):
    """Head layouts other than the benchmark's (head_dim 128 with groups
    1/2/4/5/8): us per decode call (graph-replayed), K/V GB/s and the
    fraction of the HBM peak, and the time at half and twice the split
    count."""
    res = {}
    for name, (heads, kv_heads, head_dim, past, desc) in GENERAL_SHAPES.items():
        log(f"[bench] {name}: {heads}q/{kv_heads}kv/d{head_dim}, {past} keys, {steps} calls")
        wl = GeneralWorkload(torch, nw, heads, kv_heads, head_dim, past)
        warm_up(torch, wl, 0.1, append=False)
        _, ms = time_graph(torch, wl, steps, warmup, append=False, reps=3)
        us = ms * 1e3 / steps
        gbs = wl.kv_bytes() / (us * 1e-6) / 1e9
        splits = wl.ctx.decode_splits(1, past)
        # the library's split count against half and twice as many
        by_splits = {}
        for n in sorted({max(1, splits // 2), min(256, splits * 2)} - {splits}):
            wl.ctx.set_decode_splits(n)
            _, ms_n = time_graph(torch, wl, steps, warmup, append=False, reps=3)
            by_splits[str(n)] = ms_n * 1e3 / steps
        wl.ctx.set_decode_splits(0)
        res[name] = {"desc": desc, "us_per_call": us, "kv_bytes": wl.kv_bytes(), "gbs": gbs,
                     "hbm_frac": gbs / HBM_PEAK_GBS, "splits": splits,
                     "us_by_forced_splits": by_splits}
        log(f"[bench] {name}: {res[name]}")
        wl.ctx.close()
        del wl
        torch.cuda.empty_cache()
    for name, (heads, kv_heads, head_dim, past, n_new, desc) in GENERAL_PREFILL_SHAPES.items():
        log(f"[bench] {name}: {heads}q/{kv_heads}kv/d{head_dim}, {n_new} onto {past}")
        wl = GeneralPrefillWorkload(torch, nw, heads, kv_heads, head_dim, past, n_new)
        warm_up(torch, wl, 0.1, append=False)
        _, ms = time_graph(torch, wl, 16, 2, append=False, reps=3)
        us = ms * 1e3 / 16
        tflops = wl.flops() / (us * 1e-6) / 1e12
        res[name] = {"desc": desc, "us_per_call": us, "tflops": tflops,
                     "mfma_frac": tflops / MFMA_F16_PEAK_TFLOPS}
        log(f"[bench] {name}: {res[name]}")
        wl.ctx.close()
        del wl
        torch.cuda.empty_cache()
    return res


def q4_cpu_baseline(kind: str, budget_s: float = 10.0):
    """The oracle's restatement of kernels/matmul_nbits_sg.wgsl on the host's
    cores for one layer's projections of the same shapes (random weights)."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    g = np.random.Generator(np.random.PCG64(6))
    hid, heads, kvh = Q4LayerWorkload.HIDDEN, Q4LayerWorkload.HEADS, Q4LayerWorkload.KV_HEADS
    shapes = {"qkv-append": [(heads * D, hid // 32), (kvh * D, hid // 32), (kvh * D, hid // 32)],
              "o-proj": [(hid, heads * D // 32)],
              "lm-head": [(Q4LayerWorkload.VOCAB, hid // 32)]}[kind]
    mats = [(g.integers(0, 256, (n, nb, 16), dtype=np.uint8),
             g.uniform(0.01, 0.03, (n, nb)).astype(np.float32),
             g.integers(0, 256, (n * nb + 1) // 2, dtype=np.uint8)) for n, nb in shapes]
    x = g.standard_normal(32 * shapes[0][1]).astype(np.float32)
    threads = oracle.max_threads()
    t0, done = time.perf_counter(), 0
    while done == 0 or time.perf_counter() - t0 < budget_s:
        for quant, scales, zp in mats:
            y = oracle.q4_gemv_f32(x, quant, scales, zp, threads=threads)
            if kind == "lm-head":
                oracle.argmax_ref(y)
        done += 1
    dt = time.perf_counter() - t0
    wbytes = sum(n * nb * 16 + n * nb * 4 + (n * nb + 1) // 2 for n, nb in shapes)
    return {"us_per_step": round(dt / done * 1e6, 1), "gbs": round(wbytes * done / dt / 1e9, 3),
            "cores": threads, "kind": "port", "sample": f"{done} calls, one layer's weights"}


def time_graph(torch, wl, steps: int, warmup: int, append=True, reps: int = 1,
               preroll: int = 32):
    """Warm up eagerly, capture `steps` steps into a HIP graph, replay it once
    untimed and `reps` times timed. Returns (wall seconds, device ms) of the
    timed replay, the median one when reps > 1 (the first replays after a
    capture can run at lower clocks).

    A freshly captured graph is first replayed untimed for at least 30 ms:
    its first replays run slower (decode-32k: 26.2-26.4 against 24.5 us per
    step over the first ~20 ms after capture, ~1 us more per dispatch). Each
    timed replay is preceded by an untimed pre-roll graph of the same
    workload's steps (min(steps, preroll) of them), launched just before the
    start event, so the GPU is busy while the host launches the timed graph.
    Each graph launch still costs ~9 us of GPU time (its per-step share is
    ~0.45 us at 20 steps, ~0.04 us at 256), which the timed region holds."""
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for s in range(warmup):
            wl.step(s, stream, append)
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for s in range(steps):
            wl.step(s, stream, append)
    pre = torch.cuda.CUDAGraph()
    with torch.cuda.graph(pre, stream=stream):
        for s in range(min(steps, preroll)):
            wl.step(s, stream, append)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    runs = []
    with torch.cuda.stream(stream):  # replay() launches on the current stream
        t_settle = time.perf_counter()
        while True:
            graph.replay()
            pre.replay()
            torch.cuda.synchronize()
            if time.perf_counter() - t_settle > 0.03:
                break
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            pre.replay()
            start.record(stream)
            graph.replay()
            end.record(stream)
            torch.cuda.synchronize()
            runs.append((time.perf_counter() - t0, start.elapsed_time(end)))
    runs.sort(key=lambda r: r[1])
    return runs[len(runs) // 2]


def warm_up(torch, wl, seconds: float = 0.25, append=True):
    """Runs the workload's steps eagerly for `seconds` before anything is
    timed: the first timed graph of a process otherwise meets a GPU whose
    clocks have not settled (26.6 against 24.9 us per decode-32k step for the
    same 20-step graph, first against later replays)."""
    stream = torch.cuda.Stream()
    t0, s = time.perf_counter(), 0
    with torch.cuda.stream(stream):
        while time.perf_counter() - t0 < seconds:
            for _ in range(16):
                wl.step(s, stream, append)
                s += 1
            stream.synchronize()


def time_eager(torch, wl, steps: int, append=True, reps: int = 1, preroll: int = 16):
    """Exactly `steps` steps issued as ordinary calls (the way the engine's
    token loop issues them), timed with events on their stream; each run is
    preceded by `preroll` untimed calls of the same steps, so the GPU holds a
    backlog of ~preroll steps while the host issues the timed ones and never
    waits for the host. Returns the median device ms over `reps` runs."""
    stream = torch.cuda.Stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    runs = []
    with torch.cuda.stream(stream):
        for _ in range(reps):
            torch.cuda.synchronize()
            for s in range(preroll):
                wl.step(s, stream, append)
            start.record(stream)
            for s in range(steps):
                wl.step(s, stream, append)
            end.record(stream)
            torch.cuda.synchronize()
            runs.append(start.elapsed_time(end))
    runs.sort()
    return runs[len(runs) // 2]


def split_kernel_us(torch, hip: Hip, wl, calls: int):
    """Duration of the split kernel alone (the dominant kernel of a decode
    call), from HIP events the runtime records at its start and end
    (nwd_set_kernel_events): eager decode-only calls over the same rotation
    of layer caches, issued back to back with an event pair each and read
    after one synchronisation, so the GPU stays as busy as in the graph
    replays (a host wait after every call let the kernel start from an idle
    GPU: 23.1 against 21.9 us per 32K matrix-core launch in a kernel trace).
    Returns the mean in us."""
    stream = torch.cuda.Stream()
    pairs = [(hip.event(), hip.event()) for _ in range(calls + 8)]
    tot = []
    try:
        for s, (e0, e1) in enumerate(pairs):
            wl.ctx.set_kernel_events(e0, e1)
            wl.step(s, stream, append=False)
        torch.cuda.synchronize()
        for s, (e0, e1) in enumerate(pairs):
            if s >= 8:
                tot.append(hip.elapsed_ms(e0, e1) * 1e3)
    finally:
        wl.ctx.set_kernel_events(None, None)
        torch.cuda.synchronize()
        for e0, e1 in pairs:
            hip.destroy(e0)
            hip.destroy(e1)
    return sum(tot) / len(tot)


def host_info() -> dict:
    """The host the CPU baselines ran on: logical CPUs, CPU model, and the
    OpenMP threads the oracle uses."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu_model": model, "threads": oracle.max_threads()}


def _oracle_kv(g, n: int, dist: str):
    """Token-major [n][Hkv][D] f32 keys or values of a workload's distribution."""
    import numpy as np

    x = g.standard_normal((n, HKV, D), dtype=np.float32)
    if dist == "outliers":
        hit = g.random((n, HKV, D)) < 0.01
        x[hit] = np.where(g.random(int(hit.sum())) < 0.5, -8.0, 8.0)
    elif dist == "head-scale":
        x *= g.uniform(0.5, 2.0, HKV).astype(np.float32)[None, :, None]
    return x


def cpu_baseline(past: int, window: int, budget_s: float = 20.0, dist: str = "normal",
                 order=None):
    """The oracle (op-for-op CPU restatement of kernels/sparse_attn.wgsl +
    kv_append.wgsl, f32, per-head workgroups over OpenMP threads) on the same
    workload shape: append+attend steps at positions past + i, i taken from
    `order` (default 0, 1, ..., window - 1, repeated), for `budget_s` seconds
    (at least one step)."""
    import numpy as np

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    threads = oracle.max_threads()
    g = np.random.Generator(np.random.PCG64(7))
    cap = past + window
    k, v = _oracle_kv(g, cap, dist), _oracle_kv(g, cap, dist)
    q = g.standard_normal((window, H, D), dtype=np.float32)
    kc = np.zeros(cap * HKV * D, np.float32)
    vc = np.zeros(cap * HKV * D, np.float32)
    kc[: cap * HKV * D] = k.reshape(-1)  # rows past a step's position are never read
    vc[: cap * HKV * D] = v.reshape(-1)
    order = list(order) if order is not None else list(range(window))
    done, nbytes, seen = 0, 0, set()
    t0 = time.perf_counter()
    while done == 0 or time.perf_counter() - t0 < budget_s:
        i = order[done % len(order)]
        p = past + i
        oracle.kv_append_f32(k[p], kc, p, HKV, D)
        oracle.kv_append_f32(v[p], vc, p, HKV, D)
        L = p + 1
        oracle.sparse_attn_f32(q[i], kc[: L * HKV * D].reshape(L, HKV, D),
                               vc[: L * HKV * D].reshape(L, HKV, D), threads=0)
        done += 1
        nbytes += kv_bytes(L)
        seen.add(i)
    dt = time.perf_counter() - t0
    return {
        "value": round(nbytes / dt / 1e9, 3),
        "unit": "GB/s",
        "us_per_step": round(dt / done * 1e6, 1),
        "cores": threads,
        "kind": "port",
        "sample": f"{done} append+attend steps over {len(seen)} of the {window} positions "
                  f"past {past} (L = {past + 1}..{past + window}), one layer, f32 token-major cache",
    }


def cpu_baseline_ragged(budget_s: float = 6.0, batch: int = 64, seed: int = 4):
    """The oracle on ragged-64 steps: each step appends one row to each of the
    64 sequences and attends its past_b + 1 keys (the lengths of the GPU
    workload; the K/V of every sequence are prefixes of one random cache)."""
    import numpy as np

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    past = np.random.Generator(np.random.PCG64(seed)).integers(512, 16385, size=batch)
    g = np.random.Generator(np.random.PCG64(8))
    cap = int(past.max()) + 1
    k, v = _oracle_kv(g, cap, "normal"), _oracle_kv(g, cap, "normal")
    q = g.standard_normal((batch, H, D), dtype=np.float32)
    kc, vc = k.reshape(-1).copy(), v.reshape(-1).copy()
    done, nbytes = 0, 0
    t0 = time.perf_counter()
    while done == 0 or time.perf_counter() - t0 < budget_s:
        for b in range(batch):
            p = int(past[b])
            oracle.kv_append_f32(k[p], kc, p, HKV, D)
            oracle.kv_append_f32(v[p], vc, p, HKV, D)
            L = p + 1
            oracle.sparse_attn_f32(q[b], kc[: L * HKV * D].reshape(L, HKV, D),
                                   vc[: L * HKV * D].reshape(L, HKV, D), threads=0)
            nbytes += kv_bytes(L)
        done += 1
    dt = time.perf_counter() - t0
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s",
            "us_per_step": round(dt / done * 1e6, 1), "cores": oracle.max_threads(),
            "kind": "port",
            "sample": f"{done} step(s) of 64 sequences, past U{{512..16384}} (seed {seed}), "
                      "one layer, f32 token-major caches"}


def cpu_baseline_prefill(budget_s: float = 8.0, past: int = 8192, n_new: int = 512):
    """The reference's prefill of prefill-512 on the host: the token loop of
    engine/runtime.js:640-643, one append+attend step per prompt token
    (L = past + 1 .. past + n_new), through the oracle. As many of the 512
    steps as fit in the budget are run, every 8th token first so the sample
    spans the chunk; the chunk's time is the mean step time x 512."""
    order = [i for r in range(8) for i in range(r, n_new, 8)]
    r = cpu_baseline(past, n_new, budget_s=budget_s, order=order)
    per = r["us_per_step"]
    return {"value": round(per * n_new / 1e3, 2), "unit": "ms per 512-token chunk",
            "us_per_step": per, "cores": r["cores"], "kind": "port",
            "sample": r["sample"].replace("append+attend steps", "token steps of the chunk")}


WORKLOADS = {
    # name: (past, window, layers, K/V distribution, description)
    "decode-32k": (32768, 64, 4, "outliers",
                   "decode-32k: B=1, 32q/8kv/d128, past 32768, K/V N(0,1) with 1% +-8 outliers, "
                   "append+attend per step, split-K, 4 layer caches rotated (537 MB)"),
    "decode-4k": (4096, 64, 32, "head-scale",
                  "decode-4k-64steps: B=1, 32q/8kv/d128, past 4096, K/V N(0,1) x per-head "
                  "U[0.5,2], append+attend per step, 32 layer caches rotated (545 MB)"),
    "decode-1k": (1024, 64, 128, "normal",
                  "decode-1k: B=1, 32q/8kv/d128, past 1024, K/V N(0,1), append+attend per step, "
                  "128 layer caches rotated (570 MB)"),
    "decode-153": (152, 1, 64, "normal",
                   "decode-153: B=1, 32q/8kv/d128, past 152, one token appended at 152 and 153 "
                   "keys attended per step, K/V N(0,1), 64 layer caches rotated (40 MB)"),
    "decode-32k-nano": (32768, 64, 4, "outliers",
                        "decode-32k-nano: decode-32k on the Nemotron-H Nano-4B attention shape, "
                        "B=1, 40q/8kv/d128 (group 5), past 32768, K/V N(0,1) with 1% +-8 "
                        "outliers, append+attend per step, 4 layer caches rotated (537 MB)", 40),
}
# Split kernels of a decode call (nwd_set_decode_kernel).
DECODE_KERNELS = {0: "dot-product (decode_split_kernel)", 1: "matrix-core (decode_mfma_kernel)"}
EXTRA_WORKLOADS = {
    "ragged-64": "ragged-64: 64 sequences, past U{512..16384} (seed 4), one query each, "
                 "append+attend per step",
    "prefill-512": "prefill-512: B=1, 512 new tokens onto 8192 cached, causal in the chunk, "
                   "kv_append of 512 rows + fp16-MFMA prefill per step",
    "prefill-512-f32q": "prefill-512-f32q: prefill-512 with fp32 queries off the fp16 grid and "
                        "fp32 outputs (the engine's activations), the query as fp16 high and low "
                        "parts in the QK^T MFMAs",
    "stream-read": "stream-read: the decode-32k K/V bytes (134 MB per launch, 4 layer caches "
                   "rotated) read with the split kernel's access pattern and nothing else",
    "plain-read": "plain-read: the decode-32k K/V bytes (134 MB per launch, 4 layer caches "
                  "rotated) read by a grid-stride kernel, the fastest of several launch shapes",
    "launch-gap": "launch-gap: back-to-back launches of an empty kernel (one store per "
                  "workgroup) with the decode's split and merge grids: the per-kernel floor",
    "mfma-ceiling": "mfma-ceiling: 256 x 512-thread workgroups of 16x16x32 fp16 MFMAs only, "
                    "v_exp_f32 only (one per two MFMAs, the prefill's ratio), both, v_fma_f32 "
                    "only (one per MFMA) and MFMAs with FMAs",
    "qkv-append": "qkv-append: B=1, Nano-4B q/k/v 4-bit projections K=3136 -> 5120+1024+1024 "
                  "with k/v rounded into the fp16 caches, 32 weight sets rotated (461 MB)",
    "o-proj": "o-proj: B=1, Nano-4B o_proj 4-bit K=5120 -> 3136 with the residual add, "
              "32 weight sets rotated (266 MB)",
    "lm-head": "lm-head: B=1, Nano-4B lm_head 4-bit K=3136 -> 131072 with the greedy pick "
               "(argmax partial in the GEMV, then the merge), 2 weight sets rotated (527 MB)",
}
# Step counts of the secondary measurements (fixed, so a short --steps only
# shortens the headline's timed region).
# Head layouts outside the benchmark's (groups 7 and 16, head sizes 256, 96
# and 64, group 7 at 64), decode-only, B = 1:
# name: (n_heads, n_kv_heads, head_dim, keys, description)
GENERAL_SHAPES = {
    "general-g7-32k": (28, 4, 128, 32768, "B=1, 28q/4kv/d128 (group 7: the Qwen2.5-7B head "
                       "layout, on the matrix-core split kernel built for group 7), 32768 keys, "
                       "fp16 I/O, decode call"),
    "general-d256-8k": (16, 8, 256, 8192, "B=1, 16q/8kv/d256 (group 2, head size 256: the "
                        "Gemma-2-9B layout, on the split kernel built for head size 256), 8192 "
                        "keys, fp16 I/O, decode call"),
    "general-d96-4k": (32, 32, 96, 4096, "B=1, 32q/32kv/d96 (group 1, head size 96: the "
                       "Phi-3-mini layout, on the head-128 split kernel's padded form), 4096 "
                       "keys, fp16 I/O, decode call"),
    "general-g16-8k": (128, 8, 128, 8192, "B=1, 128q/8kv/d128 (group 16: the Llama-3.1-405B "
                       "layout, as two groups of 8 per KV head on the matrix-core split kernel), "
                       "8192 keys, fp16 I/O, decode call"),
    "general-d64-16k": (32, 8, 64, 16384, "B=1, 32q/8kv/d64 (group 4, head size 64: the "
                        "Llama-3.2-1B layout, on the matrix-core split kernel built for head "
                        "size 64), 16384 keys, fp16 I/O, decode call"),
    "general-d64-g7-32k": (14, 2, 64, 32768, "B=1, 14q/2kv/d64 (group 7, head size 64: the "
                           "Qwen2.5-0.5B layout, on the matrix-core split kernel built for head "
                           "size 64), 32768 keys, fp16 I/O, decode call"),
}
# Prefill on other head layouts: (heads, kv heads, head_dim, past, new tokens, description).
GENERAL_PREFILL_SHAPES = {
    "general-prefill-d64": (32, 8, 64, 8192, 512, "B=1, 32q/8kv/d64 (Llama-3.2-1B layout), 512 "
                            "new tokens onto 8192, fp16 I/O, prefill call (the MFMA prefill "
                            "built for head size 64)"),
    "general-prefill-d96": (32, 32, 96, 8192, 512, "B=1, 32q/32kv/d96 (Phi-3-mini layout), 512 "
                            "new tokens onto 8192, fp16 I/O, prefill call (MFMA kernel, rows "
                            "padded to 128 dims)"),
    "general-prefill-d256": (16, 8, 256, 8192, 512, "B=1, 16q/8kv/d256 (Gemma-2-9B layout), 512 "
                             "new tokens onto 8192, fp16 I/O, prefill call (the head-256 MFMA "
                             "prefill)"),
    "general-prefill-g7": (28, 4, 128, 8192, 512, "B=1, 28q/4kv/d128 (Qwen2.5-7B layout, group "
                           "7), 512 new tokens onto 8192, fp16 I/O, prefill call (the MFMA "
                           "prefill built for group 7)"),
}

SECONDARY_STEPS = {"decode-1k": 512, "decode-32k": 256, "decode-32k-nano": 256, "decode-4k": 512,
                   "decode-153": 1024, "ragged-64": 64,
                   "prefill-512": 32, "stream-read": 64, "plain-read": 64,
                   "qkv-append": 256, "o-proj": 256, "lm-head": 32}


def hbm_roofline(achieved_gbs: float, kernel: str, algorithmic_bytes: float, traffic):
    return {"bound": "hbm", "kernel": kernel, "achieved": round(achieved_gbs, 1),
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic, "algorithmic_bytes": int(algorithmic_bytes)}


def run_decode(torch, nw, hip, name: str, steps: int, warmup: int, dec_steps: int = 0,
               other_splits=(), other_kernels=()):
    """Times `steps` append+attend steps and `dec_steps` (default `steps`)
    decode-only calls of one workload from HIP graphs, and the split kernel
    alone from eager calls; returns a dict of the measurements. For each n in
    `other_splits` the decode-only calls are timed again with the split count
    forced to n (nwd_set_decode_splits), which at short contexts also selects
    the per-KV-head form instead of one workgroup per query head. For each k
    in `other_kernels` they are timed with the split kernel forced to k
    (nwd_set_decode_kernel: 0 dot-product, 1 matrix-core)."""
    past, window, layers, dist, desc = WORKLOADS[name][:5]
    heads = WORKLOADS[name][5] if len(WORKLOADS[name]) > 5 else H
    log(f"[bench] {name}: past={past} window={window} layers={layers} heads={heads}, {steps} steps")
    wl = DecodeWorkload(torch, nw, past, window, layers, seed=1234, dist=dist, heads=heads)
    warm_up(torch, wl)
    # The step, timed two ways over exactly `steps` append+attend steps: as
    # calls issued the way the engine's token loop issues them (median of 5
    # runs, behind a pre-roll so the GPU holds a backlog), and replayed from a
    # HIP graph (median of 3). Each method adds a launch cost that is not the
    # step's: a graph launch ~9 us of GPU time per replay (0.45 us per step at
    # 20 steps), and calls leave the GPU waiting on the host where a step is
    # shorter than the host's ~5-7 us per call (short contexts). us_per_step
    # is the lower of the two; step_timing names it.
    t0 = time.perf_counter()
    ms = time_eager(torch, wl, steps, reps=5)
    wall = time.perf_counter() - t0
    calls_us_step = ms * 1e3 / steps
    _, ms_g = time_graph(torch, wl, steps, warmup, reps=3)
    graph_us_step = ms_g * 1e3 / steps
    us_step = min(calls_us_step, graph_us_step)
    step_timing = "calls" if calls_us_step <= graph_us_step else "graph"
    mean_b = wl.mean_kv_bytes(steps)
    # the decode call alone (split + merge kernels), same rotation
    n_dec = dec_steps or steps
    _, ms_dec = time_graph(torch, wl, n_dec, 0, append=False, reps=3)
    dec_us = ms_dec * 1e3 / n_dec
    dec_b = wl.mean_kv_bytes(n_dec)
    split_us = split_kernel_us(torch, hip, wl, 128)
    n_eager = min(max(steps, 256), 512)
    eager_us = time_eager(torch, wl, n_eager, reps=3) * 1e3 / n_eager
    splits = wl.ctx.decode_splits(1, wl.cap)
    forced = {}
    for n in other_splits:
        wl.ctx.set_decode_splits(n)
        _, ms_n = time_graph(torch, wl, n_dec, 0, append=False, reps=3)
        forced[str(n)] = ms_n * 1e3 / n_dec
    if other_splits:
        wl.ctx.set_decode_splits(0)
    by_kernel = {}
    for k in other_kernels:
        wl.ctx.set_decode_kernel(k)
        _, ms_k = time_graph(torch, wl, n_dec, 0, append=False, reps=3)
        by_kernel[DECODE_KERNELS[k]] = ms_k * 1e3 / n_dec
    if other_kernels:
        wl.ctx.set_decode_kernel(None)
    res = {
        "workload": name, "desc": desc, "past": past, "window": window, "layers": layers,
        "steps": steps, "us_per_step": us_step, "gbs": mean_b / (us_step * 1e-6) / 1e9,
        "decode_us": dec_us, "decode_gbs": dec_b / (dec_us * 1e-6) / 1e9,
        "split_kernel_us": split_us, "eager_us_per_step": eager_us, "graph_us_per_step": graph_us_step,
        "calls_us_per_step": calls_us_step, "step_timing": step_timing, "mean_kv_bytes": mean_b,
        "wall_s": wall, "splits": splits,
    }
    if forced:
        res["decode_us_forced_splits"] = forced
    if by_kernel:
        res["decode_us_by_kernel"] = by_kernel
    res["n_heads"] = heads
    # the launch's choice of split kernel for this shape (launch_decode in
    # nwd_decode.hip; B = 1): the matrix-core kernel for one workgroup per KV
    # head with G >= 5, or G = 4 with splits of 512+ keys that all run at once
    per_kv_head = heads * splits > 256
    g = heads // HKV
    long_splits = wl.cap >= 512 * splits and HKV * splits <= 256
    res["split_kernel"] = DECODE_KERNELS[1 if per_kv_head and (g >= 5 or (g == 4 and long_splits))
                                         else 0]
    # The dominant kernel's duration: HIP events at the split kernel's start
    # and end (eager calls), or the whole graph-timed call when that is
    # shorter (the events include the dispatch latency of an eager launch,
    # which dominates a few-microsecond kernel).
    kern_us = min(split_us, dec_us)
    kname = res["split_kernel"].split("(")[1].rstrip(")")
    kernel = (f"{kname} (HIP events at its start and end, or the whole call if shorter); "
              "the call adds decode_merge_kernel" if splits > 1
              else f"{kname} (one split, no merge: the graph-timed call or its events)")
    res["kernel_us"] = kern_us
    res["roofline"] = hbm_roofline(dec_b / (kern_us * 1e-6) / 1e9, kernel, dec_b,
                                   measured_traffic(name))
    res["roofline"]["kernel_us"] = round(kern_us, 3)
    res["call_roofline"] = {"achieved": round(res["decode_gbs"], 1),
                            "frac": round(res["decode_gbs"] / HBM_PEAK_GBS, 4),
                            "us": round(dec_us, 3)}
    log(f"[bench] {name}: step {us_step:.3f} us ({res['gbs']:.1f} GB/s; calls {calls_us_step:.3f}, "
        f"graph-replayed {graph_us_step:.3f}), "
        f"decode call {dec_us:.3f} us ({res['decode_gbs']:.1f} GB/s), split kernel {split_us:.3f} us, "
        f"{n_eager} calls {eager_us:.3f} us per step")
    wl.ctx.close()
    del wl
    torch.cuda.empty_cache()
    return res


def run_ragged(torch, nw, steps: int, warmup: int):
    log(f"[bench] ragged-64: {steps} steps")
    wl = RaggedWorkload(torch, nw)
    warm_up(torch, wl)
    wall, ms = time_graph(torch, wl, steps, warmup, reps=5)
    _, ms_main = time_graph(torch, wl, steps, 0, append=False, reps=5)
    us_step, us_main = ms * 1e3 / steps, ms_main * 1e3 / steps
    by_kernel = {}
    for k in (0, 1):  # the decode call on each split kernel (nwd_set_decode_kernel)
        wl.ctx.set_decode_kernel(k)
        _, ms_k = time_graph(torch, wl, steps, 0, append=False, reps=3)
        by_kernel[DECODE_KERNELS[k]] = ms_k * 1e3 / steps
    wl.ctx.set_decode_kernel(None)
    b = wl.mean_kv_bytes(steps)
    res = {"workload": "ragged-64", "desc": EXTRA_WORKLOADS["ragged-64"], "us_per_step": us_step,
           "decode_us": us_main, "wall_s": wall, "mean_kv_bytes": b,
           "splits": wl.ctx.decode_splits(wl.batch, wl.cap),
           # the launch's choice for this batch of 64 (see nwd_decode.hip)
           "split_kernel": DECODE_KERNELS[1 if H // HKV >= 4 else 0],
           "decode_us_by_kernel": by_kernel,
           "gbs": b / (us_step * 1e-6) / 1e9, "decode_gbs": b / (us_main * 1e-6) / 1e9}
    res["roofline"] = hbm_roofline(res["decode_gbs"],
                                   "nwd_decode_attn (split + merge kernels, one call; split kernel "
                                   f"{res['split_kernel']})", b, measured_traffic("ragged-64"))
    log(f"[bench] ragged-64: step {us_step:.1f} us, decode {us_main:.1f} us "
        f"({res['decode_gbs']:.1f} GB/s)")
    wl.ctx.close()
    del wl
    torch.cuda.empty_cache()
    return res


def run_prefill(torch, nw, steps: int, warmup: int, q_dtype: str = "f16", library=True):
    log(f"[bench] prefill-512 ({q_dtype} queries): {steps} steps")
    wl = PrefillWorkload(torch, nw, q_dtype=q_dtype)
    # The matrix cores' clock settles over the first milliseconds of this
    # load (the first timed graph ran 4-5 us per step slower than later ones):
    # one untimed pass of the same graph first.
    time_graph(torch, wl, steps, warmup, reps=3)
    wall, ms = time_graph(torch, wl, steps, warmup, reps=5)
    _, ms_main = time_graph(torch, wl, steps, 0, append=False, reps=5)
    us_step, us_main = ms * 1e3 / steps, ms_main * 1e3 / steps
    tflops = wl.flops() / (us_main * 1e-6) / 1e12
    name = "prefill-512" if q_dtype == "f16" else "prefill-512-f32q"
    res = {"workload": name, "desc": EXTRA_WORKLOADS[name], "q_dtype": q_dtype,
           "us_per_step": us_step, "prefill_us": us_main, "wall_s": wall, "flops": wl.flops(),
           "roofline": {"bound": "mfma", "kernel": "nwd_prefill_attn (prefill + split merge)",
                        "achieved": round(tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                        "unit": "TFLOP/s", "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                        "traffic": measured_traffic(name), "algorithmic_flops": wl.flops()}}
    log(f"[bench] prefill-512 ({q_dtype}): step {us_step:.1f} us (kv_append + prefill), prefill "
        f"{us_main:.1f} us ({tflops:.1f} TFLOP/s)")
    if library:
        lib = library_prefill(torch, wl)
        if "us" in lib:
            lib["nwd_speedup"] = lib["us"] / us_main
        res["library_baseline"] = lib
        log(f"[bench] prefill-512 through torch's fused attention: {lib}")
    wl.ctx.close()
    del wl
    torch.cuda.empty_cache()
    return res


def library_prefill(torch, wl, steps: int = 16):
    """The prefill-512 work through torch's own fused attention
    (scaled_dot_product_attention restricted to its flash backend, then its
    memory-efficient one; the math path is never used), on the inputs and
    cache state nwd_prefill_attn just ran on: query i of the chunk sees keys
    0 .. past + i (a lower-right causal mask). A vendor-library figure for the
    same work, with its largest difference from nwd's output."""
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    from torch.nn.attention.bias import causal_lower_right

    torch.cuda.synchronize()
    qh = wl.q.transpose(1, 2).contiguous()  # [1, H, n_new, D]
    mask = causal_lower_right(wl.n_new, wl.cap)
    ours = wl.out.float().transpose(1, 2)
    errors = []
    for name, backend in (("flash", SDPBackend.FLASH_ATTENTION),
                          ("efficient", SDPBackend.EFFICIENT_ATTENTION)):
        for gqa in (True, False):
            try:
                if gqa:
                    k, v, kw = wl.kc, wl.vc, {"enable_gqa": True}
                else:
                    k = wl.kc.repeat_interleave(H // HKV, dim=1).contiguous()
                    v = wl.vc.repeat_interleave(H // HKV, dim=1).contiguous()
                    kw = {}
                with sdpa_kernel([backend]):
                    o = F.scaled_dot_product_attention(qh, k, v, attn_mask=mask, **kw)
                    torch.cuda.synchronize()
                    err = (o.float() - ours).abs().max().item()

                    class Sdpa:
                        def step(self, s, stream, append=True):
                            F.scaled_dot_product_attention(qh, k, v, attn_mask=mask, **kw)

                    _, ms = time_graph(torch, Sdpa(), steps, 2, reps=3)
                us = ms * 1e3 / steps
                return {"impl": f"torch {torch.__version__} scaled_dot_product_attention, {name} "
                                f"backend, " + ("enable_gqa" if gqa else "K/V expanded to 32 heads"),
                        "us": us, "tflops": wl.flops() / (us * 1e-6) / 1e12,
                        "max_abs_diff_vs_nwd": err}
            except Exception as ex:  # a backend this build of torch lacks
                errors.append(f"{name} gqa={gqa}: {type(ex).__name__}: {str(ex)[:120]}")
            finally:
                torch.cuda.synchronize()
    return {"impl": "torch scaled_dot_product_attention", "error": "; ".join(errors)}


def run_stream_read(torch, nw, launches: int):
    """The read ceiling of the decode-32k access pattern (csrc/bench/
    nwd_stream_read.hip): the same 4 layer caches, one workgroup per CU (32
    splits per KV head; the decode itself runs 24 at this length, where the
    plain read measured slower), graph-replayed back to back."""
    lib = ctypes.CDLL(str(BENCH_LIB))
    lib.nwd_bench_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_void_p, ctypes.c_void_p]
    past, window, layers, dist, _ = WORKLOADS["decode-32k"]
    log(f"[bench] stream-read: {launches} launches")
    wl = DecodeWorkload(torch, nw, past, window, layers, seed=1234, dist=dist)
    keys, splits = past + 1, 256 // HKV
    out = torch.empty(HKV * splits * 256, dtype=torch.float32, device="cuda")

    class Reader:
        def step(self, s, stream, append=True):
            rc = lib.nwd_bench_stream_read(wl.kc[s % layers].data_ptr(), wl.vc[s % layers].data_ptr(),
                                           HKV, wl.cap, keys, splits, out.data_ptr(),
                                           stream.cuda_stream)
            if rc != 0:
                raise RuntimeError(f"nwd_bench_stream_read: hip error {rc}")

    _, ms = time_graph(torch, Reader(), launches, 8, reps=3)
    us = ms * 1e3 / launches
    b = kv_bytes(keys)
    res = {"workload": "stream-read", "desc": EXTRA_WORKLOADS["stream-read"], "us_per_launch": us,
           "bytes": b, "gbs": b / (us * 1e-6) / 1e9, "frac": b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS,
           "splits": splits}
    log(f"[bench] stream-read: {us:.3f} us per 134 MB launch ({res['gbs']:.1f} GB/s)")
    wl.ctx.close()
    del wl, out
    torch.cuda.empty_cache()
    return res


# Launch shapes of the plain read (threads per workgroup, 16-byte loads in
# flight per thread, workgroups): 2 to 4 wavefronts per SIMD, 4-8 KB in flight
# per wavefront, the best of a sweep of 96 shapes on MI355X among them.
PLAIN_READ_SHAPES = ((512, 4, 256), (256, 4, 512), (256, 8, 512), (256, 4, 1024),
                     (1024, 4, 256), (256, 2, 1024))


def run_plain_read(torch, nw, launches: int):
    """An independent read ceiling: the decode-32k bytes (the same 4 layer
    caches, 134 MB per launch) read by a grid-stride kernel that shares
    nothing with the decode's grid (csrc/bench/nwd_stream_read.hip,
    plain_read_kernel): every workgroup walks chunks spread over all the
    bytes, many wavefronts per CU, non-temporal loads. Each shape of
    PLAIN_READ_SHAPES is graph-replayed; the fastest is the ceiling."""
    lib = ctypes.CDLL(str(BENCH_LIB))
    lib.nwd_bench_plain_read.argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int] * 7 + [
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
    past, window, layers, dist, _ = WORKLOADS["decode-32k"]
    log(f"[bench] plain-read: {len(PLAIN_READ_SHAPES)} shapes x {launches} launches")
    wl = DecodeWorkload(torch, nw, past, window, layers, seed=1234, dist=dist)
    keys = past + 1
    out = torch.empty(max(t * g for t, _, g in PLAIN_READ_SHAPES), dtype=torch.float32,
                      device="cuda")
    b = kv_bytes(keys)

    class Reader:
        def __init__(self, shape):
            self.shape = shape

        def step(self, s, stream, append=True):
            t, u, g = self.shape
            rc = lib.nwd_bench_plain_read(wl.kc[s % layers].data_ptr(), wl.vc[s % layers].data_ptr(),
                                          HKV, wl.cap, keys, t, u, g, 1, out.data_ptr(),
                                          stream.cuda_stream, 0)
            if rc != 0:
                raise RuntimeError(f"nwd_bench_plain_read: hip error {rc}")

    by_shape = {}
    for shape in PLAIN_READ_SHAPES:
        _, ms = time_graph(torch, Reader(shape), launches, 8, reps=3)
        by_shape["x".join(map(str, shape))] = ms * 1e3 / launches
    best = min(by_shape, key=by_shape.get)
    us = by_shape[best]
    res = {"workload": "plain-read", "desc": EXTRA_WORKLOADS["plain-read"], "us_per_launch": us,
           "bytes": b, "gbs": b / (us * 1e-6) / 1e9, "frac": b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS,
           "best_shape": best, "us_by_shape_threads_x_loads_x_workgroups": by_shape}
    log(f"[bench] plain-read: {us:.3f} us per 134 MB launch ({res['gbs']:.1f} GB/s), shape {best}; "
        f"{ {k: round(v, 2) for k, v in by_shape.items()} }")
    wl.ctx.close()
    del wl, out
    torch.cuda.empty_cache()
    return res


def run_launch_gap(torch, launches: int = 512):
    """What a kernel boundary costs on the GPU (csrc/bench/nwd_stream_read.hip,
    empty_kernel): `launches` launches of a kernel whose workgroups only
    store one int, back to back in a HIP graph and as calls, with the decode
    split kernel's grid (192 x 256 threads), the merge's (32 x 64) and one
    workgroup. The graph figure is the per-launch floor of each kernel of a
    decode call (split, then merge)."""
    lib = ctypes.CDLL(str(BENCH_LIB))
    lib.nwd_bench_empty.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    sink = torch.empty(256, dtype=torch.int32, device="cuda")
    log(f"[bench] launch-gap: {launches} empty launches per shape")

    class Empty:
        def __init__(self, wgs, threads):
            self.shape = (wgs, threads)

        def step(self, s, stream, append=True):
            rc = lib.nwd_bench_empty(self.shape[0], self.shape[1], sink.data_ptr(), stream.cuda_stream)
            if rc != 0:
                raise RuntimeError(f"nwd_bench_empty: hip error {rc}")

    res = {"workload": "launch-gap", "desc": EXTRA_WORKLOADS["launch-gap"]}
    for name, shape in (("split_grid_192x256", (192, 256)), ("merge_grid_32x64", (32, 64)),
                        ("one_workgroup", (1, 64))):
        _, ms = time_graph(torch, Empty(*shape), launches, 16, reps=3)
        ms_calls = time_eager(torch, Empty(*shape), launches, reps=3)
        res[name] = {"graph_us_per_launch": ms * 1e3 / launches,
                     "calls_us_per_launch": ms_calls * 1e3 / launches}
    log(f"[bench] launch-gap: {rounded(res)}")
    return res


def run_mfma_ceiling(torch, iters: int = 2048, launches: int = 5):
    """The matrix-core ceiling under load and how much of the prefill's
    exponential work hides under its MFMAs (csrc/bench/nwd_mfma_ceiling.hip):
    256 x 512-thread workgroups running only 16x16x32 fp16 MFMAs (mode 0),
    only v_exp_f32 at the prefill's one exponential per two MFMAs (mode 1),
    both (mode 2), only v_fma_f32 at one per MFMA (mode 3) or MFMAs and
    FMAs (mode 4); with the shader clock each mode ran at. The hidden
    fractions are taken in shader cycles (time x clock), since the clock
    rises when the matrix cores are less busy."""
    lib = ctypes.CDLL(str(BENCH_LIB))
    lib.nwd_bench_mfma_ceiling.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                           ctypes.c_void_p, ctypes.c_void_p]
    log("[bench] mfma-ceiling")
    out = torch.empty(256 * 512, dtype=torch.float32, device="cuda")
    clk = torch.zeros(2, dtype=torch.int64, device="cuda")
    stream = torch.cuda.Stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    us, ghz = {}, {}
    for mode in (0, 1, 2, 3, 4):
        def launch():
            rc = lib.nwd_bench_mfma_ceiling(mode, iters, out.data_ptr(), clk.data_ptr(),
                                            stream.cuda_stream)
            if rc != 0:
                raise RuntimeError(f"nwd_bench_mfma_ceiling: hip error {rc}")
        for _ in range(2):
            launch()
        e0.record(stream)
        for _ in range(launches):
            launch()
        e1.record(stream)
        torch.cuda.synchronize()
        us[mode] = e0.elapsed_time(e1) * 1e3 / launches
        ticks, ref = (int(x) for x in clk.cpu())
        ghz[mode] = ticks / (ref / 100e6) / 1e9
    flops = 256 * 8 * iters * 32 * 2.0 * 16 * 16 * 32
    tflops = flops / (us[0] * 1e-6) / 1e12
    cyc = {m: us[m] * ghz[m] for m in us}  # thousands of shader cycles
    hid_exp = (cyc[0] + cyc[1] - cyc[2]) / cyc[1]
    hid_fma = (cyc[0] + cyc[3] - cyc[4]) / cyc[3]
    res = {"workload": "mfma-ceiling", "desc": EXTRA_WORKLOADS["mfma-ceiling"],
           "mfma_tflops": tflops, "mfma_frac_of_peak": tflops / MFMA_F16_PEAK_TFLOPS,
           "us": {"mfma": us[0], "exp": us[1], "mfma_and_exp": us[2], "fma": us[3],
                  "mfma_and_fma": us[4]},
           "clock_ghz": {"mfma": ghz[0], "exp": ghz[1], "mfma_and_exp": ghz[2], "fma": ghz[3],
                         "mfma_and_fma": ghz[4]},
           "exp_cycles_hidden_frac": hid_exp, "fma_cycles_hidden_frac": hid_fma}
    log(f"[bench] mfma-ceiling: {tflops:.0f} TFLOP/s at {ghz[0]:.2f} GHz; hidden under the MFMAs: "
        f"{hid_exp:.2f} of the exp cycles, {hid_fma:.2f} of the fma cycles; {res['us']}")
    del out, clk
    return res


def run_q4(torch, nw, name: str, steps: int, warmup: int, cpu: bool):
    """One 4-bit projection workload: us per call and weight-stream GB/s."""
    log(f"[bench] {name}: {steps} steps")
    wl = Q4LayerWorkload(torch, nw, name)
    warm_up(torch, wl, 0.1)
    wall, ms = time_graph(torch, wl, steps, warmup, reps=5)
    us = ms * 1e3 / steps
    gbs = wl.bytes_per_step() / (us * 1e-6) / 1e9
    kernel = {"qkv-append": "qkv_append_kernel (q/k/v 4-bit GEMVs, k/v into the fp16 caches)",
              "o-proj": "q4_gemv_kernel (accumulate epilogue: o_proj + residual)",
              "lm-head": "q4w_argmax_kernel + argmax_merge_kernel (lm_head + greedy pick)"}[name]
    res = {"workload": name, "desc": EXTRA_WORKLOADS[name], "us_per_step": us,
           "bytes_per_step": wl.bytes_per_step(), "gbs": gbs, "hbm_frac": gbs / HBM_PEAK_GBS,
           "traffic": measured_traffic(name), "wall_s": wall,
           "roofline": hbm_roofline(gbs, kernel, wl.bytes_per_step(), measured_traffic(name))}
    wl.ctx.close()
    del wl
    torch.cuda.empty_cache()
    if cpu:
        res["cpu_baseline"] = q4_cpu_baseline(name, budget_s=4.0)
    log(f"[bench] {name}: {res}")
    return res


def run_node_layer(past: int = 4096, steps: int = 64, warmup: int = 8):
    """The attention layers of a decode step driven from Node.js over the
    N-API addon (js/bench_layer.js: per token, the 4 attention layers of the
    Nano-4B shape, each qkv_append + append-decode + o_proj with the residual,
    as engine/runtime.js:386-393 and :447-469 dispatch them), run as a child
    process; None when node or the addon is absent."""
    import shutil
    import subprocess

    node = shutil.which("node")
    script = ROOT / "nemotron-webgpu-decode_amd" / "js" / "bench_layer.js"
    addon = ROOT / "nemotron-webgpu-decode_amd" / "lib" / "nwd_napi.node"
    if not node or not addon.exists():
        return None
    log(f"[bench] node-layer: past {past}, {steps} tokens")
    res = subprocess.run([node, str(script), str(past), str(steps), str(warmup)], capture_output=True,
                         text=True, timeout=180)
    if res.returncode != 0:
        log(f"[bench] node-layer failed: {res.stderr[-500:]}")
        return {"error": res.stderr[-300:]}
    r = json.loads(res.stdout.strip().splitlines()[-1])
    r["desc"] = ("node-layer: Nano-4B 40q/8kv, past 4096, a token's 4 attention layers from the "
                 "hidden state (q/k/v 4-bit + append + decode + o_proj + residual), every call "
                 "from JavaScript (eager) or the token replayed as a HIP graph")
    log(f"[bench] node-layer: {r}")
    return r


def measured_traffic(name: str):
    """HBM bytes per call of `name` from the committed counter summary
    (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs, scaled by the plain-copy
    calibration), or None if it has not been profiled."""
    f = ROOT / "profiles" / f"{name}_pmc.md"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("traffic_bytes_per_call:"):
            return int(float(line.split(":", 1)[1]))
    return None


def copy_bandwidth(torch, nbytes: int = 1 << 30, reps: int = 10):
    """Achievable HBM bandwidth of a plain device copy (torch copy_), read +
    write bytes per second; also the kernel used to calibrate the
    FETCH_SIZE / WRITE_SIZE counters (--copy-only)."""
    a = torch.empty(nbytes // 2, dtype=torch.float16, device="cuda").uniform_()
    b = torch.empty_like(a)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for _ in range(3):
            b.copy_(a)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            b.copy_(a)
        e1.record(s)
    torch.cuda.synchronize()
    gbs = 2 * nbytes * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del a, b
    torch.cuda.empty_cache()
    return round(gbs, 1)


def rounded(d):
    if isinstance(d, dict):
        return {k: rounded(v) for k, v in d.items() if k not in ("desc",)}
    if isinstance(d, float):
        # three decimals, or three significant digits for small magnitudes
        return round(d, 3) if d == 0.0 or abs(d) >= 0.01 else float(f"{d:.3g}")
    return d


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--workload", choices=["all", "general"] + sorted(WORKLOADS) + sorted(EXTRA_WORKLOADS),
                    default="all", help="all (default): the headline and every configuration; "
                    "a name: that workload alone (profiling)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-only", action="store_true",
                    help="only run 4 copies of 256 MiB (counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the decode-attention path runs on a single MI355X "
              "(--gpus 1); multi-GPU sharding is not built.", file=sys.stderr)
        sys.exit(2)

    import torch
    import nwd_attn as nw

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    if args.copy_only:
        log(f"[bench] copy 256 MiB x4: {copy_bandwidth(torch, 1 << 28, 4)} GB/s")
        return
    nw.load_library()
    hip = Hip()

    if args.workload != "all":
        w = args.workload
        if w in WORKLOADS:
            r = run_decode(torch, nw, hip, w, args.steps, args.warmup)
        elif w == "ragged-64":
            r = run_ragged(torch, nw, args.steps, args.warmup)
        elif w == "prefill-512":
            r = run_prefill(torch, nw, args.steps, args.warmup)
        elif w == "prefill-512-f32q":
            r = run_prefill(torch, nw, args.steps, args.warmup, q_dtype="f32", library=False)
        elif w == "stream-read":
            r = run_stream_read(torch, nw, args.steps)
        elif w == "plain-read":
            r = run_plain_read(torch, nw, args.steps)
        elif w == "mfma-ceiling":
            r = run_mfma_ceiling(torch)
        elif w == "launch-gap":
            r = run_launch_gap(torch)
        elif w == "general":
            r = run_general(torch, nw)
        else:
            r = run_q4(torch, nw, w, args.steps, args.warmup, cpu=not args.no_cpu_baseline)
        print(json.dumps(rounded(r)), flush=True)
        return

    head = run_decode(torch, nw, hip, "decode-32k", args.steps, args.warmup,
                      dec_steps=max(args.steps, SECONDARY_STEPS["decode-32k"]), other_kernels=(0, 1))
    configs = {
        "decode-32k-nano": run_decode(torch, nw, hip, "decode-32k-nano",
                                      SECONDARY_STEPS["decode-32k-nano"], 16, other_kernels=(0, 1)),
        "decode-153": run_decode(torch, nw, hip, "decode-153", SECONDARY_STEPS["decode-153"], 64),
        "decode-1k": run_decode(torch, nw, hip, "decode-1k", SECONDARY_STEPS["decode-1k"], 32,
                                other_splits=(16, 32)),
        "decode-4k": run_decode(torch, nw, hip, "decode-4k", SECONDARY_STEPS["decode-4k"], 32),
        "ragged-64": run_ragged(torch, nw, SECONDARY_STEPS["ragged-64"], 8),
        "prefill-512": run_prefill(torch, nw, SECONDARY_STEPS["prefill-512"], 4),
        "prefill-512-f32q": run_prefill(torch, nw, SECONDARY_STEPS["prefill-512"], 4, q_dtype="f32",
                                        library=False),
    }
    # the attention layer's 4-bit projections and the step's lm_head with its
    # greedy pick (the rows around the path), each with its roofline
    for q4 in ("qkv-append", "o-proj", "lm-head"):
        configs[q4] = run_q4(torch, nw, q4, SECONDARY_STEPS[q4], 8, cpu=not args.no_cpu_baseline)
    node_layer = run_node_layer()
    if node_layer is not None:
        configs["node-layer"] = node_layer
    general = run_general(torch, nw)
    stream = run_stream_read(torch, nw, SECONDARY_STEPS["stream-read"])
    plain = run_plain_read(torch, nw, SECONDARY_STEPS["plain-read"])
    gap = run_launch_gap(torch)
    ceiling = run_mfma_ceiling(torch)
    for k in ("prefill-512", "prefill-512-f32q"):
        pre = configs[k]["roofline"]
        pre["frac_of_mfma_ceiling"] = pre["achieved"] / ceiling["mfma_tflops"]
    for k in ("decode-32k-nano",):
        configs[k]["frac_of_plain_read"] = plain["us_per_launch"] / configs[k]["decode_us"]
    copy_gbs = copy_bandwidth(torch)
    log(f"[bench] device copy {copy_gbs} GB/s (read+write)")
    cpu = None
    if not args.no_cpu_baseline:
        host = host_info()
        log(f"[bench] cpu baselines on {host}")
        cpu = cpu_baseline(head["past"], head["window"], dist="outliers")
        cpu.update(host)
        log(f"[bench] cpu decode-32k: {cpu}")
        per_config = {
            "decode-153": lambda: cpu_baseline(152, 1, budget_s=3.0),
            "decode-4k": lambda: cpu_baseline(4096, 64, budget_s=5.0, dist="head-scale"),
            "ragged-64": cpu_baseline_ragged,
            "prefill-512": cpu_baseline_prefill,
        }
        for k, fn in per_config.items():
            configs[k]["cpu_baseline"] = dict(fn(), **host)
            log(f"[bench] cpu {k}: {configs[k]['cpu_baseline']}")

    us_step, gbs = head["us_per_step"], head["gbs"]
    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_step / 1e3, 6),
        "us_per_step": round(us_step, 3),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "storage_dtype": "f16",
        "data": "synthetic, seeded: fp16 Q N(0,1), K/V as the workload states",
        "config": {
            "workload": head["desc"],
            "batch": 1, "n_heads": H, "n_kv_heads": HKV, "head_dim": D,
            "past": head["past"], "window": head["window"],
            "layers": head["layers"], "decode_splits": head["splits"],
            "timing": "exactly `steps` append+attend steps timed with hipEvents on their "
                      "stream after a 0.25 s warm-up, two ways: as calls issued like a token "
                      "loop (median of 5 runs, behind 16 untimed calls so the GPU never waits "
                      "for the host) and replayed from a HIP graph (median of 3, behind an "
                      "untimed pre-roll graph); us_per_step is the lower, step_timing names it",
        },
        "step_timing": head["step_timing"],
        "calls_us_per_step": round(head["calls_us_per_step"], 3),
        "graph_us_per_step": round(head["graph_us_per_step"], 3),
        "eager_us_per_step": round(head["eager_us_per_step"], 3),
        "roofline": rounded(head["roofline"]),
        "decode_call": {"us": round(head["decode_us"], 3), "gbs": round(head["decode_gbs"], 1),
                        "frac": round(head["decode_gbs"] / HBM_PEAK_GBS, 4),
                        "split_kernel_us": round(head["split_kernel_us"], 3),
                        "split_kernel": head["split_kernel"],
                        "us_by_kernel": rounded(head.get("decode_us_by_kernel", {})),
                        # the call against the fastest plain read of the same bytes
                        "frac_of_plain_read": round(plain["us_per_launch"] / head["decode_us"], 4),
                        "split_kernel_frac_of_plain_read":
                            round(plain["us_per_launch"] / head["kernel_us"], 4)},
        "cpu_baseline": cpu,
        "configs": {k: rounded({kk: vv for kk, vv in v.items() if kk != "mean_kv_bytes"})
                    for k, v in configs.items()},
        "stream_read": rounded(stream),
        "plain_read": rounded(plain),
        "launch_gap": rounded(gap),
        "general_shapes": rounded(general),
        "mfma_ceiling": rounded(ceiling),
        "device_copy_gbs": copy_gbs,
        "wall_s_timed": round(head["wall_s"], 4),
        "library_source_sha256": nw.source_hash(),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
