"""Benchmark of the decode-attention path on one MI355X.

One "step" is one attention-layer step of the reference engine
(engine/runtime.js:389-391: kv_append for K, for V, then sparse_attn): here
one nwd_append_decode launch that writes the new token's K and V rows and
attends over pos+1 keys. Default workload: 32 query heads, 8 KV heads, head_dim
128, fp16 cache, 4096 cached tokens, 64 generated tokens per window. To keep
the 256 MB Infinity Cache from serving the KV reads, each step uses the next
of 32 distinct layer caches (545 MB in total), the way a model walks its
layers; step s uses layer s % 32 and token (s // 32) % 64, at position
4096 + token.

Inputs are resident in HBM before timing starts and the steps are replayed
from a HIP graph (captured once), so the timed region is device work plus the
graph's launch gaps. Prints ONE JSON line.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "nemotron-webgpu-decode_amd"))

METRIC = "µs/attention-layer step + achieved KV-read GB/s (% of HBM peak), 1×MI355X"
HBM_PEAK_GBS = 8000.0
H, HKV, D = 32, 8, 128


def kv_bytes(L: int) -> int:
    """Algorithmic KV-read bytes of one decode over L keys: L*Hkv*D*(K+V)*2 B."""
    return L * HKV * D * 2 * 2


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class DecodeWorkload:
    """`layers` distinct caches of `past` random tokens plus `window` tokens
    of new rows and queries, all on the device."""

    def __init__(self, torch, nw, past: int, window: int, layers: int, seed: int):
        self.torch, self.past, self.window, self.layers = torch, past, window, layers
        self.cap = past + window
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        f16 = torch.float16

        def rnd(*shape):
            return torch.randn(*shape, generator=g, device="cuda", dtype=torch.float32).to(f16)

        self.kc = [rnd(1, HKV, self.cap, D) for _ in range(layers)]
        self.vc = [rnd(1, HKV, self.cap, D) for _ in range(layers)]
        self.knew = rnd(window, 1, HKV, D)
        self.vnew = rnd(window, 1, HKV, D)
        self.q = rnd(window, 1, H, D)
        self.out = torch.empty(1, H, D, dtype=f16, device="cuda")
        self.pos = torch.arange(past, past + window, dtype=torch.int32, device="cuda")
        self.ctx = nw.AttnContext(H, HKV, self.cap)

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


def time_graph(torch, wl: DecodeWorkload, steps: int, warmup: int, append=True):
    """Warm up eagerly, capture `steps` steps into a HIP graph, replay it once
    untimed and once timed. Returns (wall seconds, device ms) of the timed replay."""
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for s in range(warmup):
            wl.step(s, stream, append)
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for s in range(steps):
            wl.step(s, stream, append)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):  # replay() launches on the current stream
        graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start.record(stream)
        graph.replay()
        end.record(stream)
        torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, start.elapsed_time(end)


def time_eager(torch, wl: DecodeWorkload, steps: int):
    stream = torch.cuda.Stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for s in range(steps):
        wl.step(s, stream)
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end)


def cpu_baseline(past: int, window: int, budget_s: float = 20.0):
    """The oracle (op-for-op CPU restatement of kernels/sparse_attn.wgsl +
    kv_append.wgsl, f32, per-head workgroups over OpenMP threads) on the same
    workload, for as many steps of the window as fit in `budget_s`."""
    import numpy as np

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    threads = oracle.max_threads()
    g = np.random.Generator(np.random.PCG64(7))
    cap = past + window
    k = g.standard_normal((cap, HKV, D), dtype=np.float32)
    v = g.standard_normal((cap, HKV, D), dtype=np.float32)
    q = g.standard_normal((window, H, D), dtype=np.float32)
    kc = np.zeros(cap * HKV * D, np.float32)
    vc = np.zeros(cap * HKV * D, np.float32)
    kc[: past * HKV * D] = k[:past].reshape(-1)
    vc[: past * HKV * D] = v[:past].reshape(-1)
    done, nbytes = 0, 0
    t0 = time.perf_counter()
    for i in range(window):
        p = past + i
        oracle.kv_append_f32(k[p], kc, p, HKV, D)
        oracle.kv_append_f32(v[p], vc, p, HKV, D)
        L = p + 1
        oracle.sparse_attn_f32(q[i], kc[: L * HKV * D].reshape(L, HKV, D),
                               vc[: L * HKV * D].reshape(L, HKV, D), threads=0)
        done += 1
        nbytes += kv_bytes(L)
        if time.perf_counter() - t0 > budget_s:
            break
    dt = time.perf_counter() - t0
    return {
        "value": round(nbytes / dt / 1e9, 3),
        "unit": "GB/s",
        "us_per_step": round(dt / done * 1e6, 1),
        "cores": threads,
        "kind": "port",
        "sample": f"{done} of the {window} append+attend steps at past {past} "
                  f"(L = {past + 1}..{past + done}), one layer, f32 token-major cache",
    }


def measure_32k(torch, nw):
    """Split-K at 32K context: 4 rotating layer caches (537 MB), 64 steps."""
    wl = DecodeWorkload(torch, nw, past=32768, window=64, layers=4, seed=33)
    steps = 64
    _, ms = time_graph(torch, wl, steps, warmup=8)
    _, ms_dec = time_graph(torch, wl, steps, warmup=0, append=False)
    b = wl.mean_kv_bytes(steps)
    res = {
        "workload": "decode-32k: past 32768, 4 layer caches rotated, 64 steps",
        "us_per_step": round(ms * 1e3 / steps, 3),
        "decode_us": round(ms_dec * 1e3 / steps, 3),
        "kv_read_gbs": round(b / (ms_dec * 1e-3 / steps) / 1e9, 1),
        "splits": wl.ctx.decode_splits(1, wl.cap),
    }
    res["hbm_frac"] = round(res["kv_read_gbs"] / HBM_PEAK_GBS, 4)
    wl.ctx.close()
    return res


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2048)
    ap.add_argument("--warmup", type=int, default=256)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-32k", action="store_true")
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

    past, window, layers = 4096, 64, 32
    log(f"[bench] setup: past={past} window={window} layers={layers}")
    wl = DecodeWorkload(torch, nw, past, window, layers, seed=1234)
    log(f"[bench] timing {args.steps} steps (graph), warmup {args.warmup}")
    wall, ms = time_graph(torch, wl, args.steps, args.warmup)
    us_step = ms * 1e3 / args.steps
    mean_b = wl.mean_kv_bytes(args.steps)
    gbs = mean_b / (us_step * 1e-6) / 1e9
    log(f"[bench] step: {us_step:.3f} us, {gbs:.1f} GB/s")
    # the dominant kernel work alone: decode calls only, same rotation
    _, ms_dec = time_graph(torch, wl, args.steps, 0, append=False)
    dec_us = ms_dec * 1e3 / args.steps
    achieved = mean_b / (dec_us * 1e-6) / 1e9
    eager_ms = time_eager(torch, wl, min(args.steps, 512))
    eager_us = eager_ms * 1e3 / min(args.steps, 512)
    log(f"[bench] decode-only {dec_us:.3f} us ({achieved:.1f} GB/s); eager step {eager_us:.3f} us")
    splits = wl.ctx.decode_splits(1, wl.cap)
    wl.ctx.close()
    del wl
    torch.cuda.empty_cache()

    extra = None
    if not args.no_32k:
        log("[bench] 32k split-K")
        extra = measure_32k(torch, nw)
        log(f"[bench] 32k: {extra}")
    copy_gbs = copy_bandwidth(torch)
    log(f"[bench] device copy {copy_gbs} GB/s (read+write)")
    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline")
        cpu = cpu_baseline(past, window)
        log(f"[bench] cpu: {cpu}")

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
        "data": "synthetic (seeded N(0,1) fp16 K/V/Q)",
        "config": {
            "workload": "decode-4k-64steps: B=1, 32q/8kv/d128, past 4096, append+attend "
                        "per step, 32 layer caches rotated",
            "batch": 1, "n_heads": H, "n_kv_heads": HKV, "head_dim": D, "past": past,
            "window": window, "layers": layers, "decode_splits": splits,
            "timing": "one HIP graph replay of `steps` steps, hipEvents",
        },
        "eager_us_per_step": round(eager_us, 3),
        "roofline": {
            "bound": "hbm",
            "kernel": "nwd_decode_attn = decode_split_kernel + decode_merge_kernel",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "decode_us": round(dec_us, 3),
        },
        "cpu_baseline": cpu,
        "decode_32k": extra,
        "device_copy_gbs": copy_gbs,
        "wall_s_timed": round(wall, 4),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
