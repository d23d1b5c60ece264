"""Builds libnwd_attn.so (the gfx950 HIP kernels + C ABI) in-tree.

Usage: python nemotron-webgpu-decode_amd/build.py [--jobs N]

Each .hip file under csrc/ is compiled to an object with hipcc for gfx950
only, then linked into lib/libnwd_attn.so. Packed-fp32 instruction selection
is disabled for the device code (-packed-fp32-ops).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "lib" / "libnwd_attn.so"
BENCH_LIB = PKG / "lib" / "libnwd_bench.so"  # measurement kernels for bench.py
ADDON = PKG / "lib" / "nwd_napi.node"
INCLUDE = PKG.parent / "include"
NODE_INCLUDE = Path(os.environ.get("NODE_INCLUDE", "/usr/include/node"))

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-command-line-argument",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


# Per-source flags. The prefill kernel's scores are finite or -inf (masked),
# so its max reductions need no NaN quieting: without it each fmaxf operand
# costs an extra v_max (measured 12% of the kernel's time).
FILE_FLAGS = {"nwd_prefill.hip": ["-fno-honor-nans"]}


def _compile(src: Path) -> Path:
    out = OBJ / (src.stem + ".o")
    cmd = [HIPCC, *DEVICE_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msg = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{msg}")
    if msg.strip():
        print(msg, file=sys.stderr)
    return out


def build(jobs: int | None = None) -> Path:
    """Compiles every csrc/*.hip and links lib/libnwd_attn.so; returns its path."""
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found: the HIP library cannot be built")
    OBJ.mkdir(exist_ok=True)
    LIB.parent.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = jobs or min(len(sources), os.cpu_count() or 1, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB)
    build_bench()
    return LIB


def build_bench() -> Path:
    """Links lib/libnwd_bench.so from csrc/bench/*.hip: kernels that only
    bench.py uses (the stream-read ceiling), kept out of the product ABI."""
    objs = [_compile(src) for src in sorted((CSRC / "bench").glob("*.hip"))]
    tmp = BENCH_LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"bench library link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, BENCH_LIB)
    return BENCH_LIB


def build_addon() -> Path | None:
    """Builds the Node.js N-API addon (lib/nwd_napi.node) over libnwd_attn.so
    with g++ (host code only). Returns None when the Node headers are absent."""
    if not (NODE_INCLUDE / "node_api.h").exists():
        return None
    src = PKG / "addon" / "nwd_napi.cc"
    tmp = ADDON.with_suffix(".node.tmp")
    cmd = ["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall",
           "-D__HIP_PLATFORM_AMD__", "-DNODE_GYP_MODULE_NAME=nwd_napi",
           f"-I{NODE_INCLUDE}", f"-I{INCLUDE}", "-I/opt/rocm/include", str(src),
           "-o", str(tmp), f"-L{LIB.parent}", "-lnwd_attn", "-L/opt/rocm/lib", "-lamdhip64",
           "-Wl,-rpath,$ORIGIN", "-Wl,-rpath,/opt/rocm/lib"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"addon build failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, ADDON)
    return ADDON


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    print(build(ap.parse_args().jobs))
    print(build_addon())
