"""Builds libnwd_attn.so (the gfx950 HIP kernels + C ABI) in-tree.

Usage: python nemotron-webgpu-decode_amd/build.py [--jobs N] [--variants]

Each .hip file under csrc/ is compiled to an object with hipcc for gfx950
only, then linked into lib/libnwd_attn.so. Packed-fp32 instruction selection
is disabled for the device code (-packed-fp32-ops).

Two debug variants of the same sources (--variants, or build_variants()):
  lib/check/libnwd_attn.so  -DNWD_CHECK: every kernel store checks its
                            address against its buffer, drops it when it is
                            outside and flags it in the device status word;
  lib/asan/libnwd_attn.so   host code built with AddressSanitizer (device
                            code unchanged: GPU ASan is not used), plus
                            lib/asan/nwd_abi_asan, a host driver program
                            linked with the ASan runtime that exercises the
                            C ABI (tests/asan/nwd_abi_asan.cc).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import hashlib
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "lib" / "libnwd_attn.so"
CHECK_LIB = PKG / "lib" / "check" / "libnwd_attn.so"
ASAN_LIB = PKG / "lib" / "asan" / "libnwd_attn.so"
ASAN_DRIVER = PKG / "lib" / "asan" / "nwd_abi_asan"
ASAN_DRIVER_SRC = PKG.parent / "tests" / "asan" / "nwd_abi_asan.cc"
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
FILE_FLAGS = {"nwd_prefill.hip": ["-fno-honor-nans"], "nwd_prefill_d64.hip": ["-fno-honor-nans"],
              "nwd_prefill_wide.hip": ["-fno-honor-nans"]}

# Host-only AddressSanitizer: -Xarch_host sits right before each -fsanitize=,
# so the device code is built exactly as in the product library.
ASAN_HOST_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]


def source_files() -> list:
    """The files nwd_source_hash covers, those libnwd_attn.so is built from:
    csrc/*.hip and *.h in name order, then include/nwd_attn.h (the measurement
    kernels under csrc/bench/ go to another library)."""
    files = sorted(p for p in CSRC.glob("*") if p.suffix in (".hip", ".h"))
    return files + [INCLUDE / "nwd_attn.h"]


def source_hash() -> str:
    """SHA-256 over each source file's path (relative to the repository
    root), a NUL and its bytes; the value nwd_source_hash() returns for a
    library built from these files."""
    h = hashlib.sha256()
    root = PKG.parent
    for f in source_files():
        h.update(f.relative_to(root).as_posix().encode() + b"\0")
        h.update(f.read_bytes())
    return h.hexdigest()


def _compile(src: Path, objdir: Path = OBJ, extra: tuple = ()) -> Path:
    out = objdir / (src.stem + ".o")
    if src.name == "nwd_api.hip":
        extra = (*extra, f'-DNWD_SOURCE_HASH="{source_hash()}"')
    cmd = [HIPCC, *DEVICE_FLAGS, *FILE_FLAGS.get(src.name, []), *extra, "-c", str(src), "-o",
           str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msg = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{msg}")
    if msg.strip():
        print(msg, file=sys.stderr)
    return out


def _sources() -> list:
    """csrc/*.hip, the largest first: the longest compiles start at once."""
    return sorted(CSRC.glob("*.hip"), key=lambda p: (-p.stat().st_size, p.name))


def _check_hipcc() -> None:
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found: the HIP library cannot be built")


def _link(lib: Path, objs: list, link_extra: tuple = ()) -> Path:
    lib.parent.mkdir(parents=True, exist_ok=True)
    tmp = lib.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *link_extra, "-o", str(tmp),
           *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of {lib.name} failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, lib)
    return lib


def _build_lib(lib: Path, objdir: Path, extra: tuple = (), link_extra: tuple = (),
               jobs: int | None = None) -> Path:
    _check_hipcc()
    objdir.mkdir(parents=True, exist_ok=True)
    sources = _sources()
    jobs = jobs or min(len(sources), os.cpu_count() or 1, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, objdir, extra), sources))
    return _link(lib, sorted(objs), link_extra)


def build(jobs: int | None = None) -> Path:
    """Compiles every csrc/*.hip and links lib/libnwd_attn.so; returns its path."""
    _build_lib(LIB, OBJ, jobs=jobs)
    build_bench()
    return LIB


def build_check(jobs: int | None = None) -> Path:
    """lib/check/libnwd_attn.so: the kernels with -DNWD_CHECK store checks."""
    return _build_lib(CHECK_LIB, OBJ / "check", ("-DNWD_CHECK",), jobs=jobs)


def build_asan(jobs: int | None = None) -> Path:
    """lib/asan/libnwd_attn.so (host code under AddressSanitizer) and the
    host driver lib/asan/nwd_abi_asan linked against it. The shared library
    leaves the ASan runtime to the program that loads it: the driver links it
    in, so nothing is preloaded."""
    _build_lib(ASAN_LIB, OBJ / "asan", tuple(ASAN_HOST_FLAGS), jobs=jobs)
    _build_asan_driver()
    return ASAN_LIB


def _build_asan_driver() -> None:
    tmp = ASAN_DRIVER.with_suffix(".tmp")
    # a host-only program (no .hip source): hipcc drives clang, whose ASan
    # runtime matches the library's instrumentation
    cmd = [HIPCC, "-O1", "-g", "-std=c++17", *ASAN_HOST_FLAGS, f"-I{INCLUDE}",
           str(ASAN_DRIVER_SRC), "-o", str(tmp), f"-L{ASAN_LIB.parent}", "-lnwd_attn",
           "-Wl,-rpath,$ORIGIN", "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"ASan driver build failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, ASAN_DRIVER)


def build_variants(jobs: int | None = None) -> list:
    """Both debug variants; each compiles every source again. The two builds
    run side by side: each is bound by its longest source (nwd_decode_hd.hip)."""
    with cf.ThreadPoolExecutor(max_workers=2) as ex:
        check = ex.submit(build_check, jobs)
        asan = ex.submit(build_asan, jobs)
        return [check.result(), asan.result()]


def build_all(jobs: int | None = None) -> list:
    """The product library and both debug variants from one pool of compile
    jobs (every source three times, the largest first), then their links,
    the ASan driver and the bench library: about the time of the product
    build plus a third, where build() and build_variants() in turn take
    about twice it. Returns the three library paths."""
    _check_hipcc()
    forms = [(LIB, OBJ, ()), (CHECK_LIB, OBJ / "check", ("-DNWD_CHECK",)),
             (ASAN_LIB, OBJ / "asan", tuple(ASAN_HOST_FLAGS))]
    for _, objdir, _ in forms:
        objdir.mkdir(parents=True, exist_ok=True)
    tasks = [(src, objdir, extra) for src in _sources() for _, objdir, extra in forms]
    jobs = jobs or min(len(tasks), os.cpu_count() or 1, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda t: _compile(*t), tasks))
    libs = []
    for i, (lib, _, _) in enumerate(forms):
        libs.append(_link(lib, sorted(objs[i::len(forms)])))
    _build_asan_driver()
    build_bench()
    return libs


def build_bench() -> Path:
    """Links lib/libnwd_bench.so from csrc/bench/*.hip: kernels that only
    bench.py uses (the stream-read ceiling), kept out of the product ABI."""
    OBJ.mkdir(exist_ok=True)
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
    ap.add_argument("--variants", action="store_true",
                    help="also build lib/check and lib/asan (debug variants)")
    args = ap.parse_args()
    if args.variants:
        print(build_all(args.jobs))
    else:
        print(build(args.jobs))
    print(build_addon())
