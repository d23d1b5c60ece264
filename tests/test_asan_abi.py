"""The C ABI's host code under AddressSanitizer and LeakSanitizer, without a
GPU: lib/asan/nwd_abi_asan (built by nemotron-webgpu-decode_amd/build.py
--variants from tests/asan/nwd_abi_asan.cc, linked with the ASan runtime)
runs every validation and error path of include/nwd_attn.h that returns
before the HIP runtime is used. Any ASan or leak report fails the run."""
import os
import subprocess

import nwd_attn as nw

DRIVER = nw.PKG_DIR / "lib" / "asan" / "nwd_abi_asan"


def test_abi_validation_paths_under_asan():
    assert DRIVER.exists(), f"{DRIVER} is missing: python nemotron-webgpu-decode_amd/build.py --variants"
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1")
    res = subprocess.run([str(DRIVER), "cpu"], capture_output=True, text=True, timeout=60, env=env)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "Sanitizer" not in res.stderr, res.stderr
    assert "cpu checks:" in res.stdout and ", 0 failed" in res.stdout, res.stdout
