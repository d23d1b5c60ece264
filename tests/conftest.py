"""Shared pytest setup: the `gpu` marker and import paths.

`-m "not gpu"` runs the oracle checks, the host-side validation and the
library-load checks on any machine; `-m gpu` runs the parity tests of the
HIP library on an MI355X.
"""
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "nemotron-webgpu-decode_amd", ROOT / "oracle", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")
