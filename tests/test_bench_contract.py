"""The benchmark's command-line contract and the entry points, on the CPU:
more than one GPU is refused with a message, a missing GPU fails loudly,
and the workloads are the shapes the measurements are quoted on."""
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _run(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True,
                          text=True, timeout=300, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr or "single MI355X" in r.stderr
    assert r.stdout == ""


def test_no_gpu_fails_loudly():
    import torch
    if torch.cuda.is_available():
        return  # only meaningful where no GPU is visible
    r = _run("--steps", "1", "--warmup", "0")
    assert r.returncode == 1
    assert "needs a GPU" in r.stderr
    assert r.stdout == ""


def test_workload_shapes():
    sys.path.insert(0, str(ROOT))
    import bench
    assert bench.WORKLOADS["decode-4k"][:2] == (4096, 64)
    assert bench.WORKLOADS["decode-32k"][:2] == (32768, 64)
    assert bench.WORKLOADS["decode-153"][:2] == (152, 1)  # L = 153 every step
    assert (bench.H, bench.HKV, bench.D) == (32, 8, 128)
    assert bench.HBM_PEAK_GBS == 8000.0
    # 4 H D sum_i (P + i + 1) for 512 queries onto 8192 cached tokens
    flops = 4.0 * 32 * 128 * sum(8192 + i + 1 for i in range(512))
    assert abs(flops - 7.087e10) / 7.087e10 < 1e-3


def test_entry_points_exist():
    sys.path.insert(0, str(ROOT))
    import __graft_entry__ as g
    assert callable(g.build) and callable(g.smoke)
