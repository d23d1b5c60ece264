"""Build-time check of the decode kernels' inline-assembly transpose reads.

decode_mfma_kernel (csrc/nwd_decode_mfma.h, instantiated in nwd_decode.hip;
its head-64 form in nwd_decode_mfma64.hip) issues its eight (four) V^T
operand reads as inline `ds_read_b64_tr_b16` (lds_read_tr16_asm in
csrc/nwd_common.h), runs
the softmax, and only then waits for them with an inline
`s_waitcnt lgkmcnt(0)` (lds_reads_done). The compiler treats each read's
result as ready when the asm statement ends, so the code is correct only if
nothing touches a read's destination registers before that wait: no copy,
no move, no other use. This test compiles both units for gfx950 to AMD
assembly (code built here) and walks every path from each transpose read,
through branches, to the first `lgkmcnt(0)` wait, and fails if any
instruction on the way reads or writes one of the read's destination VGPRs.
"""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "nemotron-webgpu-decode_amd" / "csrc"
HIPCC = "/opt/rocm/bin/hipcc"

_VREG = re.compile(r"\bv(\d+)\b")
_VRANGE = re.compile(r"\bv\[(\d+):(\d+)\]")
_LABEL = re.compile(r"^(\.?[A-Za-z_][\w.$]*):")


def _regs(operands: str) -> set:
    out = set()
    for a, b in _VRANGE.findall(operands):
        out.update(range(int(a), int(b) + 1))
    for a in _VREG.findall(_VRANGE.sub(" ", operands)):
        out.add(int(a))
    return out


def _parse(asm: str):
    """Instructions as (mnemonic, operands) with label -> index."""
    insts, labels = [], {}
    for raw in asm.splitlines():
        line = raw.split(";", 1)[0].strip()
        if not line:
            continue
        m = _LABEL.match(line)
        if m:
            labels[m.group(1)] = len(insts)
            continue
        if line.startswith("."):
            continue
        parts = line.split(None, 1)
        insts.append((parts[0], parts[1] if len(parts) > 1 else ""))
    return insts, labels


def _violations(insts, labels):
    found, checked = [], 0
    for i, (mn, ops) in enumerate(insts):
        if mn != "ds_read_b64_tr_b16":
            continue
        checked += 1
        dest = _regs(ops.split(",")[0])
        stack, seen = [i + 1], set()
        while stack:
            j = stack.pop()
            while j < len(insts) and j not in seen:
                seen.add(j)
                m2, o2 = insts[j]
                if m2 == "s_waitcnt" and "lgkmcnt(0)" in o2:
                    break
                if m2 == "s_endpgm":
                    break
                if m2 != "ds_read_b64_tr_b16" and _regs(o2) & dest:
                    found.append((i, j, f"{mn} {ops}", f"{m2} {o2}"))
                if m2.startswith("s_branch"):
                    stack.append(labels[o2.strip()])
                    break
                if m2.startswith("s_cbranch"):
                    stack.append(labels[o2.strip()])
                j += 1
    return found, checked


def test_checker_flags_a_use_before_the_wait():
    """The walk itself: a move of a destination register before the wait,
    also on a branch path, is flagged; a use after the wait is not."""
    ok = """
    ds_read_b64_tr_b16 v[10:11], v5
    v_add_f32 v1, v2, v3
    s_cbranch_vccz .LBB0_2
    v_mov_b32 v4, v6
.LBB0_2:
    s_waitcnt lgkmcnt(0)
    v_mov_b32 v4, v10
    s_endpgm
"""
    bad_branch = ok.replace("v_mov_b32 v4, v6", "s_branch .LBB0_3").replace(
        "    s_endpgm\n", "    s_endpgm\n.LBB0_3:\n    v_mov_b32 v7, v[11:12]\n    s_branch .LBB0_2\n")
    assert _violations(*_parse(ok)) == ([], 1)
    found, _ = _violations(*_parse(bad_branch))
    assert len(found) == 1 and "v[11:12]" in found[0][3]


@pytest.mark.skipif(shutil.which(HIPCC) is None and not Path(HIPCC).exists(), reason="hipcc absent")
@pytest.mark.parametrize("unit", ["nwd_decode.hip", "nwd_decode_mfma64.hip"])
def test_transpose_read_registers_untouched_until_the_wait(tmp_path, unit):
    out = tmp_path / "decode.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
           "-Xclang", "-packed-fp32-ops", f"-I{ROOT / 'include'}", "--cuda-device-only", "-S",
           str(CSRC / unit), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stderr[-3000:]
    found, checked = _violations(*_parse(out.read_text()))
    assert checked >= 8, f"only {checked} transpose reads found"
    assert not found, found[:5]
