"""The Node.js host (js/attention_layer.js + N-API addon) driving the library
the way DecodeEngine drives its attention layers (engine/runtime.js:635-648),
checked against the oracle: every token, every attention layer."""
import json
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle
from attn_cases import max_abs

ROOT = Path(__file__).resolve().parent.parent
JS = ROOT / "nemotron-webgpu-decode_amd" / "js"

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")]


def _run(tmp_path, heads, kv_heads, tokens, max_seq):
    out = tmp_path / f"run_{heads}_{tokens}"
    print(f"node check_attention {heads}/{kv_heads} tokens={tokens}", flush=True)
    res = subprocess.run(["node", str(JS / "check_attention.js"), str(out), str(heads),
                          str(kv_heads), str(tokens), str(max_seq)],
                         capture_output=True, text=True, timeout=180)
    assert res.returncode == 0, res.stdout + res.stderr
    man = json.loads((out / "manifest.json").read_text())
    n_l = len(man["layers"])
    D = man["headDim"]
    q = np.fromfile(out / "q.f32", np.float32).reshape(tokens, n_l, heads, D)
    k = np.fromfile(out / "k.f32", np.float32).reshape(tokens, n_l, kv_heads, D)
    v = np.fromfile(out / "v.f32", np.float32).reshape(tokens, n_l, kv_heads, D)
    o = np.fromfile(out / "o.f32", np.float32).reshape(tokens, n_l, heads, D)
    return man, q, k, v, o


@pytest.mark.parametrize("heads,kv_heads,tokens,max_seq", [(40, 8, 153, 256), (32, 8, 256, 256)])
def test_node_host_matches_oracle(tmp_path, heads, kv_heads, tokens, max_seq):
    man, q, k, v, o = _run(tmp_path, heads, kv_heads, tokens, max_seq)
    # the cache holds the f32 rows rounded to fp16 (kv_append's rule)
    kh = oracle.f16_to_f32(oracle.f32_to_f16(k))
    vh = oracle.f16_to_f32(oracle.f32_to_f16(v))
    worst = 0.0
    steps = range(tokens) if tokens <= 160 else list(range(0, tokens, 7)) + [tokens - 1]
    for t in steps:
        for li in range(len(man["layers"])):
            want = oracle.sparse_attn_f32(q[t, li], kh[:t + 1, li], vh[:t + 1, li], threads=0)
            worst = max(worst, max_abs(o[t, li], want))
    assert worst < 2e-3, worst
    if tokens == max_seq:  # engine/runtime.js:448: the next step must throw
        assert "exceeds maxSeq" in man["guard"]
