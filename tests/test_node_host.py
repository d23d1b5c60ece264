"""The Node.js host (js/attention_layer.js over the N-API addon) loads and
reports the library's validation errors. No kernel is launched here."""
import json
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
JS = ROOT / "nemotron-webgpu-decode_amd" / "js"
ADDON = ROOT / "nemotron-webgpu-decode_amd" / "lib" / "nwd_napi.node"

pytestmark = pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")


def _node(script: str) -> str:
    res = subprocess.run(["node", "-e", script], cwd=JS, capture_output=True, text=True, timeout=60)
    assert res.returncode == 0, res.stderr
    return res.stdout


def test_addon_exports():
    assert ADDON.exists(), "build the addon: python nemotron-webgpu-decode_amd/build.py"
    out = _node("const a = require('../lib/nwd_napi.node'); console.log(JSON.stringify(Object.keys(a)))")
    names = set(json.loads(out))
    assert {"create", "destroy", "cacheBytes", "malloc", "free", "upload", "download", "zero",
            "sync", "kvAppend", "decode", "appendDecode", "prefill", "deviceStatus",
            "q4Gemv", "qkvAppend", "argmax", "lmHeadArgmax", "setI32", "captureBegin",
            "captureEnd", "graphLaunch", "graphDestroy"} <= names


def test_create_errors_are_thrown_with_the_library_message():
    out = _node("""
const a = require('../lib/nwd_napi.node');
const msgs = [];
for (const d of [{nHeads: 30, nKvHeads: 8, maxSeq: 16}, {nHeads: 24, nKvHeads: 8, headDim: 513, maxSeq: 16},
                 {nHeads: 32, nKvHeads: 8, maxSeq: 0}]) {
  try { a.create(d); msgs.push('no-throw'); } catch (e) { msgs.push(e.message); }
}
try { a.decode(null, 0n, 0n, 0n, 0n, 0n, 1, 0); msgs.push('no-throw'); } catch (e) { msgs.push(e.message); }
try { a.q4Gemv(null, 0n, {}, 0n, 1, 0); msgs.push('no-throw'); } catch (e) { msgs.push(e.message); }
try { a.qkvAppend(null, 0n, {}, {}, {}, 0n, 0n, 0n, 0n, 1); msgs.push('no-throw'); } catch (e) { msgs.push(e.message); }
try { a.argmax(null, 0n, 16, 0n, 1); msgs.push('no-throw'); } catch (e) { msgs.push(e.message); }
try { a.lmHeadArgmax(null, 0n, {}, null, 0n, 1); msgs.push('no-throw'); } catch (e) { msgs.push(e.message); }
console.log(JSON.stringify(msgs));
""")
    m = json.loads(out)
    assert "not a multiple of n_kv_heads" in m[0]
    assert "head_dim 513 exceeds 512" in m[1]
    assert "sizes must be positive" in m[2]
    assert m[3].startswith("decode:")
    assert m[4].startswith("q4Gemv:") and m[5].startswith("qkvAppend:")
    assert m[6].startswith("argmax:") and m[7].startswith("lmHeadArgmax:")


def test_js_module_parses():
    res = subprocess.run(["node", "--check", str(JS / "attention_layer.js")], capture_output=True,
                         text=True, timeout=60)
    assert res.returncode == 0, res.stderr
    res = subprocess.run(["node", "--check", str(JS / "check_attention.js")], capture_output=True,
                         text=True, timeout=60)
    assert res.returncode == 0, res.stderr
    for script in ("check_layer.js", "check_head.js", "bench_layer.js"):
        res = subprocess.run(["node", "--check", str(JS / script)], capture_output=True,
                             text=True, timeout=60)
        assert res.returncode == 0, res.stderr
