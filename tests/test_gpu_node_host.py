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
from q4_cases import gemv_f64

ROOT = Path(__file__).resolve().parent.parent
JS = ROOT / "nemotron-webgpu-decode_amd" / "js"

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")]


def _run(tmp_path, heads, kv_heads, tokens, max_seq, chunks="", head_dim=128):
    out = tmp_path / f"run_{heads}_{tokens}_{chunks.replace(',', '-')}_{head_dim}"
    print(f"node check_attention {heads}/{kv_heads}/d{head_dim} tokens={tokens} chunks={chunks}",
          flush=True)
    res = subprocess.run(["node", str(JS / "check_attention.js"), str(out), str(heads),
                          str(kv_heads), str(tokens), str(max_seq), chunks, str(head_dim)],
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


@pytest.mark.parametrize("heads,kv_heads,tokens,max_seq,chunks,head_dim", [
    (40, 8, 153, 256, "", 128),
    (32, 8, 256, 256, "", 128),
    # a 101-token prompt as two prefill chunks, then decode steps
    (40, 8, 153, 256, "37,64", 128),
    # the whole capacity through prefill chunks, then both guards
    (32, 8, 256, 256, "1,127,128", 128),
    # other head layouts: head size 96 with group 3 (padded group, padded
    # rows), head size 64 with group 3 through prefill chunks first, head
    # size 256 (the head-256 prefill) and group 16 (two groups of 8 per KV
    # head) through prefill chunks
    (6, 2, 90, 128, "", 96),
    (12, 4, 70, 96, "17,20", 64),
    (4, 2, 60, 64, "9,30", 256),
    (32, 2, 40, 48, "5,19", 128),
])
def test_node_host_matches_oracle(tmp_path, heads, kv_heads, tokens, max_seq, chunks, head_dim):
    """Every token through the decode step, or the first ones through chunked
    prefill (query t of a chunk attends keys 0..t, the reference's result for
    a prompt run token by token)."""
    man, q, k, v, o = _run(tmp_path, heads, kv_heads, tokens, max_seq, chunks, head_dim)
    assert man["headDim"] == head_dim
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
    assert "no prompt chunk open" in man["chunkGuard"]
    if tokens == max_seq:  # engine/runtime.js:448: the next step must throw
        assert "exceeds maxSeq" in man["guard"]
        assert "exceeds maxSeq" in man["prefillGuard"]


@pytest.mark.parametrize("mode", ["eager", "graph", "prefill"])
def test_node_host_full_layer_from_hidden_state(tmp_path, mode):
    """js/check_layer.js: one attention layer per token from the normalised
    hidden state (q/k/v projections + kv_append, attention, o_proj + residual
    add, engine/runtime.js:386-393) with 4-bit weights. Checked stage by
    stage against the oracle: the attention output against the chain q4 GEMV
    -> fp16 cache -> sparse_attn restatement (2e-3), and the residual against
    h_in + o_proj(attention output) in float64 (1e-6 of sum |w a|, plus one
    f32 rounding of the add). `graph`: the token's calls are captured once
    into a HIP graph and replayed every token (AttentionSlice.captureToken,
    attention sized for the capacity). `prefill`: the 12 tokens as two prompt
    chunks (AttentionSlice.prefillLayerFromHidden: n-row GEMVs, kv_append,
    the causal prefill, o_proj over the n rows), with the same checks."""
    out = tmp_path / "layer"
    print(f"node check_layer hidden=512 tokens=12 {mode}", flush=True)
    res = subprocess.run(["node", str(JS / "check_layer.js"), str(out), "512", "12", mode],
                         capture_output=True, text=True, timeout=180)
    assert res.returncode == 0, res.stdout + res.stderr
    man = json.loads((out / "manifest.json").read_text())
    H, Hkv, D, hid, T = man["heads"], man["kvHeads"], man["headDim"], man["hidden"], man["tokens"]

    def w(name, n, nb):
        return (np.fromfile(out / f"w{name}.quant", np.uint8).reshape(n, nb, 16),
                np.fromfile(out / f"w{name}.scales", np.float32).reshape(n, nb),
                np.fromfile(out / f"w{name}.zp", np.uint8))

    wq, wk, wv = w("q", H * D, hid // 32), w("k", Hkv * D, hid // 32), w("v", Hkv * D, hid // 32)
    wo = w("o", hid, H * D // 32)
    hnorm = np.fromfile(out / "hnorm.f32", np.float32).reshape(T, hid)
    hin = np.fromfile(out / "hin.f32", np.float32).reshape(T, hid)
    attn = np.fromfile(out / "attn.f32", np.float32).reshape(T, H, D)
    hout = np.fromfile(out / "hout.f32", np.float32).reshape(T, hid)
    k_rows, v_rows, worst = [], [], 0.0
    # Both modes against the oracle on the same fp32 queries (the prefill
    # keeps the scaled fp32 query as fp16 high and low parts).
    for t in range(T):
        q = oracle.q4_gemv_f32(hnorm[t], *wq).reshape(H, D)
        for rows, wm in ((k_rows, wk), (v_rows, wv)):
            rows.append(oracle.f16_to_f32(oracle.f32_to_f16(oracle.q4_gemv_f32(hnorm[t], *wm)))
                        .reshape(Hkv, D))
        want = oracle.sparse_attn_f32(q, np.stack(k_rows), np.stack(v_rows))
        worst = max(worst, max_abs(attn[t], want))
        o64, bound = gemv_f64(attn[t].reshape(-1), *wo)
        h64 = hin[t].astype(np.float64) + o64
        slack = 1e-6 * bound + np.abs(h64) * 2.0 ** -23
        assert np.all(np.abs(hout[t] - h64) <= slack), t
    assert worst < 2e-3, worst


def test_node_host_greedy_head(tmp_path):
    """js/check_head.js: GreedyHead (lm_head GEMV + greedy pick,
    engine/runtime.js:397-399) on a 32768-token 4-bit lm_head. The logits are
    within 1e-6 of sum |w a| of the float64 projection, and the token read
    back equals the oracle's pick on those logits, bit-exact."""
    out = tmp_path / "head"
    print("node check_head vocab=32768 hidden=3136 steps=4", flush=True)
    res = subprocess.run(["node", str(JS / "check_head.js"), str(out), "32768", "3136", "4"],
                         capture_output=True, text=True, timeout=180)
    assert res.returncode == 0, res.stdout + res.stderr
    man = json.loads((out / "manifest.json").read_text())
    V, hid, T = man["vocab"], man["hidden"], man["steps"]
    nb = hid // 32
    quant = np.fromfile(out / "quant.u8", np.uint8).reshape(V, nb, 16)
    scales = np.fromfile(out / "scales.f32", np.float32).reshape(V, nb)
    zp = np.fromfile(out / "zp.u8", np.uint8)
    h = np.fromfile(out / "h.f32", np.float32).reshape(T, hid)
    logits = np.fromfile(out / "logits.f32", np.float32).reshape(T, V)
    tokens = np.fromfile(out / "tokens.u32", np.uint32)
    for t in range(T):
        y64, bound = gemv_f64(h[t], quant, scales, zp)
        assert np.all(np.abs(logits[t] - y64) <= 1e-6 * bound), t
        assert tokens[t] == oracle.argmax_ref(logits[t]), t


def test_node_host_bad_position_reported_at_readback():
    """The token loop does not wait for the device (engine/runtime.js:447-469):
    endStep never synchronises, so an out-of-range device position written
    in token 7 of 20 is reported by the readback after the loop (then
    cleared), not by the step; a clean run reads back without error."""
    print("node check_status tokens=20 bad=7", flush=True)
    res = subprocess.run(["node", str(JS / "check_status.js"), "20", "7"], capture_output=True,
                         text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    r = json.loads(res.stdout.strip().splitlines()[-1])
    bad, clean = r["corrupted"], r["clean"]
    assert bad["stepError"] is None, bad
    assert bad["readbackError"] and "position" in bad["readbackError"], bad
    assert bad["secondReadback"] == "ok", bad
    assert clean == {"stepError": None, "readbackError": None, "secondReadback": "ok"}, clean


def test_node_addon_rejects_copies_past_a_buffer():
    """A wrongly sized typed array must not write past a device
    buffer; the addon refuses copies that do not fit inside one allocation,
    and AttentionSlice checks the q/k/v/attnO lengths."""
    script = r"""
    const { AttentionSlice, addon } = require('./attention_layer');
    const out = {};
    const p = addon.malloc(64);
    const tryIt = (name, f) => { try { f(); out[name] = 'ok'; } catch (e) { out[name] = String(e.message); } };
    tryIt('fits', () => addon.upload(p, new Float32Array(16)));
    tryIt('upload', () => addon.upload(p, new Float32Array(17)));
    tryIt('download', () => addon.download(new Float32Array(17), p));
    tryIt('offset', () => addon.upload(p + 8n, new Float32Array(15)));
    tryIt('setI32', () => addon.setI32(p + 64n, 1));
    tryIt('zero', () => addon.zero(p, 65));
    addon.free(p);
    const s = new AttentionSlice({ heads: 8, kvHeads: 2, headDim: 128, maxSeq: 8, layers: [0] });
    tryIt('setQKV', () => s.setQKV(new Float32Array(8 * 128), new Float32Array(2 * 128 + 1),
                                   new Float32Array(2 * 128)));
    tryIt('readAttnO', () => s.readAttnO(new Float32Array(10)));
    s.destroy();
    console.log(JSON.stringify(out));
    """
    print("node addon range checks", flush=True)
    res = subprocess.run(["node", "-e", script], capture_output=True, text=True, timeout=60, cwd=JS)
    assert res.returncode == 0, res.stdout + res.stderr
    r = json.loads(res.stdout.strip().splitlines()[-1])
    assert r["fits"] == "ok", r
    for k in ("upload", "download", "offset", "setI32", "zero"):
        assert "do not fit" in r[k], (k, r)
    assert "setQKV k" in r["setQKV"] and "readAttnO" in r["readAttnO"], r
