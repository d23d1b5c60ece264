'use strict';
// Drives AttentionSlice the way DecodeEngine.generate drives the attention
// layers (engine/runtime.js:635-648): token after token, every attention
// layer, the position advancing once per token. Inputs come from a seeded
// LCG; inputs and attention outputs are written to <outDir> for the Python
// parity test, which checks them against the oracle.
//
// usage: node check_attention.js <outDir> [heads kvHeads tokens maxSeq [chunks [headDim]]]
// chunks (e.g. "37,64"): the first tokens go through chunked prefill in
// chunks of these sizes, the rest one decode step each; the inputs are the
// same either way. headDim defaults to 128 (engine/config.js:12).
const fs = require('fs');
const path = require('path');
const { AttentionSlice } = require('./attention_layer');

function lcg(seed) {
  let s = seed >>> 0;
  return () => {
    s = (Math.imul(s, 1664525) + 1013904223) >>> 0;
    return s / 4294967296;
  };
}

function normals(rand, n) {
  const out = new Float32Array(n);
  for (let i = 0; i < n; i += 2) {
    const u = Math.max(rand(), 1e-12);
    const r = Math.sqrt(-2 * Math.log(u));
    const t = 2 * Math.PI * rand();
    out[i] = r * Math.cos(t);
    if (i + 1 < n) out[i + 1] = r * Math.sin(t);
  }
  return out;
}

function main() {
  const outDir = process.argv[2];
  const heads = Number(process.argv[3] || 40);
  const kvHeads = Number(process.argv[4] || 8);
  const tokens = Number(process.argv[5] || 153);
  const maxSeq = Number(process.argv[6] || 256);
  const headDim = Number(process.argv[8] || 128);
  fs.mkdirSync(outDir, { recursive: true });
  const slice = new AttentionSlice({ heads, kvHeads, headDim, maxSeq });
  const chunks = (process.argv[7] || '').split(',').filter((x) => x).map(Number);
  const rand = lcg(20260512);
  const nL = slice.layers.length;
  // inputs of token t, layer li at t * nL + li, drawn in that order
  const qAll = [];
  const kAll = [];
  const vAll = [];
  for (let t = 0; t < tokens; t++) {
    for (let li = 0; li < nL; li++) {
      qAll.push(normals(rand, heads * headDim));
      kAll.push(normals(rand, kvHeads * headDim));
      vAll.push(normals(rand, kvHeads * headDim));
    }
  }
  const oAll = new Array(tokens * nL);
  const gather = (arrs, t0, n, li, w) => {
    const out = new Float32Array(n * w);
    for (let j = 0; j < n; j++) out.set(arrs[(t0 + j) * nL + li], j * w);
    return out;
  };
  let t = 0;
  for (const n of chunks) {
    slice.beginPrefill(n);
    slice.layers.forEach((layer, li) => {
      slice.prefillLayer(layer, gather(qAll, t, n, li, heads * headDim),
                         gather(kAll, t, n, li, kvHeads * headDim),
                         gather(vAll, t, n, li, kvHeads * headDim));
      const o = slice.readPrefillO();
      for (let j = 0; j < n; j++)
        oAll[(t + j) * nL + li] = o.slice(j * heads * headDim, (j + 1) * heads * headDim);
    });
    slice.endPrefill();
    t += n;
  }
  for (; t < tokens; t++) {
    slice.beginStep();
    slice.layers.forEach((layer, li) => {
      const at = t * nL + li;
      slice.setQKV(qAll[at], kAll[at], vAll[at]);
      if ((t + layer) % 2 === 0) slice.encodeLayer(layer);
      else slice.encodeLayerTwoCalls(layer);
      oAll[at] = slice.readAttnO();
    });
    slice.endStep();
  }
  // the maxSeq guard (runtime.js:448) must throw, not write past the cache
  let guard = 'no-throw';
  let prefillGuard = 'no-throw';
  // a chunk call outside beginPrefill .. endPrefill must throw, not append
  let chunkGuard = 'no-throw';
  try {
    slice.prefillLayer(slice.layers[0], new Float32Array(0), new Float32Array(0), new Float32Array(0));
  } catch (e) {
    chunkGuard = String(e.message);
  }
  if (tokens === maxSeq) {
    try {
      slice.beginStep();
    } catch (e) {
      guard = String(e.message);
    }
    try {
      slice.beginPrefill(1);
    } catch (e) {
      prefillGuard = String(e.message);
    }
  }
  const cat = (arrs) => Buffer.concat(arrs.map((a) => Buffer.from(a.buffer, a.byteOffset, a.byteLength)));
  fs.writeFileSync(path.join(outDir, 'q.f32'), cat(qAll));
  fs.writeFileSync(path.join(outDir, 'k.f32'), cat(kAll));
  fs.writeFileSync(path.join(outDir, 'v.f32'), cat(vAll));
  fs.writeFileSync(path.join(outDir, 'o.f32'), cat(oAll));
  fs.writeFileSync(path.join(outDir, 'manifest.json'), JSON.stringify({
    heads, kvHeads, headDim, tokens, maxSeq, layers: slice.layers, guard, prefillGuard, chunkGuard, chunks,
  }));
  slice.destroy();
  console.log(`check_attention: ${tokens} tokens x ${slice.layers.length} layers written to ${outDir}`);
}

main();
