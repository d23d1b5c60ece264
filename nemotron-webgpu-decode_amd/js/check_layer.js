'use strict';
// Drives one attention layer of AttentionSlice from the normalised hidden
// state, the way DecodeEngine runs it per token (engine/runtime.js:386-393:
// q/k/v projections, kv_append, attention, o_proj, residual add), with
// seeded random 4-bit weights in the reference's MatMulNBits format. The
// weights, inputs, attention outputs and updated residual stream are written
// to <outDir> for the Python parity test, which checks them against the
// oracle.
//
// usage: node check_layer.js <outDir> [hidden tokens [eager|graph|prefill]]
// prefill: the tokens go through the layer as two prompt chunks
// (AttentionSlice.prefillLayerFromHidden), with the same inputs.
const fs = require('fs');
const path = require('path');
const { AttentionSlice, addon } = require('./attention_layer');

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

// One projection [32 * nBlocks -> n]: quant [n][nBlocks][16] bytes, scales
// [n][nBlocks], packed 4-bit zero points.
function randomQ4(rand, n, nBlocks) {
  const quant = new Uint8Array(n * nBlocks * 16);
  for (let i = 0; i < quant.length; i++) quant[i] = Math.floor(rand() * 256);
  const scales = new Float32Array(n * nBlocks);
  for (let i = 0; i < scales.length; i++) scales[i] = 0.005 + 0.01 * rand();
  const zp = new Uint8Array(Math.ceil((n * nBlocks) / 2));
  for (let i = 0; i < zp.length; i++) zp[i] = Math.floor(rand() * 256);
  return { quant, scales, zp, n, nBlocks };
}

function main() {
  const outDir = process.argv[2];
  const hidden = Number(process.argv[3] || 512);
  const tokens = Number(process.argv[4] || 12);
  const mode = process.argv[5] || 'eager';
  const useGraph = mode === 'graph';  // replay one captured token graph
  const heads = 40;
  const kvHeads = 8;
  const headDim = 128;
  const layer = 12;
  fs.mkdirSync(outDir, { recursive: true });
  const slice = new AttentionSlice({ heads, kvHeads, headDim, maxSeq: 64, layers: [layer] });
  const rand = lcg(20261201);
  const hostW = {
    q: randomQ4(rand, heads * headDim, hidden / 32),
    k: randomQ4(rand, kvHeads * headDim, hidden / 32),
    v: randomQ4(rand, kvHeads * headDim, hidden / 32),
    o: randomQ4(rand, hidden, (heads * headDim) / 32),
  };
  const devW = {};
  for (const [name, w] of Object.entries(hostW)) devW[name] = slice.uploadQ4(w);
  slice.setLayerWeights(layer, devW);

  const outs = { hnorm: [], hin: [], attn: [], hout: [] };
  if (mode === 'prefill') {
    const first = Math.floor(tokens / 2);
    for (const n of [first, tokens - first]) {
      const hNorm = new Float32Array(n * hidden);
      const hIn = new Float32Array(n * hidden);
      for (let j = 0; j < n; j++) {  // the per-token order of the token loop below
        hNorm.set(normals(rand, hidden), j * hidden);
        hIn.set(normals(rand, hidden), j * hidden);
      }
      const hNormDev = addon.malloc(n * hidden * 4);
      const hDev = addon.malloc(n * hidden * 4);
      addon.upload(hNormDev, hNorm);
      addon.upload(hDev, hIn);
      slice.beginPrefill(n);
      slice.prefillLayerFromHidden(layer, hNormDev, hDev);
      const attn = slice.readPrefillO();
      slice.endPrefill();
      const hOut = new Float32Array(n * hidden);
      addon.download(hOut, hDev);
      for (let j = 0; j < n; j++) {
        outs.hnorm.push(hNorm.slice(j * hidden, (j + 1) * hidden));
        outs.hin.push(hIn.slice(j * hidden, (j + 1) * hidden));
        outs.attn.push(attn.slice(j * heads * headDim, (j + 1) * heads * headDim));
        outs.hout.push(hOut.slice(j * hidden, (j + 1) * hidden));
      }
      addon.free(hNormDev);
      addon.free(hDev);
    }
  }
  const hNormDev = addon.malloc(hidden * 4);
  const hDev = addon.malloc(hidden * 4);
  const graph = useGraph ? slice.captureToken(hNormDev, hDev) : null;
  for (let t = mode === 'prefill' ? tokens : 0; t < tokens; t++) {
    const hNorm = normals(rand, hidden);
    const hIn = normals(rand, hidden);
    addon.upload(hNormDev, hNorm);
    addon.upload(hDev, hIn);
    slice.beginStep();
    if (graph) slice.runToken(graph);
    else slice.encodeLayerFromHidden(layer, hNormDev, hDev);
    slice.endStep();
    const hOut = new Float32Array(hidden);
    addon.download(hOut, hDev);
    outs.hnorm.push(hNorm);
    outs.hin.push(hIn);
    outs.attn.push(slice.readAttnO());
    outs.hout.push(hOut);
  }
  const bytes = (a) => Buffer.from(a.buffer, a.byteOffset, a.byteLength);
  const cat = (arrs) => Buffer.concat(arrs.map(bytes));
  for (const [name, arrs] of Object.entries(outs)) {
    fs.writeFileSync(path.join(outDir, `${name}.f32`), cat(arrs));
  }
  for (const [name, w] of Object.entries(hostW)) {
    fs.writeFileSync(path.join(outDir, `w${name}.quant`), bytes(w.quant));
    fs.writeFileSync(path.join(outDir, `w${name}.scales`), bytes(w.scales));
    fs.writeFileSync(path.join(outDir, `w${name}.zp`), bytes(w.zp));
  }
  fs.writeFileSync(path.join(outDir, 'manifest.json'), JSON.stringify({
    heads, kvHeads, headDim, hidden, tokens, graph: useGraph, mode,
  }));
  addon.free(hNormDev);
  addon.free(hDev);
  slice.destroy();
}

main();
