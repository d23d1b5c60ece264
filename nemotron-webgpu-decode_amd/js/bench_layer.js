'use strict';
// Times the attention layers of a decode step driven from Node the way
// DecodeEngine drives them (engine/runtime.js:386-393 per attention layer,
// :447-469 per token): per token, beginStep (guard + device position
// write), then for each of the model's 4 attention layers qkvAppend + decode
// + q4Gemv(accumulate) from the normalised hidden state, then endStep; no
// token waits for the device (as the reference's submitStep,
// runtime.js:447-469); the device status is checked, which synchronises, once
// after the timed tokens. Nano-4B shapes (40 query heads, 8 KV
// heads, hidden 3136), seeded random 4-bit weights per layer, caches filled
// with `past` tokens. Prints one JSON line.
//
// usage: node bench_layer.js [past tokens steps warmup]
const { AttentionSlice, NANO4B, ATTN_LAYERS, addon } = require('./attention_layer');

function lcg(seed) {
  let s = seed >>> 0;
  return () => {
    s = (Math.imul(s, 1664525) + 1013904223) >>> 0;
    return s / 4294967296;
  };
}

function randomQ4(rand, n, nBlocks) {
  const quant = new Uint8Array(n * nBlocks * 16);
  for (let i = 0; i < quant.length; i++) quant[i] = (rand() * 256) | 0;
  const scales = new Float32Array(n * nBlocks);
  for (let i = 0; i < scales.length; i++) scales[i] = 0.005 + 0.01 * rand();
  const zp = new Uint8Array(Math.ceil((n * nBlocks) / 2));
  for (let i = 0; i < zp.length; i++) zp[i] = (rand() * 256) | 0;
  return { quant, scales, zp, n, nBlocks };
}

function main() {
  const past = Number(process.argv[2] || 4096);
  const steps = Number(process.argv[3] || 64);
  const warmup = Number(process.argv[4] || 8);
  const { hidden, heads, kvHeads, headDim } = NANO4B;
  const slice = new AttentionSlice({ heads, kvHeads, headDim, maxSeq: past + warmup + steps,
                                     layers: ATTN_LAYERS });
  const rand = lcg(20261201);
  const qd = heads * headDim, kvd = kvHeads * headDim;
  for (const i of ATTN_LAYERS) {
    slice.setLayerWeights(i, {
      q: slice.uploadQ4(randomQ4(rand, qd, hidden / 32)),
      k: slice.uploadQ4(randomQ4(rand, kvd, hidden / 32)),
      v: slice.uploadQ4(randomQ4(rand, kvd, hidden / 32)),
      o: slice.uploadQ4(randomQ4(rand, hidden, qd / 32)),
    });
  }
  // Caches of `past` random fp16 tokens (N(0,1)-like values from a uniform sum).
  const cacheHalves = Number(slice.cacheBytes) / 2;
  const rows = new Uint16Array(cacheHalves);
  const f16 = (x) => {  // round-to-nearest fp16 bits of |x| < 8 (normal range only)
    const f = new Float32Array([x]);
    const u = new Uint32Array(f.buffer)[0];
    const sign = (u >>> 16) & 0x8000, e = ((u >>> 23) & 0xff) - 127 + 15, m = u & 0x7fffff;
    if (e <= 0) return sign;
    let h = sign | (e << 10) | (m >>> 13);
    if ((m & 0x1fff) > 0x1000 || ((m & 0x1fff) === 0x1000 && (h & 1))) h += 1;
    return h;
  };
  for (let i = 0; i < cacheHalves; i++) rows[i] = f16(rand() + rand() + rand() - 1.5);
  for (const i of ATTN_LAYERS) {
    addon.upload(slice.kCache.get(i), rows);
    addon.upload(slice.vCache.get(i), rows);
  }
  slice.seq = past;
  const hNorm = addon.malloc(hidden * 4), h = addon.malloc(hidden * 4);
  const x = new Float32Array(hidden);
  for (let i = 0; i < hidden; i++) x[i] = 2 * rand() - 1;
  addon.upload(hNorm, x);
  addon.upload(h, x);

  // eager: every call from JavaScript; graph: one captured token replayed
  const eager = () => {
    for (const i of ATTN_LAYERS) slice.encodeLayerFromHidden(i, hNorm, h);
  };
  const graph = slice.captureToken(hNorm, h);
  const replay = () => slice.runToken(graph);
  const time = (body) => {
    const start = slice.seq;
    const run = () => {
      slice.beginStep();
      body();
      slice.endStep();
    };
    for (let t = 0; t < warmup; t++) run();
    slice.checkStatus();
    const t0 = process.hrtime.bigint();
    for (let t = 0; t < steps; t++) run();
    slice.checkStatus();  // the device has finished every timed token
    const us = Number(process.hrtime.bigint() - t0) / 1e3 / steps;
    slice.seq = start;  // both modes attend over the same lengths
    return us;
  };
  const usEager = time(eager), usGraph = time(replay);
  const n = ATTN_LAYERS.length;
  console.log(JSON.stringify({
    workload: 'node-layer', past, steps, warmup, layers: n,
    us_per_token_eager: Number(usEager.toFixed(2)),
    us_per_token_graph: Number(usGraph.toFixed(2)),
    us_per_layer_step_eager: Number((usEager / n).toFixed(2)),
    us_per_layer_step_graph: Number((usGraph / n).toFixed(2)),
  }));
  addon.free(hNorm);
  addon.free(h);
  slice.destroy();
}

main();
