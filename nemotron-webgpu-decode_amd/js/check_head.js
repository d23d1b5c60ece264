'use strict';
// Drives GreedyHead (lm_head + greedy pick, engine/runtime.js:397-399) with a
// seeded random 4-bit lm_head in the reference's MatMulNBits format, for a
// few final-norm states; writes the weights, inputs, logits and picked tokens
// to <outDir> for the Python parity test, which checks them against the
// oracle.
//
// usage: node check_head.js <outDir> [vocab hidden steps]
const fs = require('fs');
const path = require('path');
const { AttentionSlice, GreedyHead, addon } = require('./attention_layer');

function lcg(seed) {
  let s = seed >>> 0;
  return () => {
    s = (Math.imul(s, 1664525) + 1013904223) >>> 0;
    return s / 4294967296;
  };
}

function main() {
  const outDir = process.argv[2];
  const vocab = Number(process.argv[3] || 32768);
  const hidden = Number(process.argv[4] || 3136);
  const steps = Number(process.argv[5] || 4);
  fs.mkdirSync(outDir, { recursive: true });
  const rand = lcg(20261202);
  const nBlocks = hidden / 32;
  const quant = new Uint8Array(vocab * nBlocks * 16);
  for (let i = 0; i < quant.length; i++) quant[i] = Math.floor(rand() * 256);
  const scales = new Float32Array(vocab * nBlocks);
  for (let i = 0; i < scales.length; i++) scales[i] = 0.005 + 0.01 * rand();
  const zp = new Uint8Array(Math.ceil((vocab * nBlocks) / 2));
  for (let i = 0; i < zp.length; i++) zp[i] = Math.floor(rand() * 256);

  const slice = new AttentionSlice({ maxSeq: 16, layers: [12] });
  const head = new GreedyHead(slice, slice.uploadQ4({ quant, scales, zp, n: vocab, nBlocks }));
  const hDev = addon.malloc(hidden * 4);
  const hs = [];
  const logits = [];
  const tokens = new Uint32Array(steps);
  for (let t = 0; t < steps; t++) {
    const h = new Float32Array(hidden);
    for (let i = 0; i < hidden; i++) h[i] = 2 * rand() - 1;
    addon.upload(hDev, h);
    head.encode(hDev, true);
    tokens[t] = head.readToken();
    hs.push(h);
    logits.push(head.readLogits());
  }
  const bytes = (a) => Buffer.from(a.buffer, a.byteOffset, a.byteLength);
  fs.writeFileSync(path.join(outDir, 'quant.u8'), bytes(quant));
  fs.writeFileSync(path.join(outDir, 'scales.f32'), bytes(scales));
  fs.writeFileSync(path.join(outDir, 'zp.u8'), bytes(zp));
  fs.writeFileSync(path.join(outDir, 'h.f32'), Buffer.concat(hs.map(bytes)));
  fs.writeFileSync(path.join(outDir, 'logits.f32'), Buffer.concat(logits.map(bytes)));
  fs.writeFileSync(path.join(outDir, 'tokens.u32'), bytes(tokens));
  fs.writeFileSync(path.join(outDir, 'manifest.json'), JSON.stringify({ vocab, hidden, steps }));
  addon.free(hDev);
  head.destroy();
  slice.destroy();
}

main();
