'use strict';
// The token loop does not wait for the device (engine/runtime.js:447-469),
// so a bad device position is reported at the next readback, not at the
// step: this drives AttentionSlice for `tokens` tokens, overwrites the device
// position with an out-of-range value in token `bad` (after beginStep wrote
// the valid one), and records where the error surfaces. A second run without
// the corruption must read back cleanly. Prints one JSON line.
//
// usage: node check_status.js [tokens bad]
const { AttentionSlice, addon } = require('./attention_layer');

function run(tokens, bad) {
  const slice = new AttentionSlice({ heads: 8, kvHeads: 2, headDim: 128, maxSeq: 64, layers: [0, 1] });
  const q = new Float32Array(8 * 128).fill(0.01);
  const kv = new Float32Array(2 * 128).fill(0.5);
  const res = { stepError: null, readbackError: null, secondReadback: 'ok' };
  try {
    for (let t = 0; t < tokens; t++) {
      slice.beginStep();
      if (t === bad) addon.setI32(slice.pos, slice.maxSeq + 5);
      for (const layer of slice.layers) {
        slice.setQKV(q, kv, kv);
        slice.encodeLayer(layer);
      }
      slice.endStep();
    }
  } catch (e) {
    res.stepError = String(e.message);
  }
  try {
    slice.readAttnO();
  } catch (e) {
    res.readbackError = String(e.message);
  }
  try {
    slice.readAttnO();  // the flag was cleared by the first check
  } catch (e) {
    res.secondReadback = String(e.message);
  }
  slice.destroy();
  return res;
}

const tokens = Number(process.argv[2] || 20);
const bad = Number(process.argv[3] || 7);
console.log(JSON.stringify({ tokens, bad, corrupted: run(tokens, bad), clean: run(tokens, -1) }));
