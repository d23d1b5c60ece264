'use strict';
// Attention slice of the reference DecodeEngine (engine/runtime.js) on the
// MI355X library, through the N-API addon (addon/nwd_napi.cc).
//
// The reference, per attention layer and token:
//   _alloc    f32 q/k/v/attnO buffers and per-layer K/V caches
//             [maxSeq][kvHeads][headDim] (engine/runtime.js:120-123,170-173)
//   _bind     kvK = [k, kCache, uKv], kvV = [v, vCache, uKv],
//             attn = [q, kCache, vCache, attnO, uAttn]   (:331-333)
//   _ops      kvK, kvV, attn dispatched in one pass        (:389-391)
//   submitStep guard seq < maxSeq (:448); uKv.seq = seq, uAttn.seq = seq+1
//             (:451-452); submit; seq++ (:467) — it never waits for the
//             device; generate enqueues every token and reads the outputs
//             once at the end (:641-647, readOutputs :490-511)
//   reset     zero-fill the caches (:615-633)
// The token loop here does not wait for the device either: beginStep writes
// the position with a stream-ordered write and endStep only advances seq.
// A kernel that sees an out-of-range device position sets a sticky status
// word; it is checked (one synchronisation) when outputs are read back
// (readAttnO, GreedyHead.readToken / readLogits), by checkStatus(), or every
// `statusEvery` tokens when that option is set.
// Here the three dispatches are one appendDecode call, the caches are fp16
// (head-major, see include/nwd_attn.h), and the position is one device int32
// that the host writes before each step, as the reference writes its
// uniforms. q/k/v/attnO stay f32, the reference's activation type, so the
// q/k/v GEMVs and the o_proj GEMV bind unchanged.
//
// A prompt can also go through the attention layers as chunks (beginPrefill,
// prefillLayer, endPrefill): the reference runs each prompt token through the
// whole decode step (generate, runtime.js:640-643); here a chunk's rows are
// appended with one kvAppend and attended with one causal prefill call per
// layer, with the same result for every token.
//
// With the layer's 4-bit weights registered (setLayerWeights), the whole
// attention layer from the normalised hidden state runs on the library too:
// the reference's L-q, L-k, L-v, L-kvK, L-kvV, L-attn, L-o, L-add
// (runtime.js:386-393) become qkvAppend, decode and q4Gemv(accumulate).
const path = require('path');

const ADDON = path.join(__dirname, '..', 'lib', 'nwd_napi.node');
// eslint-disable-next-line import/no-dynamic-require
const addon = require(ADDON);

// Nemotron-3-Nano-4B attention shapes (engine/config.js:10-12,24,31).
const NANO4B = { hidden: 3136, heads: 40, kvHeads: 8, headDim: 128, maxSeq: 256 };
const Q4_PLAIN = 0;       // nwd_q4_gemv epilogue: y = W.a
const Q4_ACCUMULATE = 2;  // nwd_q4_gemv epilogue: y = y + W.a (o_proj + residual add)
const ATTN_LAYERS = [12, 17, 24, 32];

function expectF32(a, n, what) {
  if (!(a instanceof Float32Array) || a.length !== n)
    throw new Error(`${what}: expected a Float32Array of ${n} values, got ` +
                    `${a && a.constructor ? a.constructor.name : typeof a} of ${a ? a.length : 0}`);
}

class AttentionSlice {
  constructor({ heads = NANO4B.heads, kvHeads = NANO4B.kvHeads, headDim = NANO4B.headDim,
                maxSeq = NANO4B.maxSeq, layers = ATTN_LAYERS, statusEvery = 0 } = {}) {
    this.heads = heads;
    this.statusEvery = statusEvery;  // 0: check the device status only at readback
    this.kvHeads = kvHeads;
    this.headDim = headDim;
    this.maxSeq = maxSeq;
    this.layers = layers.slice();
    this.ctx = addon.create({ nHeads: heads, nKvHeads: kvHeads, headDim, maxSeq, maxBatch: 1,
                              qF16: 0, oF16: 0, kvF16: 0 });
    const f32 = (n) => addon.malloc(n * 4);
    this.q = f32(heads * headDim);
    this.k = f32(kvHeads * headDim);
    this.v = f32(kvHeads * headDim);
    this.attnO = f32(heads * headDim);
    this.cacheBytes = addon.cacheBytes(this.ctx);
    this.kCache = new Map();
    this.vCache = new Map();
    for (const i of this.layers) {
      this.kCache.set(i, addon.malloc(this.cacheBytes));
      this.vCache.set(i, addon.malloc(this.cacheBytes));
    }
    this.pos = addon.malloc(4);
    this.chunk = null;         // prefill buffers {n, q, k, v, o}, grown on demand
    this.weights = new Map();  // layer -> {q, k, v, o} nwd_q4_weight descriptors
    this.owned = [];           // device buffers uploadQ4 allocated
    this.graphs = [];          // token graphs captureToken made
    this.seq = 0;
    this.reset();
  }

  // A host projection in the reference's MatMulNBits format
  // (engine/weights.js:99-104: quant Uint8Array [n][nBlocks][16], scales
  // Float32Array [n][nBlocks], zp Uint8Array of packed 4-bit zero points) on
  // the device, as the descriptor qkvAppend / q4Gemv take.
  uploadQ4({ quant, scales, zp, n, nBlocks }) {
    const put = (arr) => {
      const p = addon.malloc(arr.byteLength);
      addon.upload(p, arr);
      this.owned.push(p);
      return p;
    };
    return { quant: put(quant), scales: put(scales), zp: put(zp), n, nBlocks };
  }

  // runtime.js:321-324: the q4 projections of attention layer i.
  setLayerWeights(i, { q, k, v, o }) {
    if (!this.kCache.has(i)) throw new Error(`layer ${i} is not an attention layer`);
    this.weights.set(i, { q, k, v, o });
  }

  // runtime.js:386-393 for attention layer i: hNorm (f32 [hidden], device) ->
  // q / k / v projections with k / v written into the caches, attention, and
  // o_proj added into the residual stream h (f32 [hidden], device).
  // maxLen bounds the keys attended (default: this token's seq + 1).
  encodeLayerFromHidden(i, hNorm, h, maxLen = this.seq + 1) {
    const w = this.weights.get(i);
    if (!w) throw new Error(`layer ${i} has no weights (setLayerWeights)`);
    addon.qkvAppend(this.ctx, hNorm, w.q, w.k, w.v, this.q, this.kCache.get(i), this.vCache.get(i),
                    this.pos, 1);
    addon.decode(this.ctx, this.q, this.kCache.get(i), this.vCache.get(i), this.pos, this.attnO, 1,
                 maxLen);
    addon.q4Gemv(this.ctx, this.attnO, w.o, h, 1, Q4_ACCUMULATE);
  }

  // The reference builds its op list once and submits it every token
  // (engine/runtime.js:385-429). Here one token's attention layers
  // (encodeLayerFromHidden for every layer, in order) are captured once into
  // a HIP graph; runToken replays it between beginStep and endStep with one
  // call. The position is read from the device at replay, and attention is
  // sized for the whole capacity (maxSeq), so one graph serves every token.
  captureToken(hNorm, h) {
    addon.captureBegin();
    let graph = null;
    try {
      for (const i of this.layers) this.encodeLayerFromHidden(i, hNorm, h, this.maxSeq);
    } finally {
      graph = addon.captureEnd();
    }
    this.graphs.push(graph);
    return graph;
  }

  runToken(graph) {
    addon.graphLaunch(graph);
  }

  // runtime.js:615-633 (the KV part of reset)
  reset() {
    this.seq = 0;
    for (const i of this.layers) {
      addon.zero(this.kCache.get(i), this.cacheBytes);
      addon.zero(this.vCache.get(i), this.cacheBytes);
    }
  }

  // runtime.js:448,451-452: guard and position write before the token's ops
  // (stream-ordered, without waiting for the device, as writeBuffer)
  beginStep() {
    if (this.seq >= this.maxSeq) throw new Error(`seq ${this.seq} exceeds maxSeq ${this.maxSeq}`);
    addon.setI32(this.pos, this.seq);
  }

  // What the q/k/v GEMVs of a layer write (runtime.js:386-388, outputs :120-122).
  setQKV(q, k, v) {
    expectF32(q, this.heads * this.headDim, 'setQKV q');
    expectF32(k, this.kvHeads * this.headDim, 'setQKV k');
    expectF32(v, this.kvHeads * this.headDim, 'setQKV v');
    addon.upload(this.q, q);
    addon.upload(this.k, k);
    addon.upload(this.v, v);
  }

  // runtime.js:389-391 for attention layer i: kvK, kvV, attn in one call.
  encodeLayer(i) {
    if (!this.kCache.has(i)) throw new Error(`layer ${i} is not an attention layer`);
    addon.appendDecode(this.ctx, this.q, this.k, this.v, this.kCache.get(i), this.vCache.get(i),
                       this.pos, this.attnO, 1, this.seq + 1);
  }

  // The two-dispatch form kept by the reference (kv_append, then attention):
  // same results, used by the harness to check both entry points.
  encodeLayerTwoCalls(i) {
    addon.kvAppend(this.ctx, this.k, this.v, this.kCache.get(i), this.vCache.get(i), this.pos, 1, 1);
    addon.decode(this.ctx, this.q, this.kCache.get(i), this.vCache.get(i), this.pos, this.attnO, 1,
                 this.seq + 1);
  }

  // Chunked prefill of n prompt tokens (the reference's generate loop,
  // runtime.js:640-643, runs them one decode step each): guard and position
  // as beginStep, for the whole chunk.
  beginPrefill(n) {
    if (!(Number.isInteger(n) && n >= 1)) throw new Error(`beginPrefill: bad token count ${n}`);
    if (this.seq + n > this.maxSeq)
      throw new Error(`seq ${this.seq} + ${n} prompt tokens exceeds maxSeq ${this.maxSeq}`);
    if (!this.chunk || this.chunk.n < n) {
      if (this.chunk) for (const b of ['q', 'k', 'v', 'o']) addon.free(this.chunk[b]);
      const qBytes = n * this.heads * this.headDim * 4;
      const kvBytes = n * this.kvHeads * this.headDim * 4;
      this.chunk = { n, q: addon.malloc(qBytes), k: addon.malloc(kvBytes), v: addon.malloc(kvBytes),
                     o: addon.malloc(qBytes) };
    }
    this.chunkLen = n;
    addon.setI32(this.pos, this.seq);
  }

  // The chunk's q [n][heads][headDim], k and v [n][kvHeads][headDim] (f32)
  // for attention layer i: the rows go to the caches at seq .. seq+n-1
  // (kvAppend), then query j attends keys 0 .. seq+j (prefill).
  prefillLayer(i, q, k, v) {
    if (!this.kCache.has(i)) throw new Error(`layer ${i} is not an attention layer`);
    const n = this.openChunk('prefillLayer');
    expectF32(q, n * this.heads * this.headDim, 'prefillLayer q');
    expectF32(k, n * this.kvHeads * this.headDim, 'prefillLayer k');
    expectF32(v, n * this.kvHeads * this.headDim, 'prefillLayer v');
    addon.upload(this.chunk.q, q);
    addon.upload(this.chunk.k, k);
    addon.upload(this.chunk.v, v);
    addon.kvAppend(this.ctx, this.chunk.k, this.chunk.v, this.kCache.get(i), this.vCache.get(i),
                   this.pos, 1, n);
    addon.prefill(this.ctx, this.chunk.q, this.kCache.get(i), this.vCache.get(i), this.pos,
                  this.chunk.o, 1, n, this.seq + n);
  }

  // runtime.js:386-393 for the chunk's n tokens through attention layer i,
  // from their normalised hidden states hNorm (f32 [n][hidden], device):
  // the q, k and v projections as n-row GEMVs, the k/v rows appended and the
  // chunk attended, and o_proj added into the residual rows h (f32
  // [n][hidden], device).
  prefillLayerFromHidden(i, hNorm, h) {
    const w = this.weights.get(i);
    if (!w) throw new Error(`layer ${i} has no weights (setLayerWeights)`);
    const n = this.openChunk('prefillLayerFromHidden');
    addon.q4Gemv(this.ctx, hNorm, w.q, this.chunk.q, n, Q4_PLAIN);
    addon.q4Gemv(this.ctx, hNorm, w.k, this.chunk.k, n, Q4_PLAIN);
    addon.q4Gemv(this.ctx, hNorm, w.v, this.chunk.v, n, Q4_PLAIN);
    addon.kvAppend(this.ctx, this.chunk.k, this.chunk.v, this.kCache.get(i), this.vCache.get(i),
                   this.pos, 1, n);
    addon.prefill(this.ctx, this.chunk.q, this.kCache.get(i), this.vCache.get(i), this.pos,
                  this.chunk.o, 1, n, this.seq + n);
    addon.q4Gemv(this.ctx, this.chunk.o, w.o, h, n, Q4_ACCUMULATE);
  }

  // The last prefill's attention output, [n][heads][headDim] f32.
  readPrefillO(out) {
    const n = this.openChunk('readPrefillO') * this.heads * this.headDim;
    if (out === undefined) out = new Float32Array(n);
    expectF32(out, n, 'readPrefillO');
    this.checkStatus();
    addon.download(out, this.chunk.o);
    return out;
  }

  endPrefill() {
    this.seq += this.openChunk('endPrefill');
    this.chunkLen = 0;
  }

  // The token count of the chunk between beginPrefill and endPrefill.
  openChunk(who) {
    if (!this.chunkLen) throw new Error(`${who}: no prompt chunk open (beginPrefill)`);
    return this.chunkLen;
  }

  // runtime.js:467: seq++ without waiting for the device.
  endStep() {
    this.seq += 1;
    if (this.statusEvery > 0 && this.seq % this.statusEvery === 0) this.checkStatus();
  }

  // Waits for the work enqueued so far and throws if a kernel saw an
  // out-of-range device position since the last check (the flag is then
  // cleared). The reference's host guard (runtime.js:448) is beginStep's.
  checkStatus() {
    addon.deviceStatus(this.ctx);
  }

  readAttnO(out = new Float32Array(this.heads * this.headDim)) {
    expectF32(out, this.heads * this.headDim, 'readAttnO');
    this.checkStatus();
    addon.download(out, this.attnO);
    return out;
  }

  destroy() {
    for (const g of this.graphs) addon.graphDestroy(g);
    if (this.chunk) for (const b of ['q', 'k', 'v', 'o']) addon.free(this.chunk[b]);
    for (const p of [this.q, this.k, this.v, this.attnO, this.pos, ...this.owned]) addon.free(p);
    for (const i of this.layers) {
      addon.free(this.kCache.get(i));
      addon.free(this.vCache.get(i));
    }
    addon.destroy(this.ctx);
    this.ctx = null;
  }
}

// The end of a decode step (engine/runtime.js:397-399): lm-head GEMV, then
// argmax_partial and argmax_merge, leaving the token id on the device (the
// reference's tokenOut, :125-128) for the next step's embedding. Here the
// lm_head projection and the partial pick are one launch and the merge a
// second; the index has the reference's exact tie order.
class GreedyHead {
  constructor(slice, weight) {
    this.ctx = slice.ctx;  // shares the attention slice's context (stream order)
    this.w = weight;       // nwd_q4_weight descriptor of lm_head (slice.uploadQ4)
    this.tokenOut = addon.malloc(4);
    this.logits = null;
  }

  // hNorm: the final norm's output, f32 [hidden] on the device (runtime.js:396).
  encode(hNorm, keepLogits = false) {
    if (keepLogits && !this.logits) this.logits = addon.malloc(this.w.n * 4);
    addon.lmHeadArgmax(this.ctx, hNorm, this.w, keepLogits ? this.logits : null, this.tokenOut, 1);
  }

  // Readbacks are where the token loop waits for the device: the status of
  // every step enqueued so far is checked first (a bad device position
  // throws here).
  readToken() {
    addon.deviceStatus(this.ctx);
    const t = new Uint32Array(1);
    addon.download(t, this.tokenOut);
    return t[0];
  }

  readLogits(out = new Float32Array(this.w.n)) {
    if (!this.logits) throw new Error('readLogits: encode(hNorm, true) keeps no logits yet');
    expectF32(out, this.w.n, 'readLogits');
    addon.deviceStatus(this.ctx);
    addon.download(out, this.logits);
    return out;
  }

  destroy() {
    addon.free(this.tokenOut);
    if (this.logits) addon.free(this.logits);
  }
}

module.exports = { AttentionSlice, GreedyHead, NANO4B, ATTN_LAYERS, addon };
