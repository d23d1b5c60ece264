// nwd_argmax.h — the reference's greedy pick as one 64-bit maximum.
//
// kernels/argmax_partial.wgsl + argmax_merge.wgsl (engine/runtime.js:209,
// 398-399) split n logits into 256 slices of n_slice = ceil(n / 256); a
// thread walks its slice with stride 256 keeping its first strictly greater
// value (from -3.402823466e38), and two 256-wide trees (threads, then
// slices) keep the left position on ties. Two tied entries of such a tree
// meet at the lowest bit where their positions differ, and the one with a 0
// there wins; so the reference returns the largest value strictly above
// -3.402823466e38, ties going to the smallest
//   key = (bitrev8(slice) * 256 + bitrev8(thread)) * steps + step,
// steps = ceil(n_slice / 256), or index 0 if no value qualifies.
//
// That order is a total order on (value, key), so any reduction tree gives
// the reference's index. Each candidate is encoded as
//   ordered(value) << 32 | (0xFFFFFFFF - key)
// (ordered: the IEEE bits mapped to an unsigned order), and the pick is the
// largest encoding; non-candidates encode as 0.
#pragma once

#include "nwd_common.h"

namespace nwd {

struct ArgmaxShape {
  uint32_t n_slice;  // ceil(n / 256)
  uint32_t steps;    // ceil(n_slice / 256)
};

__host__ __device__ inline ArgmaxShape argmax_shape(uint32_t n) {
  const uint32_t n_slice = (n + 255) / 256;
  return ArgmaxShape{n_slice, (n_slice + 255) / 256};
}

__device__ inline uint32_t bitrev8(uint32_t v) { return __builtin_bitreverse32(v) >> 24; }

__device__ inline uint32_t argmax_key(uint32_t i, ArgmaxShape s) {
  const uint32_t slice = i / s.n_slice, r = i - slice * s.n_slice;
  return (bitrev8(slice) * 256 + bitrev8(r & 255)) * s.steps + (r >> 8);
}

__device__ inline uint32_t argmax_index(uint32_t key, ArgmaxShape s) {
  const uint32_t step = key % s.steps, q = key / s.steps;
  return bitrev8(q >> 8) * s.n_slice + step * 256 + bitrev8(q & 255);
}

__device__ inline unsigned long long argmax_enc(float v, uint32_t i, ArgmaxShape s) {
  // Candidates are strictly above -3.402823466e38; comparisons with NaN fail.
  if (!(v > -3.402823466e38f)) return 0ull;
  uint32_t b = __float_as_uint(v);
  if (b == 0x80000000u) b = 0u;  // -0 ties with +0 in the reference's comparisons
  const uint32_t ordered = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)ordered << 32) | (0xFFFFFFFFu - argmax_key(i, s));
}

__device__ inline uint32_t argmax_decode(unsigned long long enc, ArgmaxShape s) {
  if (enc == 0ull) return 0u;
  return argmax_index(0xFFFFFFFFu - (uint32_t)enc, s);
}

// Largest encoding over the 64 lanes of a wave, in every lane.
__device__ inline unsigned long long wave_max_u64(unsigned long long e) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const unsigned long long o = __shfl_xor(e, m, 64);
    e = o > e ? o : e;
  }
  return e;
}

}  // namespace nwd
