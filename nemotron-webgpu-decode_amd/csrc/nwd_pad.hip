// nwd_pad.hip — decode at head_dim 128 with groups of 3, 6 or 7 query heads
// on the kernels built for groups of 4 and 8 (nwd_decode.hip).
//
// The reference kernel maps query head h to KV head h / (H / Hkv) for any
// group (kernels/sparse_attn.wgsl:38-39). nwd_decode.hip serves a whole group
// per workgroup, reading each K/V row once, for groups 1, 2, 4, 5 and 8. A
// group of 3 (6, 7) is run as a group of 4 (8): the query rows are copied
// into a padded layout with zero rows after each group's real heads, the
// decode runs on it, and the real heads' rows are copied out. Decode is bound
// by the K/V stream, which the padding leaves unchanged; the zero rows'
// outputs are discarded. The copies are two small launches (B x Hkv x 8 x 128
// values each), so the host takes this path from a key bound up.
#include "nwd_common.h"
#include "nwd_internal.h"

namespace nwd {

constexpr int kPadThreads = 256;

// qp[b][hk][g][d] = g < G ? q[b][hk * G + g][d] : 0, Gf rows per KV head.
template <typename T>
__global__ __launch_bounds__(kPadThreads) void pad_rows_kernel(const T* __restrict__ q,
                                                               T* __restrict__ qp, int64_t n,
                                                               int G, int Gf) {
  const int64_t i = (int64_t)blockIdx.x * kPadThreads + threadIdx.x;
  if (i >= n) return;
  const int d = (int)(i % kHeadDim);
  const int64_t r = i / kHeadDim;  // padded row (b, hk, g)
  const int g = (int)(r % Gf);
  const int64_t bh = r / Gf;       // b * Hkv + hk
  qp[i] = g < G ? q[(bh * G + g) * kHeadDim + d] : T(0);
}

// out[b][hk * G + g][d] = op[b][hk][g][d] for g < G.
template <typename T>
__global__ __launch_bounds__(kPadThreads) void unpad_rows_kernel(const T* __restrict__ op,
                                                                 T* __restrict__ out, int64_t n,
                                                                 int G, int Gf) {
  const int64_t i = (int64_t)blockIdx.x * kPadThreads + threadIdx.x;
  if (i >= n) return;
  const int d = (int)(i % kHeadDim);
  const int64_t r = i / kHeadDim;  // real row (b, h)
  const int g = (int)(r % G);
  const int64_t bh = r / G;
  out[i] = op[(bh * Gf + g) * kHeadDim + d];
}

int padded_group(int group) {
  if (group == 3) return 4;
  if (group == 6 || group == 7) return 8;
  return 0;
}

Shape padded_shape(const Shape& s) {
  Shape p = s;
  p.group = padded_group(s.group);
  p.n_heads = s.n_kv * p.group;
  p.general = 0;
  return p;
}

template <typename TQ, typename TO>
static hipError_t run_padded(const Shape& s, const DecodeCall& c, const Workspace& ws, void* q_pad,
                             void* out_pad, hipStream_t stream) {
  const Shape p = padded_shape(s);
  const int64_t n_pad = (int64_t)c.batch * p.n_heads * kHeadDim;
  const int64_t n_real = (int64_t)c.batch * s.n_heads * kHeadDim;
  pad_rows_kernel<TQ><<<(unsigned)((n_pad + kPadThreads - 1) / kPadThreads), kPadThreads, 0, stream>>>(
      static_cast<const TQ*>(c.q), static_cast<TQ*>(q_pad), n_pad, s.group, p.group);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  DecodeCall cp = c;
  cp.q = q_pad;
  cp.out = out_pad;
  e = launch_decode(p, cp, ws, stream);
  if (e != hipSuccess) return e;
  unpad_rows_kernel<TO><<<(unsigned)((n_real + kPadThreads - 1) / kPadThreads), kPadThreads, 0, stream>>>(
      static_cast<const TO*>(out_pad), static_cast<TO*>(c.out), n_real, s.group, p.group);
  return hipGetLastError();
}

hipError_t launch_padded_decode(const Shape& s, const DecodeCall& c, const Workspace& ws,
                                void* q_pad, void* out_pad, hipStream_t stream) {
  if (padded_group(s.group) == 0 || s.head_dim != kHeadDim || !q_pad || !out_pad)
    return hipErrorInvalidValue;
  if (s.q16)
    return s.o16 ? run_padded<f16, f16>(s, c, ws, q_pad, out_pad, stream)
                 : run_padded<f16, float>(s, c, ws, q_pad, out_pad, stream);
  return s.o16 ? run_padded<float, f16>(s, c, ws, q_pad, out_pad, stream)
               : run_padded<float, float>(s, c, ws, q_pad, out_pad, stream);
}

}  // namespace nwd
