// nwd_pad.hip — decode and prefill with groups the kernels cannot take as
// they are (3, 6, 7 at head sizes other than 128 and 64, and larger groups
// with no built divisor, nwd::kernel_group) on the kernels of the next
// group they take (nwd_decode.hip, nwd_decode_hd.hip, nwd_prefill.hip,
// nwd_prefill_wide.hip), at the head sizes those kernels take (multiples of
// 8 up to 256).
//
// The reference kernel maps query head h to KV head h / (H / Hkv) for any
// group (kernels/sparse_attn.wgsl:38-39). The decode and prefill kernels
// serve a whole group per workgroup, reading each K/V row once, for groups
// 1, 2, 4, 5 and 8 (and at head sizes 128 and 64 every group up to 8). A
// group of 3 (6, 7) is run as a group of 4 (8): the query rows are copied
// into a padded layout with zero rows after each group's real heads, the
// kernels run on it, and the real heads' rows are copied out. Decode is
// bound by the K/V stream, which the padding leaves unchanged; the zero
// rows' outputs are discarded. A prefill chunk goes through in sub-chunks
// sized to the context's padded buffers, each with its first positions
// offset.
#include "nwd_common.h"
#include "nwd_internal.h"

namespace nwd {

constexpr int kPadThreads = 256;

// qp[b][hk][g][d] = g < G ? q[b][hk * G + g][d] : 0, Gf rows per KV head.
template <typename T>
__global__ __launch_bounds__(kPadThreads) void pad_rows_kernel(const T* __restrict__ q,
                                                               T* __restrict__ qp, int64_t n,
                                                               int G, int Gf, int D) {
  const int64_t i = (int64_t)blockIdx.x * kPadThreads + threadIdx.x;
  if (i >= n) return;
  const int d = (int)(i % D);
  const int64_t r = i / D;  // padded row (b, hk, g)
  const int g = (int)(r % Gf);
  const int64_t bh = r / Gf;       // b * Hkv + hk
  qp[i] = g < G ? q[(bh * G + g) * D + d] : T(0);
}

// out[b][hk * G + g][d] = op[b][hk][g][d] for g < G.
template <typename T>
__global__ __launch_bounds__(kPadThreads) void unpad_rows_kernel(const T* __restrict__ op,
                                                                 T* __restrict__ out, int64_t n,
                                                                 int G, int Gf, int D) {
  const int64_t i = (int64_t)blockIdx.x * kPadThreads + threadIdx.x;
  if (i >= n) return;
  const int d = (int)(i % D);
  const int64_t r = i / D;  // real row (b, h)
  const int g = (int)(r % G);
  const int64_t bh = r / G;
  out[i] = op[(bh * Gf + g) * D + d];
}

// Prefill: rows qp[b][i][hk][g][d] = g < G ? q[b][c0 + i][hk * G + g][d] : 0
// for the nc tokens c0 .. c0 + nc - 1 of the chunk; thread i < batch also
// writes the sub-chunk's first position, pos0[b] clamped into the cache as
// the prefill kernels clamp it, plus c0 (an out-of-range chunk is flagged
// once, on its first sub-chunk).
template <typename T>
__global__ __launch_bounds__(kPadThreads) void pad_chunk_kernel(
    const T* __restrict__ q, T* __restrict__ qp, const int32_t* __restrict__ pos0,
    int32_t* __restrict__ pos_sub, int64_t n, int batch, int n_new, int c0, int nc, int n_kv,
    int G, int Gf, int cap, int D, int* __restrict__ status) {
  const int64_t i = (int64_t)blockIdx.x * kPadThreads + threadIdx.x;
  if (i < batch) {
    int P0 = pos0[i];
    if (P0 < 0 || P0 > cap - n_new) {
      if (c0 == 0) atomicOr(status, kStatusBadPos);
      P0 = P0 < 0 ? 0 : cap - n_new;
    }
    pos_sub[i] = P0 + c0;
  }
  if (i >= n) return;
  const int d = (int)(i % D);
  int64_t r = i / D;
  const int g = (int)(r % Gf);
  r /= Gf;
  const int hk = (int)(r % n_kv);
  r /= n_kv;
  const int t = (int)(r % nc);
  const int64_t b = r / nc;
  qp[i] = g < G ? q[(((b * n_new + c0 + t) * n_kv + hk) * G + g) * D + d] : T(0);
}

// out[b][c0 + i][hk * G + g][d] = op[b][i][hk][g][d] for g < G.
template <typename T>
__global__ __launch_bounds__(kPadThreads) void unpad_chunk_kernel(
    const T* __restrict__ op, T* __restrict__ out, int64_t n, int n_new, int c0, int nc, int n_kv,
    int G, int Gf, int D) {
  const int64_t i = (int64_t)blockIdx.x * kPadThreads + threadIdx.x;
  if (i >= n) return;
  const int d = (int)(i % D);
  int64_t r = i / D;  // (b, t, hk, g) of the sub-chunk's real rows
  const int g = (int)(r % G);
  r /= G;
  const int hk = (int)(r % n_kv);
  r /= n_kv;
  const int t = (int)(r % nc);
  const int64_t b = r / nc;
  out[(((b * n_new + c0 + t) * n_kv + hk) * G + g) * D + d] =
      op[(((b * nc + t) * n_kv + hk) * Gf + g) * D + d];
}

bool padded_decode_shape(int head_dim, int group) {
  const int gp = padded_group(head_dim, group);
  return gp > 0 && split_decode_shape(head_dim, gp);
}

Shape padded_shape(const Shape& s) {
  Shape p = s;
  p.group = padded_group(s.head_dim, s.group);
  p.n_heads = s.n_kv * p.group;
  return p;
}

template <typename TQ, typename TO>
static hipError_t run_padded(const Shape& s, const DecodeCall& c, const Workspace& ws, void* q_pad,
                             void* out_pad, hipStream_t stream) {
  const Shape p = padded_shape(s);
  const int D = s.head_dim;
  const int64_t n_pad = (int64_t)c.batch * p.n_heads * D;
  const int64_t n_real = (int64_t)c.batch * s.n_heads * D;
  pad_rows_kernel<TQ><<<(unsigned)((n_pad + kPadThreads - 1) / kPadThreads), kPadThreads, 0, stream>>>(
      static_cast<const TQ*>(c.q), static_cast<TQ*>(q_pad), n_pad, s.group, p.group, D);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  DecodeCall cp = c;
  cp.q = q_pad;
  cp.out = out_pad;
  e = launch_decode(p, cp, ws, stream);
  if (e != hipSuccess) return e;
  unpad_rows_kernel<TO><<<(unsigned)((n_real + kPadThreads - 1) / kPadThreads), kPadThreads, 0, stream>>>(
      static_cast<const TO*>(out_pad), static_cast<TO*>(c.out), n_real, s.group, p.group, D);
  return hipGetLastError();
}

hipError_t launch_padded_decode(const Shape& s, const DecodeCall& c, const Workspace& ws,
                                void* q_pad, void* out_pad, hipStream_t stream) {
  if (!padded_decode_shape(s.head_dim, s.group) || !q_pad || !out_pad) return hipErrorInvalidValue;
  if (s.q16)
    return s.o16 ? run_padded<f16, f16>(s, c, ws, q_pad, out_pad, stream)
                 : run_padded<f16, float>(s, c, ws, q_pad, out_pad, stream);
  return s.o16 ? run_padded<float, f16>(s, c, ws, q_pad, out_pad, stream)
               : run_padded<float, float>(s, c, ws, q_pad, out_pad, stream);
}


template <typename TQ, typename TO>
static hipError_t run_padded_prefill(const Shape& s, const void* q, const void* kc, const void* vc,
                                     const int32_t* pos0, void* out, int batch, int n_new,
                                     int max_len, const Workspace& ws, const PadBuffers& pb,
                                     hipStream_t stream) {
  const Shape p = padded_shape(s);
  const int D = s.head_dim;
  for (int c0 = 0; c0 < n_new; c0 += pb.chunk_tokens) {
    const int nc = min(pb.chunk_tokens, n_new - c0);
    const int64_t n_pad = (int64_t)batch * nc * p.n_heads * D;
    const int64_t n_real = (int64_t)batch * nc * s.n_heads * D;
    const int64_t n_launch = n_pad > batch ? n_pad : batch;
    pad_chunk_kernel<TQ><<<(unsigned)((n_launch + kPadThreads - 1) / kPadThreads), kPadThreads, 0, stream>>>(
        static_cast<const TQ*>(q), static_cast<TQ*>(pb.q_pad), pos0, pb.pos_sub, n_pad, batch, n_new,
        c0, nc, s.n_kv, s.group, p.group, s.cap, D, ws.status);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    e = launch_prefill(p, pb.q_pad, kc, vc, pb.pos_sub, pb.out_pad, batch, nc, max_len, ws, stream);
    if (e != hipSuccess) return e;
    unpad_chunk_kernel<TO><<<(unsigned)((n_real + kPadThreads - 1) / kPadThreads), kPadThreads, 0, stream>>>(
        static_cast<const TO*>(pb.out_pad), static_cast<TO*>(out), n_real, n_new, c0, nc, s.n_kv, s.group,
        p.group, D);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_padded_prefill(const Shape& s, const void* q, const void* k_cache,
                                 const void* v_cache, const int32_t* pos0, void* out, int batch,
                                 int n_new, int max_len, const Workspace& ws, const PadBuffers& pb,
                                 hipStream_t stream) {
  if (padded_group(s.head_dim, s.group) == 0 || !prefill_head_dim(s.head_dim) || !pb.q_pad || !pb.out_pad ||
      !pb.pos_sub || pb.chunk_tokens < 1)
    return hipErrorInvalidValue;
  if (s.q16)
    return s.o16 ? run_padded_prefill<f16, f16>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, pb, stream)
                 : run_padded_prefill<f16, float>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, pb, stream);
  return s.o16 ? run_padded_prefill<float, f16>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, pb, stream)
               : run_padded_prefill<float, float>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, pb, stream);
}

}  // namespace nwd
