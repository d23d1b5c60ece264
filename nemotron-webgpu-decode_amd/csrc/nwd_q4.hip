// nwd_q4.hip — 4-bit GEMV for gfx950, plain and fused with kv_append.
//
// Replaces kernels/matmul_nbits_sg.wgsl main (:81-137), the projection the
// reference runs for every linear layer of a decode step, here for the
// attention layer: the q/k/v projections of the normalised hidden state
// (engine/runtime.js:386-388) followed by kv_append of k and v (:389-390),
// and o_proj (:392) followed by the residual add (:393, kernels/add.wgsl).
//
// Weights are in the reference's format (engine/weights.js:99-104): quant
// uint8 [N][n_blocks][16] (32 weights per block along K, element 2j in the
// low nibble of byte j), scales f32 [N][n_blocks], zero points 4-bit packed
// in order of the flat index col * n_blocks + blk. One weight is
// (nib - zp) * scale.
//
// Mapping: a 256-thread workgroup (4 wavefronts) owns 16 consecutive output
// columns, 4 per wavefront. Lane l of a wavefront owns the K-blocks l, l+64,
// l+128, l+192 (kSlots of them) of its 4 columns: it holds the activation of
// those blocks in registers (32 f32 each, plus their sum) and requests every
// quant run (16 bytes), scale and zero-point byte of its 4 columns before
// computing, so a wavefront has all its weight bytes in flight at once. A
// block contributes scale * (sum_i nib_i * x_i - zp * sum_i x_i): 32 FMAs on
// nibbles converted with v_cvt_f32_ubyte, then one FMA and one multiply-add.
// The 64 lanes' partial sums of a column are added with DPP row steps and
// lane-swap exchanges, and lane 0 writes the 4 columns.
//
// The reference instead gives each of its 4-column workgroups 256 threads
// striding over the blocks (98 for K = 3136, so 158 threads idle) and
// reduces through subgroup shuffles and workgroup memory. Its summation
// order is not reproduced: results agree with it to float32 rounding (the
// parity tests bound the difference by 1e-6 of sum |w x|).
//
// Weight traffic is the roofline: 16.5 bytes per 32 weights (quant, scale,
// zero point). The activation (12.5 KB at K = 3136) is read by every
// wavefront from L2.
#include "nwd_argmax.h"
#include "nwd_common.h"
#include "nwd_internal.h"

namespace nwd {

constexpr int kQ4Waves = 4;
constexpr int kQ4Threads = kQ4Waves * 64;
constexpr int kQ4Cols = 4;                       // output columns per wavefront
constexpr int kQ4WgCols = kQ4Waves * kQ4Cols;    // per workgroup

// One activation row's blocks of this lane, in registers.
template <int kSlots> struct Q4Act {
  float x[kSlots][32];
  float sum[kSlots];
};

template <int kSlots>
__device__ inline void q4_load_act(const float* __restrict__ x, int n_blocks, Q4Act<kSlots>& a) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < kSlots; ++j) {
    const int blk = min(lane + 64 * j, n_blocks - 1);  // in range; extra slots get no weight
    const f32x4* p = reinterpret_cast<const f32x4*>(x + blk * 32);
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const f32x4 t = p[v];
      a.x[j][4 * v + 0] = t[0];
      a.x[j][4 * v + 1] = t[1];
      a.x[j][4 * v + 2] = t[2];
      a.x[j][4 * v + 3] = t[3];
    }
  }
}

// Sums of the lane's activation blocks (after the weight loads are issued,
// so that waiting for the activation does not wait for them).
template <int kSlots>
__device__ inline void q4_act_sums(Q4Act<kSlots>& a) {
#pragma unroll
  for (int j = 0; j < kSlots; ++j) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) s += a.x[j][i];
    a.sum[j] = s;
  }
}

// Wavefront-wide dot products of columns col0 .. col0+3 of `m` with the
// activation in `a`; every lane returns the 4 sums. Columns past m.n read
// column m.n - 1 (their results are not written).
template <int kSlots>
__device__ inline void q4_columns(const Q4Mat& m, int n_blocks, int col0, Q4Act<kSlots>& a,
                                  float (&out)[kQ4Cols]) {
  const int lane = threadIdx.x & 63;
  uint4 qv[kQ4Cols][kSlots];
  float sc[kQ4Cols][kSlots];
  uint32_t zb[kQ4Cols][kSlots];
  int64_t idx[kQ4Cols][kSlots];
#pragma unroll
  for (int c = 0; c < kQ4Cols; ++c) {
    const int col = min(col0 + c, m.n - 1);
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
      const int blk = min(lane + 64 * j, n_blocks - 1);
      idx[c][j] = (int64_t)col * n_blocks + blk;
      qv[c][j] = *reinterpret_cast<const uint4*>(m.quant + idx[c][j] * 16);
      sc[c][j] = m.scales[idx[c][j]];
      zb[c][j] = m.zp[idx[c][j] >> 1];
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // every load above is issued before any compute
  q4_act_sums<kSlots>(a);
#pragma unroll
  for (int c = 0; c < kQ4Cols; ++c) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
      const uint32_t w[4] = {qv[c][j].x, qv[c][j].y, qv[c][j].z, qv[c][j].w};
      float d = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        uint32_t lo = w[k] & 0x0F0F0F0Fu, hi = (w[k] >> 4) & 0x0F0F0F0Fu;
        // Opaque to the optimiser, so each nibble becomes one
        // v_cvt_f32_ubyteN of the masked word instead of a bit-field
        // extract plus a conversion.
        asm volatile("" : "+v"(lo), "+v"(hi));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          d = fmaf((float)((lo >> (8 * e)) & 255u), a.x[j][8 * k + 2 * e], d);
          d = fmaf((float)((hi >> (8 * e)) & 255u), a.x[j][8 * k + 2 * e + 1], d);
        }
      }
      const float z = (float)((idx[c][j] & 1) ? (zb[c][j] >> 4) : (zb[c][j] & 15u));
      const float blk_sum = sc[c][j] * fmaf(-z, a.sum[j], d);
      acc += lane + 64 * j < n_blocks ? blk_sum : 0.f;
    }
    out[c] = sum64(acc);
  }
}

template <int kSlots, int kEpi>
__global__ __launch_bounds__(kQ4Threads) void q4_gemv_kernel(const float* __restrict__ x,
                                                             const Q4Mat m, int n_blocks,
                                                             float* __restrict__ y) {
  const int b = blockIdx.y;
  const int col0 = blockIdx.x * kQ4WgCols + (threadIdx.x >> 6) * kQ4Cols;
  if (col0 >= m.n) return;  // whole wavefront
  Q4Act<kSlots> a;
  q4_load_act<kSlots>(x + (int64_t)b * n_blocks * 32, n_blocks, a);
  float r[kQ4Cols];
  q4_columns<kSlots>(m, n_blocks, col0, a, r);
  if ((threadIdx.x & 63) != 0) return;
  float* yb = y + (int64_t)b * m.n;
  float prev[kQ4Cols];
  if constexpr (kEpi == kQ4Accumulate) {
#pragma unroll
    for (int c = 0; c < kQ4Cols; ++c) prev[c] = col0 + c < m.n ? yb[col0 + c] : 0.f;
  }
#pragma unroll
  for (int c = 0; c < kQ4Cols; ++c) {
    float v = r[c];
    if constexpr (kEpi == kQ4Relu2) {
      const float t = fmaxf(v, 0.f);
      v = t * t;
    }
    if constexpr (kEpi == kQ4Accumulate) v = prev[c] + v;  // H[i] = H[i] + B[i]
    if (col0 + c < m.n) yb[col0 + c] = v;
  }
}

// lm_head with the argmax partial in its epilogue (engine/runtime.js:397-
// 399: the lm-head GEMV, then argmax_partial): each workgroup's 16 logits
// become one 64-bit record (nwd_argmax.h) for argmax_merge_kernel. No
// wavefront returns before the barrier: columns past n are computed on the
// clamped column n - 1 and not recorded.
template <int kSlots>
__global__ __launch_bounds__(kQ4Threads) void q4_argmax_kernel(
    const float* __restrict__ x, const Q4Mat m, int n_blocks, float* __restrict__ logits,
    unsigned long long* __restrict__ records) {
  __shared__ unsigned long long best;
  if (threadIdx.x == 0) best = 0ull;
  __syncthreads();
  const int b = blockIdx.y;
  const int col0 = blockIdx.x * kQ4WgCols + (threadIdx.x >> 6) * kQ4Cols;
  Q4Act<kSlots> a;
  q4_load_act<kSlots>(x + (int64_t)b * n_blocks * 32, n_blocks, a);
  float r[kQ4Cols];
  q4_columns<kSlots>(m, n_blocks, col0, a, r);
  if ((threadIdx.x & 63) == 0) {
    const ArgmaxShape s = argmax_shape(m.n);
    unsigned long long e = 0ull;
#pragma unroll
    for (int c = 0; c < kQ4Cols; ++c) {
      const int col = col0 + c;
      if (col < m.n) {
        if (logits) logits[(int64_t)b * m.n + col] = r[c];
        const unsigned long long v = argmax_enc(r[c], col, s);
        e = v > e ? v : e;
      }
    }
    atomicMax(&best, e);
  }
  __syncthreads();
  if (threadIdx.x == 0) records[(int64_t)b * gridDim.x + blockIdx.x] = best;
}

// Columns [0, Nq) are q, [Nq, Nq + Nkv) k, [Nq + Nkv, Nq + 2 Nkv) v; every
// range is a multiple of 128 (whole heads), so a workgroup's 16 columns lie
// in one of them.
template <int kSlots, bool kQ16>
__global__ __launch_bounds__(kQ4Threads) void qkv_append_kernel(
    const float* __restrict__ x, const Q4Mat mq, const Q4Mat mk, const Q4Mat mv, int n_blocks,
    void* __restrict__ q_out, f16* __restrict__ k_cache, f16* __restrict__ v_cache,
    const int32_t* __restrict__ pos, int n_kv, int cap, int* __restrict__ status) {
  const int b = blockIdx.y;
  int col0 = blockIdx.x * kQ4WgCols + (threadIdx.x >> 6) * kQ4Cols;
  int which = 0;
  if (col0 >= mq.n) {
    col0 -= mq.n;
    which = 1;
    if (col0 >= mk.n) {
      col0 -= mk.n;
      which = 2;
    }
  }
  const Q4Mat& m = which == 0 ? mq : (which == 1 ? mk : mv);
  Q4Act<kSlots> a;
  q4_load_act<kSlots>(x + (int64_t)b * n_blocks * 32, n_blocks, a);
  float r[kQ4Cols];
  q4_columns<kSlots>(m, n_blocks, col0, a, r);
  if ((threadIdx.x & 63) != 0) return;
  if (which == 0) {
    const int64_t at = (int64_t)b * mq.n + col0;
    if constexpr (kQ16) {
      f16x4 h;
#pragma unroll
      for (int c = 0; c < kQ4Cols; ++c) h[c] = (f16)r[c];
      *reinterpret_cast<f16x4*>(static_cast<f16*>(q_out) + at) = h;
    } else {
      *reinterpret_cast<f32x4*>(static_cast<float*>(q_out) + at) = f32x4{r[0], r[1], r[2], r[3]};
    }
    return;
  }
  // kv_append (kernels/kv_append.wgsl:12-18) of this row's 4 values, rounded
  // to fp16, at position pos[b]; a position outside the cache writes nothing
  // and is reported through the status word.
  const int p = pos[b];
  if (p < 0 || p >= cap) {
    if (col0 == 0) atomicOr(status, kStatusBadPos);  // once per projection
    return;
  }
  f16x4 h;
#pragma unroll
  for (int c = 0; c < kQ4Cols; ++c) h[c] = (f16)r[c];
  f16* cache = which == 1 ? k_cache : v_cache;
  *reinterpret_cast<f16x4*>(cache + cache_index(b, p, col0 / kHeadDim, col0 % kHeadDim, n_kv, cap)) = h;
}

namespace {

int q4_slots(int n_blocks) { return (n_blocks + 63) / 64; }

template <int kSlots>
hipError_t launch_gemv_slots(const float* x, const Q4Mat& w, int n_blocks, float* y, int batch,
                             int epilogue, hipStream_t stream) {
  const dim3 grid((w.n + kQ4WgCols - 1) / kQ4WgCols, batch);
  switch (epilogue) {
    case kQ4None:
      q4_gemv_kernel<kSlots, kQ4None><<<grid, kQ4Threads, 0, stream>>>(x, w, n_blocks, y);
      break;
    case kQ4Relu2:
      q4_gemv_kernel<kSlots, kQ4Relu2><<<grid, kQ4Threads, 0, stream>>>(x, w, n_blocks, y);
      break;
    default:
      q4_gemv_kernel<kSlots, kQ4Accumulate><<<grid, kQ4Threads, 0, stream>>>(x, w, n_blocks, y);
      break;
  }
  return hipGetLastError();
}

template <int kSlots>
hipError_t launch_qkv_slots(const Shape& s, const float* x, const Q4Mat& wq, const Q4Mat& wk,
                            const Q4Mat& wv, int n_blocks, void* q_out, void* k_cache,
                            void* v_cache, const int32_t* pos, int batch, int* status,
                            hipStream_t stream) {
  const dim3 grid((wq.n + wk.n + wv.n) / kQ4WgCols, batch);
  f16* kc = static_cast<f16*>(k_cache);
  f16* vc = static_cast<f16*>(v_cache);
  if (s.q16)
    qkv_append_kernel<kSlots, true><<<grid, kQ4Threads, 0, stream>>>(
        x, wq, wk, wv, n_blocks, q_out, kc, vc, pos, s.n_kv, s.cap, status);
  else
    qkv_append_kernel<kSlots, false><<<grid, kQ4Threads, 0, stream>>>(
        x, wq, wk, wv, n_blocks, q_out, kc, vc, pos, s.n_kv, s.cap, status);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_q4_gemv(const float* x, const Q4Mat& w, int n_blocks, float* y, int batch,
                          int epilogue, hipStream_t stream) {
  switch (q4_slots(n_blocks)) {
    case 1: return launch_gemv_slots<1>(x, w, n_blocks, y, batch, epilogue, stream);
    case 2: return launch_gemv_slots<2>(x, w, n_blocks, y, batch, epilogue, stream);
    case 3: return launch_gemv_slots<3>(x, w, n_blocks, y, batch, epilogue, stream);
    case 4: return launch_gemv_slots<4>(x, w, n_blocks, y, batch, epilogue, stream);
    default: return hipErrorInvalidValue;
  }
}

int q4_argmax_records_per_row(int n) { return (n + kQ4WgCols - 1) / kQ4WgCols; }

hipError_t launch_q4_argmax(const float* x, const Q4Mat& w, int n_blocks, float* logits,
                            uint32_t* out, int batch, unsigned long long* records,
                            hipStream_t stream) {
  const int per_row = q4_argmax_records_per_row(w.n);
  const dim3 grid(per_row, batch);
  switch (q4_slots(n_blocks)) {
    case 1: q4_argmax_kernel<1><<<grid, kQ4Threads, 0, stream>>>(x, w, n_blocks, logits, records); break;
    case 2: q4_argmax_kernel<2><<<grid, kQ4Threads, 0, stream>>>(x, w, n_blocks, logits, records); break;
    case 3: q4_argmax_kernel<3><<<grid, kQ4Threads, 0, stream>>>(x, w, n_blocks, logits, records); break;
    case 4: q4_argmax_kernel<4><<<grid, kQ4Threads, 0, stream>>>(x, w, n_blocks, logits, records); break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_argmax_merge(records, per_row, w.n, out, batch, stream);
}

hipError_t launch_qkv_append(const Shape& s, const float* x, const Q4Mat& wq, const Q4Mat& wk,
                             const Q4Mat& wv, int n_blocks, void* q_out, void* k_cache,
                             void* v_cache, const int32_t* pos, int batch, int* status,
                             hipStream_t stream) {
  switch (q4_slots(n_blocks)) {
    case 1: return launch_qkv_slots<1>(s, x, wq, wk, wv, n_blocks, q_out, k_cache, v_cache, pos, batch, status, stream);
    case 2: return launch_qkv_slots<2>(s, x, wq, wk, wv, n_blocks, q_out, k_cache, v_cache, pos, batch, status, stream);
    case 3: return launch_qkv_slots<3>(s, x, wq, wk, wv, n_blocks, q_out, k_cache, v_cache, pos, batch, status, stream);
    case 4: return launch_qkv_slots<4>(s, x, wq, wk, wv, n_blocks, q_out, k_cache, v_cache, pos, batch, status, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace nwd
