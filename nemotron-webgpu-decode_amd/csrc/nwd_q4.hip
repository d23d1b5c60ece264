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
// Mapping: a 256-thread workgroup (4 wavefronts) owns 16 / kSplit groups of
// 4 consecutive output columns; kSplit wavefronts share a group, each taking
// 1/kSplit of the K-blocks (kSplit = 4 at K = 5120, 2 at K = 3136: at least
// 32 blocks per wavefront). Lane l of a wavefront owns the blocks first + l,
// first + l + 64, ... (kSlots of them) of its part for the group's 4 columns:
// it holds the activation of those blocks in registers (32 f32 each, plus
// their sum) and requests every quant run (16 bytes), scale and zero-point
// byte before computing, so a wavefront has all its weight bytes in flight
// at once. A block contributes scale * (sum_i nib_i * x_i - zp * sum_i x_i):
// 32 FMAs on nibbles converted with v_cvt_f32_ubyte, then one FMA and one
// multiply-add. The 64 lanes' partial sums of a column are added with DPP
// row steps and lane-swap exchanges, the parts' sums through LDS in part
// order, and one lane writes the 4 columns. Splitting K over wavefronts
// shortens each wavefront's serial chain (the kernels are latency-bound at
// batch 1): 7.8 -> 7.0 us for q/k/v, 7.5 -> 6.6 us for o_proj.
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

// Blocks [first, end) of the row, lane l taking first + l, first + l + 64,
// ... (clamped in range; slots past end get no weight).
template <int kSlots>
__device__ inline void q4_load_act(const float* __restrict__ x, int first, int end, Q4Act<kSlots>& a) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < kSlots; ++j) {
    const int blk = min(first + lane + 64 * j, end - 1);
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
__device__ inline void q4_columns(const Q4Mat& m, int n_blocks, int first, int end, int col0,
                                  Q4Act<kSlots>& a, float (&out)[kQ4Cols]) {
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
      const int blk = min(first + lane + 64 * j, end - 1);
      idx[c][j] = (int64_t)col * n_blocks + blk;
      // non-temporal: each weight byte is read once per call (1-2% faster
      // here; the wide form below keeps the default policy, under which the
      // lm_head measured 52.5 us against 56.4 with its quant stream, 73.1
      // with all three streams, non-temporal)
      qv[c][j] = __builtin_bit_cast(
          uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(m.quant + idx[c][j] * 16)));
      sc[c][j] = __builtin_nontemporal_load(m.scales + idx[c][j]);
      zb[c][j] = __builtin_nontemporal_load(m.zp + (idx[c][j] >> 1));
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
      acc += first + lane + 64 * j < end ? blk_sum : 0.f;
    }
    out[c] = sum64(acc);
  }
}

// kSplit wavefronts share a group of 4 columns, each taking 1/kSplit of
// the blocks; their sums are added through LDS in part order.
template <int kSplit> struct Q4Part {
  static constexpr int kGroups = kQ4Waves / kSplit;  // column groups per workgroup
  static constexpr int kWgCols = kGroups * kQ4Cols;
  int col0, first, end, part;
  __device__ Q4Part(int n_blocks) {
    const int w = threadIdx.x >> 6;
    part = w % kSplit;
    col0 = (blockIdx.x * kGroups + w / kSplit) * kQ4Cols;
    const int per = (n_blocks + kSplit - 1) / kSplit;
    first = min(part * per, n_blocks - 1);
    end = min(part * per + per, n_blocks);
  }
  // Adds the parts' sums into part 0's lane 0; true on that lane.
  __device__ bool reduce(float (&r)[kQ4Cols]) {
    if constexpr (kSplit == 1) {
      return (threadIdx.x & 63) == 0;
    } else {
      __shared__ float sums[kQ4Waves][kQ4Cols];
      const int w = threadIdx.x >> 6;
      if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int c = 0; c < kQ4Cols; ++c) sums[w][c] = r[c];
      }
      __syncthreads();
      if (part != 0 || (threadIdx.x & 63) != 0) return false;
#pragma unroll
      for (int c = 0; c < kQ4Cols; ++c) {
        float v = sums[w][c];
#pragma unroll
        for (int p = 1; p < kSplit; ++p) v += sums[w + p][c];
        r[c] = v;
      }
      return true;
    }
  }
};

template <int kSlots, int kSplit, int kEpi>
__global__ __launch_bounds__(kQ4Threads) void q4_gemv_kernel(const float* __restrict__ x,
                                                             const Q4Mat m, int n_blocks,
                                                             float* __restrict__ y) {
  const int b = blockIdx.y;
  Q4Part<kSplit> pt(n_blocks);
  const int col0 = pt.col0;
  if (kSplit == 1 && col0 >= m.n) return;  // whole wavefront (no barrier follows)
  float* yb = y + (int64_t)b * m.n;
  // The residual is requested with the weights, not after the reduction,
  // where it would add a dependent memory round trip to the chain.
  float prev[kQ4Cols];
  if constexpr (kEpi == kQ4Accumulate) {
#pragma unroll
    for (int c = 0; c < kQ4Cols; ++c) prev[c] = yb[min(col0 + c, m.n - 1)];
  }
  Q4Act<kSlots> a;
  q4_load_act<kSlots>(x + (int64_t)b * n_blocks * 32, pt.first, pt.end, a);
  float r[kQ4Cols];
  q4_columns<kSlots>(m, n_blocks, pt.first, pt.end, col0, a, r);
  if (!pt.reduce(r) || col0 >= m.n) return;
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
  q4_load_act<kSlots>(x + (int64_t)b * n_blocks * 32, 0, n_blocks, a);
  float r[kQ4Cols];
  q4_columns<kSlots>(m, n_blocks, 0, n_blocks, col0, a, r);
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

// ---------------------------------------------------------------------------
// Wide form, for projections with many columns (lm_head: 131072). A 128-thread
// workgroup owns 16 columns, 8 lanes per column; lane j of a column takes
// blocks j, j+8, ... (kIters of them). The activation row goes to LDS once per
// workgroup with its block sums, so a lane's registers hold only its weights
// (all requested at once) and one block of activation at a time: about 40%
// fewer VALU instructions per weight than the form above. That form wins when
// the grid is small (a wavefront there has fewer iterations in its chain and
// each SIMD has few wavefronts to hide it); this one when the grid fills the
// chip many times over.
constexpr int kQ4wThreads = 128;
constexpr int kQ4wLanes = 8;
constexpr int kQ4wWgCols = kQ4wThreads / kQ4wLanes;  // 16, as the form above
static_assert(kQ4wWgCols == kQ4WgCols, "both forms write one record per 16 columns");
constexpr int kQ4wMinCols = 16384;  // below this the form above is used

// A block of activation takes 36 floats of LDS, not 32: the 8 lanes of a
// column read blocks j, j+8, ... together, and at a 128-byte stride every
// second one would share LDS banks; at 144 bytes their 16-byte reads land
// on distinct banks.
constexpr int kQ4wXStride = 36;
template <int kIters> struct Q4wLds {
  static constexpr int kBlocks = kIters * kQ4wLanes;  // >= n_blocks
  float x[kBlocks * kQ4wXStride];
  float sum[kBlocks];
};

// Column `col` (in range) of m dotted with activation row `xrow`; every lane
// of the column's group of 8 returns the sum. The weights of iteration i of a
// lane sit at a constant distance from its first block, so each load is one
// buffer instruction with an immediate offset; blocks past n_blocks read the
// next column's bytes, or zeros past the matrix, and get no weight.
// kStage: load the activation row and stage it in LDS first (the first
// column group of a workgroup); later groups read what the first staged.
template <int kIters, bool kStage = true>
__device__ inline float q4w_dot(const Q4Mat& m, int n_blocks, int col,
                                const float* __restrict__ xrow, Q4wLds<kIters>& lds) {
  constexpr int kXRounds = (kIters * kQ4wLanes + kQ4wThreads - 1) / kQ4wThreads;
  const int t = threadIdx.x;
  const int j = t & (kQ4wLanes - 1);
  f32x4 xv[kXRounds][8];
  if constexpr (kStage) {
#pragma unroll
    for (int r = 0; r < kXRounds; ++r) {
      const f32x4* p = reinterpret_cast<const f32x4*>(xrow + min(t + r * kQ4wThreads, n_blocks - 1) * 32);
#pragma unroll
      for (int v = 0; v < 8; ++v) xv[r][v] = p[v];
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // activation loads first: waiting for them waits for no weight
  const int cells = m.n * n_blocks;   // the host keeps 16 * cells < 2^31
  const auto rq = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(m.quant), 0, cells * 16, kBufferWord3);
  const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(m.scales), 0, cells * 4, kBufferWord3);
  const auto rz = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(m.zp), 0, (cells + 1) / 2, kBufferWord3);
  const int first = col * n_blocks + j;
  uint4 qv[kIters];
  float sc[kIters];
  uint32_t zb[kIters];
#pragma unroll
  for (int i = 0; i < kIters; ++i) {
    qv[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rq, first * 16 + 128 * i, 0, 0));
    sc[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, first * 4 + 32 * i, 0, 0));
    zb[i] = __builtin_amdgcn_raw_buffer_load_b8(rz, (first >> 1) + 4 * i, 0, 0);
    __builtin_amdgcn_sched_barrier(0);  // in iteration order: iteration i waits for i's loads only
  }
  // Block first + 8 i has the parity of `first`: the same zero-point nibble.
  const uint32_t zshift = (first & 1) * 4;
  if constexpr (kStage) {
    // Activation to LDS with block sums. Unconditional (a conditional store
    // lets the compiler sink the activation loads behind the weights): a
    // thread past n_blocks holds block n_blocks - 1 and stores it to a spare
    // slot, or to slot n_blocks - 1 itself with the same values.
#pragma unroll
    for (int r = 0; r < kXRounds; ++r) {
      const int slot = min(t + r * kQ4wThreads, Q4wLds<kIters>::kBlocks - 1);
      float s = 0.f;
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        *reinterpret_cast<f32x4*>(&lds.x[slot * kQ4wXStride + 4 * v]) = xv[r][v];
        s += (xv[r][v][0] + xv[r][v][1]) + (xv[r][v][2] + xv[r][v][3]);
      }
      lds.sum[slot] = s;
    }
    // LDS-only barrier: waits for this thread's LDS writes, not for its
    // outstanding weight loads (a __syncthreads fence would wait for those).
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
  }
  const f32x4* xl = reinterpret_cast<const f32x4*>(&lds.x[j * kQ4wXStride]);
  const float* sl = &lds.sum[j];
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < kIters; ++i) {
    const f32x4* xb = xl + (kQ4wXStride / 4) * kQ4wLanes * i;
    const uint32_t w[4] = {qv[i].x, qv[i].y, qv[i].z, qv[i].w};
    float d = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t lo = w[k] & 0x0F0F0F0Fu, hi = (w[k] >> 4) & 0x0F0F0F0Fu;
      asm volatile("" : "+v"(lo), "+v"(hi));  // one v_cvt_f32_ubyteN per nibble
      const f32x4 xe = xb[2 * k], xo = xb[2 * k + 1];  // elements 8k .. 8k+7
      d = fmaf((float)(lo & 255u), xe[0], d);
      d = fmaf((float)(hi & 255u), xe[1], d);
      d = fmaf((float)((lo >> 8) & 255u), xe[2], d);
      d = fmaf((float)((hi >> 8) & 255u), xe[3], d);
      d = fmaf((float)((lo >> 16) & 255u), xo[0], d);
      d = fmaf((float)((hi >> 16) & 255u), xo[1], d);
      d = fmaf((float)(lo >> 24), xo[2], d);
      d = fmaf((float)(hi >> 24), xo[3], d);
    }
    const float z = (float)((zb[i] >> zshift) & 15u);
    const float blk_sum = sc[i] * fmaf(-z, sl[kQ4wLanes * i], d);
    acc += j + kQ4wLanes * i < n_blocks ? blk_sum : 0.f;
    // One iteration at a time: otherwise the scheduler hoists every
    // iteration's activation reads (32 registers each) ahead of the math.
    __builtin_amdgcn_sched_barrier(0);
  }
  return sum8(acc);
}

// lm_head + argmax partial, wide form: the record of each group of 16
// columns goes to argmax_merge_kernel like the form above. A workgroup may
// take kQ4wGroups consecutive groups and stage the activation once for all
// of them; on lm_head (131072 x 3136) 1 group measured 52 us against 57.5
// and 58.9 us for 2 and 4 (fewer workgroups, and a group's weight loads wait
// for the previous group's math). The kernel written without the group loop
// compiles to another schedule that measured 56.6 us, with the same results.
constexpr int kQ4wGroups = 1;
template <int kIters>
__global__ __launch_bounds__(kQ4wThreads, 2) void q4w_argmax_kernel(
    const float* __restrict__ x, const Q4Mat m, int n_blocks, float* __restrict__ logits,
    unsigned long long* __restrict__ records, int per_row) {
  __shared__ __attribute__((aligned(16))) Q4wLds<kIters> lds;
  __shared__ unsigned long long best[kQ4wGroups];
  if (threadIdx.x < kQ4wGroups) best[threadIdx.x] = 0ull;  // visible after q4w_dot's barrier
  const int b = blockIdx.y;
#pragma unroll
  for (int g = 0; g < kQ4wGroups; ++g) {
    const int col = (blockIdx.x * kQ4wGroups + g) * kQ4wWgCols + (threadIdx.x >> 3);
    const float r = g == 0 ? q4w_dot<kIters, true>(m, n_blocks, min(col, m.n - 1), x + (int64_t)b * n_blocks * 32, lds)
                           : q4w_dot<kIters, false>(m, n_blocks, min(col, m.n - 1), x + (int64_t)b * n_blocks * 32, lds);
    if ((threadIdx.x & (kQ4wLanes - 1)) == 0 && col < m.n) {
      if (logits) logits[(int64_t)b * m.n + col] = r;
      atomicMax(&best[g], argmax_enc(r, col, argmax_shape(m.n)));
    }
  }
  __syncthreads();
  if (threadIdx.x < kQ4wGroups) {
    const int rec = blockIdx.x * kQ4wGroups + threadIdx.x;
    if (rec < per_row) records[(int64_t)b * per_row + rec] = best[threadIdx.x];
  }
}

// Columns [0, Nq) are q, [Nq, Nq + Nkv) k, [Nq + Nkv, Nq + 2 Nkv) v, with
// Nq = H * D and Nkv = Hkv * D. The host accepts only shapes where both are
// multiples of 16 and D of 4, so a workgroup's 16 columns lie in one range
// and a wavefront's 4 in one head (at D = 128 always).
template <int kSlots, int kSplit, bool kQ16>
__global__ __launch_bounds__(kQ4Threads) void qkv_append_kernel(
    const float* __restrict__ x, const Q4Mat mq, const Q4Mat mk, const Q4Mat mv, int n_blocks,
    void* __restrict__ q_out, f16* __restrict__ k_cache, f16* __restrict__ v_cache,
    const int32_t* __restrict__ pos, int n_kv, int D, int cap, int* __restrict__ status) {
  const int b = blockIdx.y;
  Q4Part<kSplit> pt(n_blocks);
  int col0 = pt.col0;
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
  const int p = which == 0 ? 0 : pos[b];  // requested before the weights, as the residual above
  Q4Act<kSlots> a;
  q4_load_act<kSlots>(x + (int64_t)b * n_blocks * 32, pt.first, pt.end, a);
  float r[kQ4Cols];
  q4_columns<kSlots>(m, n_blocks, pt.first, pt.end, col0, a, r);
  if (!pt.reduce(r)) return;
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
  if (p < 0 || p >= cap) {
    if (col0 == 0) atomicOr(status, kStatusBadPos);  // once per projection
    return;
  }
  f16x4 h;
#pragma unroll
  for (int c = 0; c < kQ4Cols; ++c) h[c] = (f16)r[c];
  f16* cache = which == 1 ? k_cache : v_cache;
  const int64_t at = cache_index_d(b, p, col0 / D, col0 % D, n_kv, cap, D);
  if (!in_bounds(at, kQ4Cols, (int64_t)gridDim.y * n_kv * cap * D, status)) return;
  *reinterpret_cast<f16x4*>(cache + at) = h;
}

namespace {

int q4_slots(int n_blocks) { return (n_blocks + 63) / 64; }

// Iterations per lane of the wide form for n_blocks, rounded up to an
// instantiated count; 0 if n_blocks is past its limit.
int q4w_iters(int n_blocks) {
  const int need = (n_blocks + kQ4wLanes - 1) / kQ4wLanes;
  for (int k : {1, 2, 3, 4, 6, 8, 10, 13, 16, 20, 24})
    if (k >= need) return k;
  return 0;
}

template <int kSlots, int kSplit>
hipError_t launch_gemv_slots(const float* x, const Q4Mat& w, int n_blocks, float* y, int batch,
                             int epilogue, hipStream_t stream) {
  constexpr int kCols = Q4Part<kSplit>::kWgCols;
  const dim3 grid((w.n + kCols - 1) / kCols, batch);
  switch (epilogue) {
    case kQ4None:
      q4_gemv_kernel<kSlots, kSplit, kQ4None><<<grid, kQ4Threads, 0, stream>>>(x, w, n_blocks, y);
      break;
    case kQ4Relu2:
      q4_gemv_kernel<kSlots, kSplit, kQ4Relu2><<<grid, kQ4Threads, 0, stream>>>(x, w, n_blocks, y);
      break;
    default:
      q4_gemv_kernel<kSlots, kSplit, kQ4Accumulate><<<grid, kQ4Threads, 0, stream>>>(x, w, n_blocks, y);
      break;
  }
  return hipGetLastError();
}

// Waves per column group: enough that each takes at least 32 blocks.
int q4_split(int n_blocks) {
  return n_blocks >= 128 ? 4 : (n_blocks >= 64 ? 2 : 1);
}

template <int kSlots, int kSplit>
hipError_t launch_qkv_slots(const Shape& s, const float* x, const Q4Mat& wq, const Q4Mat& wk,
                            const Q4Mat& wv, int n_blocks, void* q_out, void* k_cache,
                            void* v_cache, const int32_t* pos, int batch, int* status,
                            hipStream_t stream) {
  const dim3 grid((wq.n + wk.n + wv.n) / Q4Part<kSplit>::kWgCols, batch);
  f16* kc = static_cast<f16*>(k_cache);
  f16* vc = static_cast<f16*>(v_cache);
  if (s.q16)
    qkv_append_kernel<kSlots, kSplit, true><<<grid, kQ4Threads, 0, stream>>>(
        x, wq, wk, wv, n_blocks, q_out, kc, vc, pos, s.n_kv, s.head_dim, s.cap, status);
  else
    qkv_append_kernel<kSlots, kSplit, false><<<grid, kQ4Threads, 0, stream>>>(
        x, wq, wk, wv, n_blocks, q_out, kc, vc, pos, s.n_kv, s.head_dim, s.cap, status);
  return hipGetLastError();
}

template <int kSplit>
hipError_t launch_qkv_split(const Shape& s, const float* x, const Q4Mat& wq, const Q4Mat& wk,
                            const Q4Mat& wv, int n_blocks, void* q_out, void* k_cache,
                            void* v_cache, const int32_t* pos, int batch, int* status,
                            hipStream_t stream) {
  switch (q4_slots((n_blocks + kSplit - 1) / kSplit)) {
    case 1: return launch_qkv_slots<1, kSplit>(s, x, wq, wk, wv, n_blocks, q_out, k_cache, v_cache, pos, batch, status, stream);
    case 2: return launch_qkv_slots<2, kSplit>(s, x, wq, wk, wv, n_blocks, q_out, k_cache, v_cache, pos, batch, status, stream);
    case 3: return launch_qkv_slots<3, kSplit>(s, x, wq, wk, wv, n_blocks, q_out, k_cache, v_cache, pos, batch, status, stream);
    case 4: return launch_qkv_slots<4, kSplit>(s, x, wq, wk, wv, n_blocks, q_out, k_cache, v_cache, pos, batch, status, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int kSplit>
hipError_t launch_gemv_split(const float* x, const Q4Mat& w, int n_blocks, float* y, int batch,
                             int epilogue, hipStream_t stream) {
  switch (q4_slots((n_blocks + kSplit - 1) / kSplit)) {
    case 1: return launch_gemv_slots<1, kSplit>(x, w, n_blocks, y, batch, epilogue, stream);
    case 2: return launch_gemv_slots<2, kSplit>(x, w, n_blocks, y, batch, epilogue, stream);
    case 3: return launch_gemv_slots<3, kSplit>(x, w, n_blocks, y, batch, epilogue, stream);
    case 4: return launch_gemv_slots<4, kSplit>(x, w, n_blocks, y, batch, epilogue, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_q4_gemv(const float* x, const Q4Mat& w, int n_blocks, float* y, int batch,
                          int epilogue, hipStream_t stream) {
  switch (q4_split(n_blocks)) {
    case 1: return launch_gemv_split<1>(x, w, n_blocks, y, batch, epilogue, stream);
    case 2: return launch_gemv_split<2>(x, w, n_blocks, y, batch, epilogue, stream);
    default: return launch_gemv_split<4>(x, w, n_blocks, y, batch, epilogue, stream);
  }
}

int q4_argmax_records_per_row(int n) { return (n + kQ4WgCols - 1) / kQ4WgCols; }

hipError_t launch_q4_argmax(const float* x, const Q4Mat& w, int n_blocks, float* logits,
                            uint32_t* out, int batch, unsigned long long* records,
                            hipStream_t stream) {
  const int per_row = q4_argmax_records_per_row(w.n);
  const dim3 grid(per_row, batch);
  const int iters = q4w_iters(n_blocks);  // 0 past 24 blocks per lane (K > 6144)
  // byte offsets into the quant array must stay below 2^31
  if (w.n >= kQ4wMinCols && iters > 0 && (int64_t)w.n * n_blocks * 16 < ((int64_t)1 << 31)) {
    const dim3 wgrid((per_row + kQ4wGroups - 1) / kQ4wGroups, batch);
    switch (iters) {
#define NWD_Q4W_CASE(K) \
  case K: q4w_argmax_kernel<K><<<wgrid, kQ4wThreads, 0, stream>>>(x, w, n_blocks, logits, records, per_row); break;
      NWD_Q4W_CASE(1) NWD_Q4W_CASE(2) NWD_Q4W_CASE(3) NWD_Q4W_CASE(4) NWD_Q4W_CASE(6)
      NWD_Q4W_CASE(8) NWD_Q4W_CASE(10) NWD_Q4W_CASE(13) NWD_Q4W_CASE(16) NWD_Q4W_CASE(20)
      NWD_Q4W_CASE(24)
#undef NWD_Q4W_CASE
      default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_argmax_merge(records, per_row, w.n, out, batch, stream);
  }
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
  switch (q4_split(n_blocks)) {
    case 1: return launch_qkv_split<1>(s, x, wq, wk, wv, n_blocks, q_out, k_cache, v_cache, pos, batch, status, stream);
    case 2: return launch_qkv_split<2>(s, x, wq, wk, wv, n_blocks, q_out, k_cache, v_cache, pos, batch, status, stream);
    default: return launch_qkv_split<4>(s, x, wq, wk, wv, n_blocks, q_out, k_cache, v_cache, pos, batch, status, stream);
  }
}

}  // namespace nwd
