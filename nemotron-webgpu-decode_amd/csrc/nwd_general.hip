// nwd_general.hip — decode and prefill attention for the shapes the
// specialised kernels are not built for: any head size D up to kMaxHeadDim
// and any group size G = H / Hkv.
//
// The reference kernel takes head_dim and both head counts as parameters
// (kernels/sparse_attn.wgsl:12-17, :38-43), so a caller may bind any of them.
// The split and MFMA kernels (nwd_decode.hip, nwd_decode_hd.hip,
// nwd_prefill.hip, nwd_prefill_wide.hip) take the head sizes that are
// multiples of 8 up to 256 and, through several groups per KV head or padded
// query rows, every group. The shapes left (other head sizes, K/V slabs above
// 1 GiB, and the allocation-free entry point's padded groups, which have no
// padded buffers) run here under
// the same contract: the same cache layout, position rules, status bits,
// split-K records (max in log2 units, weight sum, unnormalised o) and fp32
// arithmetic.
//
// A 256-thread workgroup serves one split of the keys of one (sequence,
// query) for gp query heads of one group (gp = G up to 8 at D <= 128, up to
// 4 at D <= 256, 2 beyond; one when D is not a multiple of 8), so the K/V
// rows are read once for all of them. With D a multiple of 8 each wavefront
// walks its own 16-key tiles with its own online softmax per head (no
// barrier in the key loop), requesting its next tile before computing the
// current one, and the four wavefronts are merged at the end; other head
// sizes run a scalar form in 64-key workgroup tiles. Scores are dotted with
// query rows held in LDS, pre-scaled by scale * log2(e) so that they come out
// in log2 units.
//
// Workgroups are dealt to the 8 XCDs round-robin in launch order. The launch
// index is remapped so that each XCD takes a contiguous range of the work in
// the order (sequence, query, KV head, split, head chunk): the workgroups
// reading the same K/V rows run on one XCD.
#include "nwd_common.h"
#include "nwd_internal.h"

namespace nwd {

constexpr int kGenThreads = 256;
constexpr int kGenWaves = kGenThreads / 64;
constexpr int kGenKeys = 64;  // keys per tile: four score threads each
constexpr int kXcds = 8;

struct GeneralArgs {
  const void* q;         // [rows][D], rows = batch * n_new * H
  const f16* k_cache;
  const f16* v_cache;
  const int32_t* pos;    // decode: pos[b] (the newest token); prefill: pos0[b]
  void* out;             // [rows][D]
  float* part_o;         // [rows][nsplit][D] (nsplit > 1)
  float2* part_ml;       // [rows][nsplit]
  int64_t records;       // capacity of part_ml in records, of part_o in records of D
  int D, n_heads, n_kv, group, cap, n_new, nsplit, prefill, split_keys;
  int gp, chunks;        // query heads per workgroup, workgroups per group (ceil(G / gp))
  int rows;              // batch * n_new * H
  int total;             // batch * n_new * Hkv * chunks * nsplit workgroups of work
  float c;               // scale * log2(e)
  int* status;
};

// Runs of 8 a score thread takes, ceil(D / 32), rounded up to 1, 2, 4, 8, 16.
int general_runs_bucket(int D) {
  const int runs = (D / 8 + 3) / 4;
  return runs <= 1 ? 1 : runs <= 2 ? 2 : runs <= 4 ? 4 : runs <= 8 ? 8 : 16;
}

int general_heads_per_workgroup(int head_dim, int group) {
  if (head_dim % 8 != 0) return 1;
  const int b = general_runs_bucket(head_dim);
  const int gp = b <= 4 ? 8 : (b == 8 ? 4 : 2);
  return group < gp ? group : gp;
}

template <bool kQ16>
__device__ inline float load_q(const void* q, int64_t i) {
  if constexpr (kQ16) return (float)static_cast<const f16*>(q)[i];
  else return static_cast<const float*>(q)[i];
}

template <bool kO16>
__device__ inline void store_o(void* out, int64_t i, float v) {
  if constexpr (kO16) static_cast<f16*>(out)[i] = (f16)v;
  else static_cast<float*>(out)[i] = v;
}

__device__ inline float wave_max(float x) {
#pragma unroll
  for (int s = 1; s < 64; s <<= 1) x = fmaxf(x, __shfl_xor(x, s));
  return x;
}

__device__ inline float wave_sum(float x) {
#pragma unroll
  for (int s = 1; s < 64; s <<= 1) x += __shfl_xor(x, s);
  return x;
}

// The work of one workgroup: nm query heads h0 .. h0 + nm - 1 of KV head hk
// (output / record rows row0 .. row0 + nm - 1, row = (b * n_new + qi) * H + h),
// its split and key range [t0, t1).
struct GenWork {
  int row0, nm, split, b, qi, h0, hk, t0, t1;
};

// false: a launch index past the work (the grid is rounded up to whole
// XCD ranges); the workgroup returns before any barrier.
__device__ inline bool general_work(const GeneralArgs& a, GenWork& w) {
  const int lin = blockIdx.x;
  const int per = (a.total + kXcds - 1) / kXcds;
  const int logical = (lin % kXcds) * per + lin / kXcds;
  if (logical >= a.total) return false;
  const int c = logical % a.chunks;
  int rest = logical / a.chunks;
  w.split = rest % a.nsplit;
  rest /= a.nsplit;
  w.hk = rest % a.n_kv;
  rest /= a.n_kv;
  w.qi = rest % a.n_new;
  w.b = rest / a.n_new;
  w.h0 = w.hk * a.group + c * a.gp;
  w.nm = min(a.gp, a.group - c * a.gp);
  w.row0 = (w.b * a.n_new + w.qi) * a.n_heads + w.h0;

  // Keys attended by the row: decode L = pos[b] + 1 (a position outside the
  // cache is flagged and clamped as the specialised decode does); prefill
  // query qi attends keys 0 .. pos0[b] + qi.
  int L;
  const int p_raw = a.pos[w.b];
  const bool flagger = threadIdx.x == 0 && w.split == 0 && w.qi == 0 && w.h0 == 0;
  if (a.prefill) {
    int P0 = p_raw;
    if (P0 < 0 || P0 > a.cap - a.n_new) {
      if (flagger) atomicOr(a.status, kStatusBadPos);
      P0 = P0 < 0 ? 0 : a.cap - a.n_new;
    }
    L = P0 + w.qi + 1;
  } else {
    const bool ok = p_raw >= 0 && p_raw < a.cap;
    if (!ok && flagger) atomicOr(a.status, kStatusBadPos);
    L = ok ? p_raw + 1 : (p_raw < 0 ? 1 : a.cap);
  }
  w.t0 = w.split * a.split_keys;
  w.t1 = w.split == a.nsplit - 1 ? L : min(L, w.t0 + a.split_keys);
  return true;
}

// The query rows of rows row0 .. row0 + n - 1 (consecutive in memory) to LDS.
template <bool kQ16>
__device__ inline void stage_q(const GeneralArgs& a, int row0, int n, float* qs) {
  const int64_t q0 = (int64_t)row0 * a.D;
  for (int i = threadIdx.x; i < n * a.D; i += kGenThreads) qs[i] = a.c * load_q<kQ16>(a.q, q0 + i);
}

// Online-softmax update for one tile. s: this thread's score (its key's, the
// same in the key's four threads), valid when the key is in range. Writes
// the key weights to ps, moves (m, l) and returns the factor earlier
// partial outputs are scaled by. Two barriers; on return ps is published.
__device__ inline float tile_softmax(float s, bool valid, float* ps, float* red_max, float* red_sum,
                                     float& m, float& l) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float tmax = wave_max(valid ? s : kNegBig);
  if (lane == 0) red_max[wave] = tmax;
  __syncthreads();
  float tile_max = red_max[0];
#pragma unroll
  for (int w = 1; w < kGenWaves; ++w) tile_max = fmaxf(tile_max, red_max[w]);
  const float m_new = fmaxf(m, tile_max);
  const float alpha = exp2f(m - m_new);
  const float p = valid ? exp2f(s - m_new) : 0.f;
  const bool lead = (tid & 3) == 0;
  if (lead) ps[tid >> 2] = p;
  const float wsum = wave_sum(lead ? p : 0.f);
  if (lane == 0) red_sum[wave] = wsum;
  __syncthreads();
  float tile_sum = 0.f;
#pragma unroll
  for (int w = 0; w < kGenWaves; ++w) tile_sum += red_sum[w];
  l = fmaf(l, alpha, tile_sum);
  m = m_new;
  return alpha;
}

// Adds the key groups' partial outputs (opart, groups * D floats, written
// by the caller before the barrier here) and writes the row's output, or its
// split record.
template <bool kO16>
__device__ inline void finish_row(const GeneralArgs& a, int row, int split, float m, float l,
                                  int groups, const float* opart) {
  __syncthreads();
  const int D = a.D;
  const int64_t qrow = (int64_t)row * D;
  const int64_t rec = (int64_t)row * a.nsplit + split;
  const int64_t rows = a.rows;
  for (int d = threadIdx.x; d < D; d += kGenThreads) {
    float o = 0.f;
    for (int g = 0; g < groups; ++g) o += opart[g * D + d];
    if (a.nsplit == 1) {
      if (in_bounds(qrow + d, 1, rows * D, a.status)) store_o<kO16>(a.out, qrow + d, o / l);
    } else if (in_bounds(rec * D + d, 1, a.records * D, a.status)) {
      a.part_o[rec * D + d] = o;
    }
  }
  if (a.nsplit > 1 && threadIdx.x == 0 && in_bounds(rec, 1, a.records, a.status))
    a.part_ml[rec] = make_float2(m, l);
}

// Max / sum over the wavefront's 16 quads when the four lanes of each quad
// hold the same value: the other quad of each 8 lanes, the other 8 of each
// 16 (DPP), then the xor-16 and xor-32 exchanges. Each quad counts once.
__device__ inline float max_quads(float x) {
  x = fmaxf(x, dpp_mov<kDppHalfMirror>(x));
  x = fmaxf(x, dpp_mov<kDppRowRor8>(x));
  return max_xor32(max_xor16(x));
}
__device__ inline float sum_quads(float x) {
  x += dpp_mov<kDppHalfMirror>(x);
  x += dpp_mov<kDppRowRor8>(x);
  return sum_xor32(sum_xor16(x));
}

// D a multiple of 8: runs of 8 fp16 values, up to GP query heads per
// workgroup. Each wavefront walks its own 16-key tiles (keys t0 + 16 w,
// then every 64th key on), with its own online softmax per head, so the key
// loop has no workgroup barrier and no wavefront waits for another's loads;
// the four wavefronts' (m, l, o) are merged once at the end. Per tile: four
// lanes per key dot every fourth run with each head's query row (LDS), a
// quad sum and the 16-key maximum and weight sum by DPP and lane-swap
// exchanges; the weights go through the wavefront's own LDS slots to the
// P.V lanes, which form 64 / (D / 8) key groups of D / 8 lanes, one run each.
// KR bounds the runs a score lane takes (ceil(D / 32)) and the keys a P.V
// lane takes per tile; kPrefetch: the wavefront's next tile is requested
// before the current one is computed (twice the registers, taken for
// KR <= 8).
constexpr int kQsFloats = 1024;  // GP * D of every instantiation
constexpr int kWaveKeys = 16;    // keys per wavefront tile
template <int KR, int GP, bool kPrefetch, bool kQ16, bool kO16>
__global__ __launch_bounds__(kGenThreads) void general_attn_wave_kernel(const GeneralArgs a) {
  static_assert(GP * KR * 32 <= kQsFloats, "query rows of the workgroup's heads fit the LDS");
  __shared__ float qs[kQsFloats];
  __shared__ float ps[kGenWaves][GP][kWaveKeys];
  __shared__ float2 mls[GP][kGenWaves];
  __shared__ float opart[kGenThreads * 8];  // 4 wavefronts x key groups x D <= 2048 floats

  GenWork w;
  if (!general_work(a, w)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int D = a.D, nm = w.nm;

  const int64_t slab = cache_index_d(w.b, 0, w.hk, 0, a.n_kv, a.cap, D);
  const f16* kb = a.k_cache + slab;
  const f16* vb = a.v_cache + slab;
  const int nr = D / 8;                       // runs per row, <= 64
  const int kk = lane >> 2, qq = lane & 3;    // score role: key of the tile, quarter
  const int kgw = 64 / nr;                    // P.V key groups per wavefront, >= 1
  const int kp = (kWaveKeys + kgw - 1) / kgw; // keys per P.V lane, <= KR
  const int kg = lane / nr, u = lane - kg * nr;
  const bool pv_on = kg < kgw;

  // Requests a tile's runs. Every load is unconditional, from an address
  // clamped into the key range and the row (keys past t1 read key t1 - 1,
  // runs past the row its last run): a load whose value is selected against
  // zero makes the compiler wait for it right away, which would serialise
  // the prefetch. The uses below skip every such value.
  f16x8 kn[KR], vn[KR];
  auto request = [&](int ts) {
    const int64_t key = min(ts + kk, w.t1 - 1);
#pragma unroll
    for (int i = 0; i < KR; ++i) {
      const int j = min(qq + 4 * i, nr - 1);
      kn[i] = *reinterpret_cast<const f16x8*>(kb + key * D + j * 8);
    }
#pragma unroll
    for (int i = 0; i < KR; ++i) {
      if (i < kp) {  // uniform
        const int64_t k = min(ts + kg * kp + i, w.t1 - 1);
        vn[i] = *reinterpret_cast<const f16x8*>(vb + k * D + u * 8);
      }
    }
  };

  // The query rows (nm * D <= 1024 values, 4 per thread) are requested
  // first, then the first tile's runs, so that storing the query rows to LDS
  // waits for them alone (loads complete in order).
  float qv[kQsFloats / kGenThreads];
  const int64_t q0 = (int64_t)w.row0 * D;
  const int nq = nm * D;
#pragma unroll
  for (int r = 0; r < kQsFloats / kGenThreads; ++r)
    qv[r] = load_q<kQ16>(a.q, q0 + min(tid + kGenThreads * r, nq - 1));
  const int first = w.t0 + kWaveKeys * wave;
  if (first < w.t1) request(first);
#pragma unroll
  for (int r = 0; r < kQsFloats / kGenThreads; ++r)
    if (tid + kGenThreads * r < nq) qs[tid + kGenThreads * r] = a.c * qv[r];
  __syncthreads();

  float m[GP], l[GP], acc[GP][8];
#pragma unroll
  for (int g = 0; g < GP; ++g) {
    m[g] = kNegBig;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  }

  for (int ts = first; ts < w.t1; ts += kWaveKeys * kGenWaves) {
    f16x8 kc[KR], vc[KR];
    if constexpr (kPrefetch) {
#pragma unroll
      for (int i = 0; i < KR; ++i) {
        kc[i] = kn[i];
        vc[i] = vn[i];
      }
      if (ts + kWaveKeys * kGenWaves < w.t1) request(ts + kWaveKeys * kGenWaves);
    } else {
      if (ts != first) request(ts);
#pragma unroll
      for (int i = 0; i < KR; ++i) {
        kc[i] = kn[i];
        vc[i] = vn[i];
      }
    }
    const bool valid = ts + kk < w.t1;
#pragma unroll
    for (int g = 0; g < GP; ++g) {
      if (g < nm) {
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < KR; ++i) {
          const int j = qq + 4 * i;
          if (j < nr) {
#pragma unroll
            for (int e = 0; e < 8; ++e) dot = fmaf(qs[g * D + j * 8 + e], (float)kc[i][e], dot);
          }
        }
        dot += dpp_mov<kDppQuadXor1>(dot);
        dot += dpp_mov<kDppQuadXor2>(dot);
        const float s = valid ? dot : kNegBig;
        const float m_new = fmaxf(m[g], max_quads(s));
        const float alpha = exp2f(m[g] - m_new);
        const float p = valid ? exp2f(s - m_new) : 0.f;
        l[g] = fmaf(l[g], alpha, sum_quads(p));
        m[g] = m_new;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] *= alpha;
        if (qq == 0) ps[wave][g][kk] = p;
      }
    }
    // The weights were written by this wavefront's own lanes: LDS serves a
    // wavefront's accesses in order, so no barrier is needed.
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int g = 0; g < GP; ++g) {
      if (g < nm) {
#pragma unroll
        for (int i = 0; i < KR; ++i) {
          const int k = kg * kp + i;
          if (pv_on && i < kp && k < kWaveKeys && ts + k < w.t1) {
            const float p = ps[wave][g][k];
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(p, (float)vc[i][e], acc[g][e]);
          }
        }
      }
    }
    __builtin_amdgcn_wave_barrier();  // this tile's reads before the next tile's writes
  }

  // Merge the four wavefronts: per head, M = max m_w, L = sum l_w 2^(m_w - M),
  // and each wavefront's partial outputs scaled by 2^(m_w - M).
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < GP; ++g)
      if (g < nm) mls[g][wave] = make_float2(m[g], l[g]);
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < GP; ++g) {
    if (g < nm) {
      float M = mls[g][0].x;
#pragma unroll
      for (int v = 1; v < kGenWaves; ++v) M = fmaxf(M, mls[g][v].x);
      float L = 0.f;
#pragma unroll
      for (int v = 0; v < kGenWaves; ++v) L = fmaf(mls[g][v].y, exp2f(mls[g][v].x - M), L);
      const float f = exp2f(m[g] - M);
      if (pv_on) {
#pragma unroll
        for (int e = 0; e < 8; ++e) opart[(wave * kgw + kg) * D + u * 8 + e] = acc[g][e] * f;
      }
      finish_row<kO16>(a, w.row0 + g, w.split, M, L, kGenWaves * kgw, opart);
      __syncthreads();  // opart is rewritten for the next head
    }
  }
}

// Any D: single fp16 values. A P.V thread owns dim u of its key group (and
// u + 256 when D > 256, one group).
template <bool kQ16, bool kO16>
__global__ __launch_bounds__(kGenThreads) void general_attn_scalar_kernel(const GeneralArgs a) {
  __shared__ float qs[kMaxHeadDim];
  __shared__ float ps[kGenKeys];
  __shared__ float red_max[kGenWaves], red_sum[kGenWaves];
  __shared__ float opart[kMaxHeadDim];  // groups * D <= max(256, D) floats

  GenWork w;
  if (!general_work(a, w)) return;  // one head per workgroup here (gp = 1)
  const int tid = threadIdx.x;
  const int D = a.D;
  stage_q<kQ16>(a, w.row0, 1, qs);
  __syncthreads();

  const int64_t slab = cache_index_d(w.b, 0, w.hk, 0, a.n_kv, a.cap, D);
  const f16* kb = a.k_cache + slab;
  const f16* vb = a.v_cache + slab;
  const int kk = tid >> 2, qq = tid & 3;
  const int groups = D >= kGenThreads ? 1 : kGenThreads / D;
  const int kg = D >= kGenThreads ? 0 : tid / D;
  const int u = D >= kGenThreads ? tid : tid - kg * D;
  const bool pv_on = kg < groups && u < D;
  const bool second = u + kGenThreads < D;

  float m = kNegBig, l = 0.f, acc = 0.f, acc2 = 0.f;
  for (int ts = w.t0; ts < w.t1; ts += kGenKeys) {
    const int key = ts + kk;
    float dot = 0.f;
    if (key < w.t1) {
      const f16* kr = kb + (int64_t)key * D;
      for (int d = qq; d < D; d += 4) dot = fmaf(qs[d], (float)kr[d], dot);
    }
    dot += __shfl_xor(dot, 1);
    dot += __shfl_xor(dot, 2);
    const float alpha = tile_softmax(dot, key < w.t1, ps, red_max, red_sum, m, l);
    acc *= alpha;
    acc2 *= alpha;
    if (pv_on) {
      const int kend = min(kGenKeys, w.t1 - ts);
      for (int k = kg; k < kend; k += groups) {
        const float p = ps[k];
        const f16* vr = vb + (int64_t)(ts + k) * D;
        acc = fmaf(p, (float)vr[u], acc);
        if (second) acc2 = fmaf(p, (float)vr[u + kGenThreads], acc2);
      }
    }
    __syncthreads();
  }
  if (pv_on) {
    opart[kg * D + u] = acc;
    if (second) opart[u + kGenThreads] = acc2;
  }
  finish_row<kO16>(a, w.row0, w.split, m, l, groups, opart);
}

// One workgroup per row and 32 dims of it: out = sum_s o_s 2^(m_s - M) /
// sum_s l_s 2^(m_s - M), M the largest m_s (split 0 always holds key 0, so M
// is finite; an empty split's record is (kNegBig, 0, 0) and weighs nothing).
// The 256 threads are 8 split groups of 32 dims; each thread requests 16
// records' values before adding them (one batch up to 128 splits), so the
// record reads overlap instead of costing a round trip per split, and the
// split groups' sums are added through LDS.
constexpr int kMergeBatch = 16;
constexpr int kMergeDims = 32;
constexpr int kMergeGroups = kGenThreads / kMergeDims;
template <bool kO16>
__global__ __launch_bounds__(kGenThreads) void general_merge_kernel(const GeneralArgs a) {
  __shared__ float wts[kGenThreads];
  __shared__ float red_max[kGenWaves], red_sum[kGenWaves];
  __shared__ float part[kMergeGroups][kMergeDims];
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t r0 = (int64_t)row * a.nsplit;
  float2 ml = make_float2(kNegBig, 0.f);
  if (tid < a.nsplit && in_bounds(r0 + tid, 1, a.records, a.status)) ml = a.part_ml[r0 + tid];
  const float wm = wave_max(ml.x);
  if (lane == 0) red_max[wave] = wm;
  __syncthreads();
  float M = red_max[0];
#pragma unroll
  for (int w = 1; w < kGenWaves; ++w) M = fmaxf(M, red_max[w]);
  const float wt = tid < a.nsplit ? exp2f(ml.x - M) : 0.f;
  wts[tid] = wt;
  const float ws = wave_sum(ml.y * wt);
  if (lane == 0) red_sum[wave] = ws;
  __syncthreads();
  float Lsum = 0.f;
#pragma unroll
  for (int w = 0; w < kGenWaves; ++w) Lsum += red_sum[w];

  const int D = a.D;
  const int sg = tid / kMergeDims, dl = tid - sg * kMergeDims;
  const int d = blockIdx.y * kMergeDims + dl;
  float o = 0.f;
  if (d < D) {
    for (int s0 = sg; s0 < a.nsplit; s0 += kMergeGroups * kMergeBatch) {
      float v[kMergeBatch];
#pragma unroll
      for (int i = 0; i < kMergeBatch; ++i) {
        const int sp = s0 + kMergeGroups * i;
        const int64_t at = (r0 + sp) * D + d;
        v[i] = sp < a.nsplit && in_bounds(at, 1, a.records * D, a.status) ? a.part_o[at] : 0.f;
      }
#pragma unroll
      for (int i = 0; i < kMergeBatch; ++i) {
        const int sp = s0 + kMergeGroups * i;
        o = fmaf(v[i], sp < a.nsplit ? wts[sp] : 0.f, o);
      }
    }
  }
  part[sg][dl] = o;
  __syncthreads();
  if (tid < kMergeDims && d < D) {
    float t = 0.f;
#pragma unroll
    for (int g = 0; g < kMergeGroups; ++g) t += part[g][tid];
    const int64_t oi = (int64_t)row * D + d;
    if (in_bounds(oi, 1, (int64_t)gridDim.x * D, a.status)) store_o<kO16>(a.out, oi, t / Lsum);
  }
}

template <typename K>
static hipError_t launch_attn(K kernel, const GeneralArgs& a, hipStream_t stream, void* ev_start,
                              void* ev_stop) {
  const int lanes = (a.total + kXcds - 1) / kXcds * kXcds;  // whole XCD ranges
  GeneralArgs arg = a;
  void* args[] = {&arg};
  if (ev_start || ev_stop)  // measurement: events at the kernel's start and end
    return hipExtLaunchKernel(reinterpret_cast<const void*>(kernel), dim3((unsigned)lanes),
                              dim3(kGenThreads), args, 0, stream, (hipEvent_t)ev_start,
                              (hipEvent_t)ev_stop, 0);
  return hipLaunchKernel(reinterpret_cast<const void*>(kernel), dim3((unsigned)lanes),
                         dim3(kGenThreads), args, 0, stream);
}

// The vector kernel instantiated for the smallest power of two of heads per
// workgroup that holds a.gp (the accumulators of unused heads would still
// take registers, and occupancy).
template <int KR, bool kPf, bool kQ16, bool kO16>
static hipError_t launch_vec(const GeneralArgs& a, hipStream_t stream, void* ev_start,
                             void* ev_stop) {
  if (a.gp <= 1) return launch_attn(general_attn_wave_kernel<KR, 1, kPf, kQ16, kO16>, a, stream, ev_start, ev_stop);
  if (a.gp <= 2) return launch_attn(general_attn_wave_kernel<KR, 2, kPf, kQ16, kO16>, a, stream, ev_start, ev_stop);
  if constexpr (KR <= 8) {
    if (a.gp <= 4) return launch_attn(general_attn_wave_kernel<KR, 4, kPf, kQ16, kO16>, a, stream, ev_start, ev_stop);
  }
  if constexpr (KR <= 4) {
    if (a.gp <= 8) return launch_attn(general_attn_wave_kernel<KR, 8, kPf, kQ16, kO16>, a, stream, ev_start, ev_stop);
  }
  return hipErrorInvalidValue;
}

template <bool kQ16, bool kO16>
static hipError_t launch_general_t(const GeneralArgs& a, int rows, hipStream_t stream,
                                   void* ev_start, void* ev_stop) {
  hipError_t e;
  if (a.D % 8 != 0) {
    e = launch_attn(general_attn_scalar_kernel<kQ16, kO16>, a, stream, ev_start, ev_stop);
  } else {
    switch (general_runs_bucket(a.D)) {
      case 1: e = launch_vec<1, true, kQ16, kO16>(a, stream, ev_start, ev_stop); break;
      case 2: e = launch_vec<2, true, kQ16, kO16>(a, stream, ev_start, ev_stop); break;
      case 4: e = launch_vec<4, true, kQ16, kO16>(a, stream, ev_start, ev_stop); break;
      case 8: e = launch_vec<8, true, kQ16, kO16>(a, stream, ev_start, ev_stop); break;
      default: e = launch_vec<16, false, kQ16, kO16>(a, stream, ev_start, ev_stop); break;
    }
  }
  if (e != hipSuccess || a.nsplit == 1) return e;
  general_merge_kernel<kO16><<<dim3((unsigned)rows, (unsigned)((a.D + kMergeDims - 1) / kMergeDims)),
                                 kGenThreads, 0, stream>>>(a);
  return hipGetLastError();
}

int general_split_keys(int span, int nsplit) {
  const int per = (span + nsplit - 1) / nsplit;
  return (per + kGenKeys - 1) / kGenKeys * kGenKeys;
}

hipError_t launch_general_attn(const Shape& s, const void* q, const void* k_cache,
                               const void* v_cache, const int32_t* pos, void* out, int batch,
                               int n_new, int prefill, int span, int nsplit, const Workspace& ws,
                               void* ev_start, void* ev_stop, hipStream_t stream) {
  const int64_t rows = (int64_t)batch * n_new * s.n_heads;
  const int gp = general_heads_per_workgroup(s.head_dim, s.group);
  const int chunks = (s.group + gp - 1) / gp;
  const int64_t total = (int64_t)batch * n_new * s.n_kv * chunks * nsplit;
  if (rows < 1 || nsplit < 1 || nsplit > kGenThreads || rows * nsplit > 0x7FFFFFF0 ||
      total > 0x7FFFFFF0 || s.head_dim < 1 || s.head_dim > kMaxHeadDim || span < 1)
    return hipErrorInvalidValue;
  if (nsplit > 1 && rows * nsplit > ws.records) return hipErrorInvalidValue;
  GeneralArgs a;
  a.q = q;
  a.k_cache = static_cast<const f16*>(k_cache);
  a.v_cache = static_cast<const f16*>(v_cache);
  a.pos = pos;
  a.out = out;
  a.part_o = ws.part_o;
  a.part_ml = ws.part_ml;
  a.records = ws.records;
  a.D = s.head_dim;
  a.n_heads = s.n_heads;
  a.n_kv = s.n_kv;
  a.group = s.group;
  a.cap = s.cap;
  a.n_new = n_new;
  a.nsplit = nsplit;
  a.prefill = prefill;
  a.split_keys = general_split_keys(span, nsplit);
  a.gp = gp;
  a.chunks = chunks;
  a.rows = (int)rows;
  a.total = (int)total;
  a.c = s.qk_scale * kLog2e;
  a.status = ws.status;
  if (s.q16)
    return s.o16 ? launch_general_t<true, true>(a, (int)rows, stream, ev_start, ev_stop)
                 : launch_general_t<true, false>(a, (int)rows, stream, ev_start, ev_stop);
  return s.o16 ? launch_general_t<false, true>(a, (int)rows, stream, ev_start, ev_stop)
               : launch_general_t<false, false>(a, (int)rows, stream, ev_start, ev_stop);
}

}  // namespace nwd
