// nwd_decode.h — the split workgroup of decode (decode_split_kernel), its
// state store and merges, and their launchers, shared by nwd_decode.hip
// (head size 128), nwd_decode_groups.hip (groups 3, 6, 7 at 128 and 64) and
// nwd_decode_hd.hip (the other head sizes), which instantiate disjoint sets
// of them; the matrix-core kernel is in nwd_decode_mfma.h.
#pragma once

#include <hip/hip_ext.h>

#include <type_traits>

#include "nwd_common.h"
#include "nwd_internal.h"

namespace nwd {


// Shape of one split workgroup: kW wavefronts, rows of kL lanes per key,
// kKpr keys per row per iteration, kT iterations' tiles in flight, head size
// kD (64, 128 or 256).
template <int kW, int kL, int kKpr_, int kT, int kD_>
struct DecodeShape {
  static constexpr int kD = kD_;
  static constexpr int kTiles = kT;
  static constexpr int kWaves = kW;
  static constexpr int kThreads = kW * 64;
  static constexpr int kLanes = kL;               // lanes per key row
  static constexpr int kRows = 64 / kL;           // key rows per wavefront
  static constexpr int kRuns = kD / 8 / kL;       // 16-byte runs per lane per key
  static constexpr int kDims = 8 * kRuns;         // dims per lane
  static constexpr int kKpr = kKpr_;              // keys per row per iteration
  static constexpr int kWaveKeys = kRows * kKpr;  // keys per wavefront per iteration
  static constexpr int kBlockKeys = kW * kWaveKeys;
  static_assert(kL == 8 || kL == 16, "rows of 8 or 16 lanes");
  static_assert(kD % (8 * kL) == 0, "whole 16-byte runs per lane");
  static constexpr bool kPadD = false;
};
// The same workgroup for rows of fewer dims (a multiple of 8 below kD, the
// call's head_dim): the 16-byte runs past a row's dims load as zeros (their
// offsets pushed past the buffer range) and are not stored, so the scores
// and outputs are those of the real dims; records keep kD dims.
template <int kW, int kL, int kKpr_, int kT, int kD_>
struct DecodePadShape : DecodeShape<kW, kL, kKpr_, kT, kD_> {
  static constexpr bool kPadD = true;
};
// The head-128 form.
template <int kW, int kL, int kKpr_, int kT>
struct DecodeCfg : DecodeShape<kW, kL, kKpr_, kT, kHeadDim> {};

// Units the key range is split in (16 keys, one matrix-core wavefront
// block, two dot-product wavefront tiles). Each split's time is that of its
// keys (a workgroup streams at the rate its own loads in flight allow), so
// the slowest split sets the launch's time: small units keep the splits
// within 16 keys of each other (4160 keys over 32 splits: 128-144 each,
// where 128-key units gave one split 256).
constexpr int kUnitKeys = 16;
// How far (log2 units) a score may exceed the online softmax's reference
// point before the reference moves (and the accumulators are rescaled).
constexpr float kRescaleSlack = 8.f;

// Sum over each aligned group of N lanes (N = 8 or 16); every lane of the
// group gets it.
template <int N>
__device__ inline float sum_lanes(float x) {
  x += dpp_mov<kDppQuadXor1>(x);
  x += dpp_mov<kDppQuadXor2>(x);
  x += dpp_mov<kDppHalfMirror>(x);
  if constexpr (N == 16) x += dpp_mov<kDppRowMirror>(x);
  return x;
}

// Max / sum of the lanes holding the same dims in every row of a wavefront
// (rows of N lanes: lanes l, l ^ N, ... up to l ^ 32).
template <int N>
__device__ inline float max_rows(float x) {
  if constexpr (N == 8) x = fmaxf(x, dpp_mov<kDppRowRor8>(x));
  return max_xor32(max_xor16(x));
}
template <int N>
__device__ inline float sum_rows(float x) {
  if constexpr (N == 8) x += dpp_mov<kDppRowRor8>(x);
  return sum_xor32(sum_xor16(x));
}

// Max / sum with the lane holding the same dims in another row: step 0
// pairs lane l with l ^ 32, step 1 with l ^ 16, step 2 with l ^ 8.
__device__ inline float row_pair_max(float x, int step) {
  if (step == 0) return max_xor32(x);
  if (step == 1) return max_xor16(x);
  return fmaxf(x, dpp_mov<kDppRowRor8>(x));
}
__device__ inline float row_pair_sum(float x, int step) {
  if (step == 0) return sum_xor32(x);
  if (step == 1) return sum_xor16(x);
  return x + dpp_mov<kDppRowRor8>(x);
}

// One 16-byte run (8 values) of a new K/V row, fp16 or fp32, loaded as raw
// words (fp16: the first 16 bytes) and converted later, so that the load
// can be issued early and nothing waits for it until the values are used.
struct SrcRun {
  f32x4 w[2];
};
__device__ inline SrcRun load_src_run_raw(const void* src, int64_t elem, bool src16) {
  SrcRun r;
  if (src16) {
    r.w[0] = *reinterpret_cast<const f32x4*>(static_cast<const f16*>(src) + elem);
    r.w[1] = f32x4{0.f, 0.f, 0.f, 0.f};  // unused; no copy of w[0], which would wait for it
  } else {
    const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(src) + elem);
    r.w[0] = p[0];
    r.w[1] = p[1];
  }
  return r;
}
// fp16 runs are bit copies; fp32 runs are rounded to nearest even, as
// kv_append does.
__device__ inline f16x8 convert_src_run(const SrcRun& r, bool src16) {
  if (src16) return __builtin_bit_cast(f16x8, r.w[0]);
  f16x8 h;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    h[e] = (f16)r.w[0][e];
    h[4 + e] = (f16)r.w[1][e];
  }
  return h;
}

// s_waitcnt vmcnt(0): every earlier global access of this thread is complete.
__device__ inline void wait_vm() { __builtin_amdgcn_s_waitcnt(0x0F70); }


// Splits one merge pass reads: all of a pass's loads are issued together, one
// memory round trip (one pass for the usual 32 splits or fewer).
constexpr int kMergePass = 32;

// Merges the nsplit records (m, l, o[D]) of one output row (b * n_heads +
// head) and writes the normalised row; run by one whole wavefront. Lane l
// owns dims 2l and 2l+1; per pass of up to 32 splits, lane s holds split
// s's (m, l), every o record of the pass is requested at once (32 coalesced
// 8-byte loads per lane), the pass maximum Mp is a wavefront reduction, the
// running maximum M is raised to max(M, Mp) with the running sums rescaled,
// and the splits' weights 2^(m_s - M) reach every lane by readlane, so
// each lane adds its dims split by split in order with no LDS and no
// barrier. Both merge forms call it, so they give the same bits. (Against
// the earlier 256-thread merge, which combined eight thread groups' partial
// sums through LDS, per call: 32K keys 24.5 against 24.9-25.0 us, 4K 8.6
// against 9.0, 40q/8kv at 32K 24.7 against 25.1.)
// The same for head sizes other than 128 (kD / 64 dims per lane, one
// 4-, 8- or 16-byte load per split and lane).
template <bool kO16, int kPolicy, int kD, bool kPadD>
__device__ inline void merge_row_wave_d(const float* __restrict__ part_o,
                                        const float2* __restrict__ part_ml, void* __restrict__ out,
                                        int64_t row, int nsplit, int64_t out_rows, int64_t records,
                                        int* status, int od) {
  constexpr int kDL = kD / 64;  // dims per lane
  static_assert(kDL == 1 || kDL == 4, "head size 64 or 256");
  const int lane = threadIdx.x & 63;
  const int64_t rec0 = row * nsplit;
  if (!in_bounds(rec0, nsplit, records, status)) return;
  const auto r_ml = __builtin_amdgcn_make_buffer_rsrc(const_cast<float2*>(part_ml + rec0), 0,
                                                      nsplit * 8, kBufferWord3);
  const auto r_o = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(part_o + rec0 * kD), 0,
                                                     nsplit * kD * 4, kBufferWord3);
  float M = kNegBig, L = 0.f, acc[kDL];
#pragma unroll
  for (int i = 0; i < kDL; ++i) acc[i] = 0.f;
  for (int s0 = 0; s0 < nsplit; s0 += kMergePass) {
    const int ns = min(kMergePass, nsplit - s0);
    const float2 ml = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(
        r_ml, (s0 + min(lane, ns - 1)) * 8, 0, kPolicy));
    float ov[kMergePass][kDL];
#pragma unroll
    for (int s = 0; s < kMergePass; ++s) {
      const uint32_t off = ((s0 + min(s, ns - 1)) * kD + kDL * lane) * 4;
      if constexpr (kDL == 1) {
        ov[s][0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r_o, off, 0, kPolicy));
      } else {
        const f32x4 v = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r_o, off, 0, kPolicy));
#pragma unroll
        for (int i = 0; i < 4; ++i) ov[s][i] = v[i];
      }
    }
    const float m = lane < ns ? ml.x : kNegBig;
    const float mn = fmaxf(M, max_xor32(max32(m)));
    const float w = lane < ns ? fast_exp2(m - mn) : 0.f;
    const float alpha = fast_exp2(M - mn);
    L = fmaf(L, alpha, sum64(ml.y * w));
#pragma unroll
    for (int i = 0; i < kDL; ++i) acc[i] *= alpha;
#pragma unroll
    for (int s = 0; s < kMergePass; ++s) {
      const float ws = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), s));
#pragma unroll
      for (int i = 0; i < kDL; ++i) acc[i] = fmaf(ov[s][i], ws, acc[i]);
    }
    M = mn;
  }
  const float inv = 1.f / L;
  if (kPadD && kDL * lane >= od) return;  // padded dims
  const int64_t at = row * od + kDL * lane;
  if (!in_bounds(at, kDL, out_rows * od, status)) return;
#pragma unroll
  for (int i = 0; i < kDL; ++i) {
    if constexpr (kO16) static_cast<f16*>(out)[at + i] = (f16)(acc[i] * inv);
    else static_cast<float*>(out)[at + i] = acc[i] * inv;
  }
}

// od: the output rows' width (kD, or the padded form's head_dim).
template <bool kO16, int kPolicy, int kD = kHeadDim, bool kPadD = false>
__device__ inline void merge_row_wave(const float* __restrict__ part_o,
                                      const float2* __restrict__ part_ml, void* __restrict__ out,
                                      int64_t row, int nsplit, int64_t out_rows, int64_t records,
                                      int* status, int od = kD) {
  if constexpr (kD != kHeadDim) {
    merge_row_wave_d<kO16, kPolicy, kD, kPadD>(part_o, part_ml, out, row, nsplit, out_rows,
                                                records, status, od);
    return;
  }
  const int lane = threadIdx.x & 63;
  const int64_t rec0 = row * nsplit;
  // uniform over the wavefront
  if (!in_bounds(rec0, nsplit, records, status)) return;
  const auto r_ml = __builtin_amdgcn_make_buffer_rsrc(const_cast<float2*>(part_ml + rec0), 0,
                                                      nsplit * 8, kBufferWord3);
  const auto r_o = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(part_o + rec0 * kHeadDim), 0,
                                                     nsplit * kHeadDim * 4, kBufferWord3);
  float M = kNegBig, L = 0.f, a0 = 0.f, a1 = 0.f;
  for (int s0 = 0; s0 < nsplit; s0 += kMergePass) {
    const int ns = min(kMergePass, nsplit - s0);
    // loads (indexes clamped in range; splits past the pass get no weight)
    const float2 ml = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(
        r_ml, (s0 + min(lane, ns - 1)) * 8, 0, kPolicy));
    float2 ov[kMergePass];
#pragma unroll
    for (int s = 0; s < kMergePass; ++s)
      ov[s] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(
          r_o, ((s0 + min(s, ns - 1)) * kHeadDim + 2 * lane) * 4, 0, kPolicy));
    const float m = lane < ns ? ml.x : kNegBig;
    const float mn = fmaxf(M, max_xor32(max32(m)));
    const float w = lane < ns ? fast_exp2(m - mn) : 0.f;
    const float alpha = fast_exp2(M - mn);
    L = fmaf(L, alpha, sum64(ml.y * w));
    a0 *= alpha;
    a1 *= alpha;
#pragma unroll
    for (int s = 0; s < kMergePass; ++s) {
      const float ws = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), s));
      a0 = fmaf(ov[s].x, ws, a0);
      a1 = fmaf(ov[s].y, ws, a1);
    }
    M = mn;
  }
  const float inv = 1.f / L;
  if (kPadD && 2 * lane >= od) return;  // padded dims
  const int64_t at = row * od + 2 * lane;
  if (!in_bounds(at, 2, out_rows * od, status)) return;
  if constexpr (kO16) {
    f16x2 v;
    v[0] = (f16)(a0 * inv);
    v[1] = (f16)(a1 * inv);
    *reinterpret_cast<f16x2*>(static_cast<f16*>(out) + at) = v;
  } else {
    *reinterpret_cast<float2*>(static_cast<float*>(out) + at) = make_float2(a0 * inv, a1 * inv);
  }
}

struct DecodeArgs {
  const void* q;
  f16* k_cache;  // written only at the fused-append row
  f16* v_cache;
  const int32_t* pos;
  void* out;
  float* part_o;
  float2* part_ml;
  int64_t records;    // capacity of part_o / part_ml in records
  const void* k_new;  // optional new rows [batch][n_kv][D] (fused append)
  const void* v_new;
  int new16;          // new rows are fp16 (else fp32)
  int* counters;      // [batch][n_kv] arrival tickets (the grid's n_kv), zero between calls
  int batch, n_heads, n_kv, cap, nsplit;
  int span;           // host bound on L: keys [0, span) are partitioned
  int strided;        // key layout over the splits: 0 contiguous ranges, 1 interleaved blocks
  int fused_merge;    // merge in the split kernel's last workgroup
  float qk_scale_log2;
  int* status;
  int head_dim;       // D of the rows in memory (a DecodePadShape kernel's; kD otherwise)
  // Groups of G query heads per KV head: the grid's KV index runs over
  // n_kv = KV heads x kv_rep such groups, and group j reads KV head
  // j / kv_rep (1: one group per KV head).
  int kv_rep;
};

// Record stores of the in-kernel merge write through to memory (agent
// coherence, cache policy sc1), so the merging workgroup can read them on
// any XCD without an L2 write-back.
constexpr int kRecPolicy = 16;

// The end of a split workgroup, shared by both loop forms: merges the
// kStates partial states its wavefronts left in LDS (lds_o [kStates][G][D]
// and lds_ml [kStates][G][2], (m, l) in log2 units) into one record per
// query head, or, with one split, the normalised output. Called by every
// thread after a barrier; thread t < 32 G owns the kD / 32-dim run t % 32
// of head t / 32. hrow0 = b * n_heads + first head.
template <int kN>
using f32xn = float __attribute__((ext_vector_type(kN)));
template <int kN>
using f16xn = f16 __attribute__((ext_vector_type(kN)));
template <int G, bool kO16, int kStates, int kD = kHeadDim, bool kPadD = false>
__device__ inline void store_split_states(const DecodeArgs& a, const float* lds_o,
                                          const float* lds_ml, int64_t hrow0, int split,
                                          int od = kD) {
  constexpr int kR = kD / 32;  // dims per thread: 2, 4 or 8
  static_assert(kR == 2 || kR == 4 || kR == 8, "head size 64, 128 or 256");
  using vec = f32xn<kR>;
  const int tid = threadIdx.x;
  const int nsplit = a.nsplit;
  if (tid < G * 32) {
    const int g = tid >> 5, d4 = tid & 31;
    float M = kNegBig;
#pragma unroll
    for (int w = 0; w < kStates; ++w) M = fmaxf(M, lds_ml[(w * G + g) * 2]);
    vec o = vec(0.f);
    float lt = 0.f;
#pragma unroll
    for (int w = 0; w < kStates; ++w) {
      const float sc = fast_exp2(lds_ml[(w * G + g) * 2] - M);
      o += *reinterpret_cast<const vec*>(&lds_o[(w * G + g) * kD + d4 * kR]) * sc;
      lt = fmaf(lds_ml[(w * G + g) * 2 + 1], sc, lt);
    }
    const int64_t out_rows = (int64_t)a.batch * a.n_heads;
    if (nsplit == 1) {
      const float inv = 1.f / lt;
      const int64_t at = (hrow0 + g) * od + d4 * kR;
      if (kPadD && d4 * kR >= od) {
        // a padded run: nothing to store
      } else if (!in_bounds(at, kR, out_rows * od, a.status)) {
        // (bounds-checked builds only) the store is dropped
      } else if constexpr (kO16) {
        f16xn<kR> v;
#pragma unroll
        for (int i = 0; i < kR; ++i) v[i] = (f16)(o[i] * inv);
        *reinterpret_cast<f16xn<kR>*>(static_cast<f16*>(a.out) + at) = v;
      } else {
        *reinterpret_cast<vec*>(static_cast<float*>(a.out) + at) = o * inv;
      }
    } else {
      // records of this split: (g, split) at hrow0 * nsplit + g * nsplit + split
      const int64_t rec0 = hrow0 * nsplit + split;
      // the descriptors below stop stores past this head group's records;
      // head g's nsplit records must lie inside the workspace
      const bool rec_ok = in_bounds((hrow0 + g) * nsplit, nsplit, a.records, a.status);
      const auto r_o = __builtin_amdgcn_make_buffer_rsrc(a.part_o + rec0 * kD, 0,
                                                         G * nsplit * kD * 4, kBufferWord3);
      const auto r_ml = __builtin_amdgcn_make_buffer_rsrc(a.part_ml + rec0, 0, G * nsplit * 8,
                                                          kBufferWord3);
      const uint32_t off = (g * nsplit * kD + d4 * kR) * 4;
      // the o run as 8- or 16-byte stores with the given cache policy
      auto store_o = [&](auto policy) {
        if constexpr (kR == 2) {
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, o), r_o, off, 0,
                                                decltype(policy)::value);
        } else if constexpr (kR == 4) {
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), r_o, off, 0,
                                                 decltype(policy)::value);
        } else {
          // (the halves copied element by element: a bit cast of o.hi compiled to
          // o.lo's registers)
          const f32x4 lo = {o[0], o[1], o[2], o[3]}, hi = {o[4], o[5], o[6], o[7]};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, lo), r_o, off, 0,
                                                 decltype(policy)::value);
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, hi), r_o, off + 16,
                                                 0, decltype(policy)::value);
        }
      };
      if (!rec_ok) {
        // (bounds-checked builds only) the stores are dropped
      } else if (a.fused_merge) {
        store_o(std::integral_constant<int, kRecPolicy>{});
        if (d4 == 0)
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, make_float2(M, lt)), r_ml,
                                                g * nsplit * 8, 0, kRecPolicy);
      } else {
        store_o(std::integral_constant<int, 0>{});
        if (d4 == 0)
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, make_float2(M, lt)), r_ml,
                                                g * nsplit * 8, 0, 0);
      }
    }
  }
}

// In-kernel merge (nwd_set_decode_merge): the workgroup that takes the last
// arrival ticket of its (b, head group) merges the group's records. One
// counter per (b, head group): per (b, hkv), or per (b, query head) in the
// per-query-head form, where batch x n_heads fits the counters (the host
// keeps at least kSubSplitMaxWorkgroups of them).
//
// Ordering (the AMDGPU memory model for gfx942-family targets, which gfx950
// follows): an agent-scope release is "write back dirty L2 lines, wait for
// the stores", an agent-scope acquire is "agent-scope load, then invalidate
// L2". The records are the only data handed over, and they are stored and
// loaded with the agent-scope cache policy sc1 itself, so they leave no
// dirty L2 line behind and no stale L2 line can serve them: the release
// reduces to waiting for this thread's record stores (vmcnt(0)) before the
// barrier that precedes the ticket, and the acquire to the sc1 loads in
// merge_row_wave, which are issued only after the ticket has returned (they
// depend on it through lds_last). Wavefront w merges heads w, w + waves, ...
template <int G, bool kO16, int kD = kHeadDim, bool kPadD = false>
__device__ inline void merge_on_last_arrival(const DecodeArgs& a, int* counter, int64_t hrow0) {
  __shared__ int lds_last;
  wait_vm();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int ticket = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    lds_last = ticket == a.nsplit - 1;
  }
  __syncthreads();
  if (!lds_last) return;
  for (int g = (int)threadIdx.x >> 6; g < G; g += (int)blockDim.x >> 6)
    merge_row_wave<kO16, kRecPolicy, kD, kPadD>(a.part_o, a.part_ml, a.out, hrow0 + g, a.nsplit,
                                                (int64_t)a.batch * a.n_heads, a.records, a.status,
                                                kPadD ? a.head_dim : kD);
  if (threadIdx.x == 0)
    __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Lane-exchange steps that merge a wavefront's row states in registers
// before they go to LDS: the fewest (up to log2 rows) that bring `bytes`,
// the LDS the unmerged states would take, under 48 KB.
constexpr int row_steps(int bytes, int rows) {
  int st = 0;
  while ((1 << st) < rows && (bytes >> st) > 48 * 1024) ++st;
  return st;
}

// kQsub workgroups per KV head, each serving G of its query heads (kQsub = 1:
// one workgroup serves the whole group).
template <int G, bool kQ16, bool kO16, int kQsub, class C>
__global__ __launch_bounds__(C::kThreads) void decode_split_kernel(const DecodeArgs a) {
  constexpr int kWaves = C::kWaves, kThreads = C::kThreads;
  constexpr int kLanes = C::kLanes, kRows = C::kRows, kRuns = C::kRuns, kDims = C::kDims;
  constexpr int kKpr = C::kKpr, kBlockKeys = C::kBlockKeys, kWaveKeys = C::kWaveKeys;
  constexpr int kTiles = C::kTiles;
  constexpr int kD = C::kD;
  constexpr bool kPadD = C::kPadD;
  // Row width in memory: kD, or the call's head size in the padded form.
  const int Dm = kPadD ? a.head_dim : kD;
  static_assert(G * 32 <= kThreads, "one run of each head per thread");
  // Row states written to LDS per wavefront (see the end of the kernel). The
  // rule depends on the shape's group size, not on the heads this
  // workgroup serves, so both forms of a shape merge in the same order (same
  // bits).
  constexpr int kRowSteps = row_steps(G * kQsub * kWaves * kRows * (kD + 2) * 4, kRows);
  constexpr int kRowStates = kRows >> kRowSteps;
  constexpr int kStates = kWaves * kRowStates;
  constexpr int kLdsFloats = kStates * G * (kD + 2);
  static_assert(kLdsFloats * 4 <= 64 * 1024, "static LDS of one workgroup");

  __shared__ __attribute__((aligned(16))) float lds[kLdsFloats];
  float* lds_o = lds;                                 // [kStates][G][D]
  float* lds_ml = lds + kStates * G * kD;        // [kStates][G][2]

  // Workgroups are dealt to the 8 XCDs round-robin in launch order, so the
  // XCD of a workgroup follows blockIdx.x. Rotating each sequence's splits
  // by b mod 8 spreads every split index over all XCDs: unrotated, with 8
  // splits XCD s got split s of every sequence, and on a ragged batch the
  // first splits hold keys of every sequence while the last ones hold
  // almost none (64 sequences of 512-16384 keys: 511 against 453 us per
  // step).
  // In the per-query-head form the KV head is the fast grid index
  // (blockIdx.y = sub * n_kv + hkv), so with 8 KV heads the kQsub
  // workgroups that read the same K/V rows land on the same XCD and its L2
  // serves their repeated reads (153 keys: 2.65 MB of HBM reads per call
  // with them on different XCDs, for 0.63 MB of K/V).
  const int b = blockIdx.z;
  const int hkv = kQsub > 1 ? (int)blockIdx.y % a.n_kv : (int)blockIdx.y;
  const int sub = kQsub > 1 ? (int)blockIdx.y / a.n_kv : 0;
  const int hgrp = hkv * kQsub + sub;  // this workgroup's group of G query heads
  // The KV head this group reads, and the KV heads in memory.
  const int kv_m = a.kv_rep > 1 ? hkv / a.kv_rep : hkv;
  const int nkv_m = a.kv_rep > 1 ? a.n_kv / a.kv_rep : a.n_kv;
  int split = blockIdx.x + (b & 7);
  while (split >= a.nsplit) split -= a.nsplit;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int row = lane / kLanes, col = lane % kLanes;

  const int nsplit = a.nsplit;
  // This split's keys (independent of the device position): iteration it
  // covers keys t0 + it * it_keys .. + kBlockKeys. Contiguous layout: the
  // split owns one range of whole units of the host bound, spread evenly over
  // the splits. Strided layout: it owns the kBlockKeys blocks split,
  // split + nsplit, ..., so at any moment the splits of a KV head read
  // neighbouring blocks of its slab.
  const int units = (a.span + kUnitKeys - 1) / kUnitKeys;
  const int u0 = (int)((int64_t)split * units / nsplit);
  const int u1 = (int)((int64_t)(split + 1) * units / nsplit);
  const int t0 = a.strided ? split * kBlockKeys : u0 * kUnitKeys;
  const int it_keys = a.strided ? nsplit * kBlockKeys : kBlockKeys;
  const int t1h = min(a.span, u1 * kUnitKeys);

  const int64_t slab = (int64_t)(b * nkv_m + kv_m) * a.cap * Dm;
  // K/V are read through buffer descriptors over the slab that end at the
  // last key a load may need: a load at or past the end fails the hardware
  // range check and returns zeros without a memory access. So the prefetch
  // past the last tile (unconditional, to keep the compiler's wait counts
  // exact) costs no memory round trip for the waits that follow the loop.
  auto slab_rsrc = [&](f16* cache, int end_key) {
    return __builtin_amdgcn_make_buffer_rsrc(cache + slab, 0, end_key * (Dm * 2),
                                             kBufferWord3);
  };

  // Byte offset of this lane's run i of a row at `off`; a padded run's is
  // pushed past the buffer range (the load returns zeros).
  auto run_off = [&](uint32_t off, int i) -> uint32_t {
    const uint32_t o = off + i * kLanes * 16;
    if constexpr (kPadD) return (col + i * kLanes) * 8 >= Dm ? o | 0x80000000u : o;
    return o;
  };
  // Whether this lane's run i holds dims of the row (always, unpadded).
  auto run_real = [&](int i) { return !kPadD || (col + i * kLanes) * 8 < Dm; };

  struct Tile {
    f16x8 k[kKpr][kRuns], v[kKpr][kRuns];
  };

  // Loads never wait for the position: keys past L are loaded (or read as
  // zeros past the descriptor's end) and masked.
  auto load_tile = [&](Tile& tl, const __amdgpu_buffer_rsrc_t rk,
                       const __amdgpu_buffer_rsrc_t rv, int it) {
    const int base = t0 + it * it_keys + wave * kWaveKeys + row;
#pragma unroll
    for (int j = 0; j < kKpr; ++j) {
      const uint32_t off = (uint32_t)(base + j * kRows) * (Dm * 2) + col * 16;
#pragma unroll
      for (int i = 0; i < kRuns; ++i) {
        tl.k[j][i] = __builtin_bit_cast(
            f16x8, __builtin_amdgcn_raw_buffer_load_b128(rk, run_off(off, i), 0, kStreamPolicy));
        tl.v[j][i] = __builtin_bit_cast(
            f16x8, __builtin_amdgcn_raw_buffer_load_b128(rv, run_off(off, i), 0, kStreamPolicy));
      }
    }
  };

  // Fused append: every workgroup requests the new rows (this lane's runs,
  // raw) before its first tile, and before the position says which split
  // owns them, so that converting them later never waits for a tile.
  const bool has_new = a.k_new != nullptr;
  SrcRun nk_raw[kRuns], nv_raw[kRuns];
  if (has_new) {
#pragma unroll
    for (int i = 0; i < kRuns; ++i) {
      const int64_t src = (int64_t)(b * nkv_m + kv_m) * Dm + (col + i * kLanes) * 8;
      if (!run_real(i)) {
        nk_raw[i] = nv_raw[i] = SrcRun{{f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}}};
        continue;
      }
      nk_raw[i] = load_src_run_raw(a.k_new, src, a.new16);
      nv_raw[i] = load_src_run_raw(a.v_new, src, a.new16);
    }
  }

  // The first kTiles - 1 tiles are requested before the position is known,
  // over the keys this split can own: up to the host bound, or up to the
  // capacity for the last split (which absorbs keys past the bound). They may
  // therefore hold cache rows at or past L, which the reference never reads;
  // their V runs are zeroed before use (a stale Inf or NaN times a zero
  // weight would be NaN). Later tiles are bounded by the split's last key.
  Tile tr[kTiles];
  {
    const int own_end = a.strided || split == nsplit - 1 ? a.cap : t1h;
    const auto ek = slab_rsrc(a.k_cache, own_end), ev = slab_rsrc(a.v_cache, own_end);
#pragma unroll
    for (int t = 0; t < kTiles - 1; ++t) load_tile(tr[t], ek, ev, t);
  }

  // Query registers: this lane's dims of each of the G heads.
  const int h0 = hgrp * G;
  const int64_t qoff = ((int64_t)b * a.n_heads + h0) * Dm + col * 8;
  f16x8 q16[kQ16 ? G : 1][kRuns];
  float q32[kQ16 ? 1 : G][kDims];
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int i = 0; i < kRuns; ++i) {
      const int64_t e = qoff + g * Dm + i * kLanes * 8;
      if (!run_real(i)) {  // a padded run: zero query dims
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          if constexpr (kQ16) q16[g][i][k] = (f16)0.f;
          else q32[g][i * 8 + k] = 0.f;
        }
        continue;
      }
      if constexpr (kQ16) {
        q16[g][i] = *reinterpret_cast<const f16x8*>(static_cast<const f16*>(a.q) + e);
      } else {
        const f32x4* qp = reinterpret_cast<const f32x4*>(static_cast<const float*>(a.q) + e);
        const f32x4 x0 = qp[0], x1 = qp[1];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          q32[g][i * 8 + k] = x0[k];
          q32[g][i * 8 + 4 + k] = x1[k];
        }
      }
    }
  }

  const int pos_raw = a.pos[b];
  const bool pos_ok = pos_raw >= 0 && pos_raw < a.cap;
  if (!pos_ok && tid == 0 && split == 0 && blockIdx.y == 0) atomicOr(a.status, kStatusBadPos);
  const int L = pos_ok ? pos_raw + 1 : (pos_raw < 0 ? 1 : a.cap);
  // Keys this split attends lie in [t0, t1); the last contiguous split also
  // takes any keys past the host bound, and strided splits run to L.
  const int t1 = a.strided || split == nsplit - 1 ? L : min(t1h, L);
  const int n_it = t1 > t0 ? (t1 - t0 + it_keys - 1) / it_keys : 0;
  const auto rk = slab_rsrc(a.k_cache, max(t1, 0)), rv = slab_rsrc(a.v_cache, max(t1, 0));

  // Fused append: the split holding the new position writes the new rows to
  // the caches as soon as the position is known (no other split reads that
  // row, and this split's own loads of it are replaced, so the store may
  // land at any time; issued here it overlaps the stream instead of adding a
  // store round trip after the epilogue), and substitutes them for the cache
  // rows it loads.
  const int pnew = L - 1;
  const bool owns_new =
      has_new && pos_ok && t0 <= pnew && pnew < t1 && (pnew - t0) % it_keys < kBlockKeys;
  // Only the iteration whose tile holds the new key substitutes it: a
  // substitution in every tile lengthened the owning workgroup's chain, the
  // critical path of the whole launch (32K keys: 28.8 against 25.8 us per
  // step with and without the append).
  const int it_new = owns_new ? (pnew - t0) / it_keys : -1;
  f16x8 nk[kRuns], nv[kRuns];
  if (owns_new) {
#pragma unroll
    for (int i = 0; i < kRuns; ++i) {
      nk[i] = convert_src_run(nk_raw[i], a.new16);
      nv[i] = convert_src_run(nv_raw[i], a.new16);
    }
    // the lanes of row 0 of wavefront 0 hold the runs of the new K row, those
    // of row 1 the V row's
    if (wave == 0 && row < 2 && sub == 0 && kv_m * a.kv_rep == hkv) {
#pragma unroll
      for (int i = 0; i < kRuns; ++i) {
        const int64_t at = slab + (int64_t)pnew * Dm + (col + i * kLanes) * 8;
        if (run_real(i) && in_bounds(at, 8, (int64_t)a.batch * nkv_m * a.cap * Dm, a.status)) {
          f16* dst = (row == 0 ? a.k_cache : a.v_cache) + at;
          *reinterpret_cast<f16x8*>(dst) = row == 0 ? nk[i] : nv[i];
        }
      }
    }
  }

  auto qk = [&](const Tile& tl, int j, int g) -> float {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < kRuns; ++i) {
      const f16x8& kk = tl.k[j][i];
      if constexpr (kQ16) {
        const f16x8& qq = q16[g][i];
#pragma unroll
        for (int e = 0; e < 8; e += 2)
          acc = dot2(f16x2{qq[e], qq[e + 1]}, f16x2{kk[e], kk[e + 1]}, acc);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = fmaf(q32[g][i * 8 + e], (float)kk[e], acc);
      }
    }
    return acc;
  };

  float m[G], l[G], acc[G][kDims];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kNegBig;
    l[g] = 0.f;
#pragma unroll
    for (int i = 0; i < kDims; ++i) acc[g][i] = 0.f;
  }

  auto compute_tile = [&](Tile& tl, int it) {
    const int base = t0 + it * it_keys + wave * kWaveKeys + row;
    if (it == it_new) {
#pragma unroll
      for (int j = 0; j < kKpr; ++j) {
        const bool sub = base + j * kRows == pnew;
#pragma unroll
        for (int i = 0; i < kRuns; ++i) {
          tl.k[j][i] = sub ? nk[i] : tl.k[j][i];
          tl.v[j][i] = sub ? nv[i] : tl.v[j][i];
        }
      }
    }
    if (it < kTiles - 1) {  // early tiles' rows at or past t1 may be stale cache rows
#pragma unroll
      for (int j = 0; j < kKpr; ++j) {
        const bool valid = base + j * kRows < t1;
#pragma unroll
        for (int i = 0; i < kRuns; ++i) {
          const u32x4 w = __builtin_bit_cast(u32x4, tl.v[j][i]);
          tl.v[j][i] = __builtin_bit_cast(f16x8, valid ? w : u32x4{0u, 0u, 0u, 0u});
        }
      }
    }
    float s[kKpr][G];
#pragma unroll
    for (int j = 0; j < kKpr; ++j) {
      const bool valid = base + j * kRows < t1;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float d = sum_lanes<kLanes>(qk(tl, j, g));
        s[j][g] = valid ? d * a.qk_scale_log2 : -INFINITY;
      }
    }
    // The reference point m of the online softmax moves only when a score
    // exceeds it by more than kRescaleSlack (log2 units), so weights stay in
    // [0, 2^kRescaleSlack] and the rescale of the accumulators, which ran on
    // almost every tile when any of the wavefront's rows and heads grew its
    // maximum, becomes rare after the first tile. The sums use the same m
    // throughout, so the result is the same softmax.
    float mn[G];
    bool grow = false;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = s[0][g];
#pragma unroll
      for (int j = 1; j < kKpr; ++j) mx = fmaxf(mx, s[j][g]);
      mn[g] = mx > m[g] + kRescaleSlack ? mx : m[g];
      grow |= mn[g] > m[g];
    }
    if (grow) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float al = fast_exp2(m[g] - mn[g]);
        m[g] = mn[g];
        l[g] *= al;
#pragma unroll
        for (int i = 0; i < kDims; ++i) acc[g][i] *= al;
      }
    }
#pragma unroll
    for (int j = 0; j < kKpr; ++j) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float p = fast_exp2(s[j][g] - m[g]);
        l[g] += p;
#pragma unroll
        for (int i = 0; i < kRuns; ++i)
#pragma unroll
          for (int e = 0; e < 8; ++e)
            acc[g][i * 8 + e] = fmaf(p, (float)tl.v[j][i][e], acc[g][i * 8 + e]);
      }
    }
  };

  // A ring of kTiles register tiles: the loads of iterations it+1 ..
  // it+kTiles-1 are in flight while iteration it is computed.
  if (n_it > 0) {
    for (int it0 = 0; it0 < n_it; it0 += kTiles) {
#pragma unroll
      for (int t = 0; t < kTiles; ++t) {
        load_tile(tr[(t + kTiles - 1) % kTiles], rk, rv, it0 + t + kTiles - 1);
        if (t == 0 || it0 + t < n_it) compute_tile(tr[t], it0 + t);
      }
    }
  }

  // Row states to LDS. The lanes l, l ^ kLanes, ... of a wavefront hold the
  // same dims of its other rows; kRowSteps of those lane exchanges (xor 32,
  // then 16, ...) merge rows in registers first, only as far as needed to
  // keep the LDS area under 64 KB (G = 8); the rest are merged below with
  // the wavefronts. (Merging all rows with lane swaps first cost ~250
  // dependent VALU instructions and NOP hazards at the end of every
  // workgroup.)
#pragma unroll
  for (int st = 0; st < kRowSteps; ++st) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float M = row_pair_max(m[g], st);
      const float sc = fast_exp2(m[g] - M);
      l[g] = row_pair_sum(l[g] * sc, st);
#pragma unroll
      for (int i = 0; i < kDims; ++i) acc[g][i] = row_pair_sum(acc[g][i] * sc, st);
      m[g] = M;
    }
  }
  if (row < kRowStates) {
    const int sidx = wave * kRowStates + row;
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int i = 0; i < kRuns; ++i) {
        f32x4* dst = reinterpret_cast<f32x4*>(&lds_o[(sidx * G + g) * kD + (col + i * kLanes) * 8]);
        dst[0] = f32x4{acc[g][i * 8], acc[g][i * 8 + 1], acc[g][i * 8 + 2], acc[g][i * 8 + 3]};
        dst[1] = f32x4{acc[g][i * 8 + 4], acc[g][i * 8 + 5], acc[g][i * 8 + 6], acc[g][i * 8 + 7]};
      }
      if (col == 0) {
        lds_ml[(sidx * G + g) * 2] = m[g];
        lds_ml[(sidx * G + g) * 2 + 1] = l[g];
      }
    }
  }
  __syncthreads();

  store_split_states<G, kO16, kStates, kD, kPadD>(a, lds_o, lds_ml, (int64_t)b * a.n_heads + h0,
                                                  split, Dm);
  if (nsplit == 1 || !a.fused_merge) return;
  merge_on_last_arrival<G, kO16, kD, kPadD>(a, a.counters + b * (a.n_kv * kQsub) + hgrp,
                                            (int64_t)b * a.n_heads + h0);
}

// Separate merge: one wavefront per (query head, sequence). (Earlier forms:
// one 256-thread workgroup per KV head, 10.8 us per 4K decode, then per
// query head, 9.7; one thread per output dim looping over the splits, its
// loads one split at a time, 9.9 against 9.35.)
template <bool kO16>
__global__ __launch_bounds__(64) void decode_merge_kernel(
    const float* __restrict__ part_o, const float2* __restrict__ part_ml,
    void* __restrict__ out, int n_heads, int nsplit, int64_t records, int* __restrict__ status) {
  const int h = blockIdx.x, b = blockIdx.y;
  merge_row_wave<kO16, 0>(part_o, part_ml, out, (int64_t)b * n_heads + h, nsplit,
                          (int64_t)gridDim.y * n_heads, records, status);
}
template <bool kO16, int kD>
__global__ __launch_bounds__(64) void decode_merge_hd_kernel(
    const float* __restrict__ part_o, const float2* __restrict__ part_ml,
    void* __restrict__ out, int n_heads, int nsplit, int64_t records, int* __restrict__ status) {
  const int h = blockIdx.x, b = blockIdx.y;
  merge_row_wave<kO16, 0, kD>(part_o, part_ml, out, (int64_t)b * n_heads + h, nsplit,
                              (int64_t)gridDim.y * n_heads, records, status);
}
// The merge of the padded form: records of kD dims, output rows of od.
template <bool kO16, int kD>
__global__ __launch_bounds__(64) void decode_merge_pad_kernel(
    const float* __restrict__ part_o, const float2* __restrict__ part_ml,
    void* __restrict__ out, int n_heads, int nsplit, int64_t records, int* __restrict__ status,
    int od) {
  const int h = blockIdx.x, b = blockIdx.y;
  merge_row_wave<kO16, 0, kD, true>(part_o, part_ml, out, (int64_t)b * n_heads + h, nsplit,
                                    (int64_t)gridDim.y * n_heads, records, status, od);
}

// The split workgroup's shape, from sweeps on MI355X (decode-only, per call,
// 32K / 4K / 153 keys): 4 wavefronts, 16-lane rows, 2 keys per row, 2 tiles
// in flight: 26.5-27.5 / 9.2-9.4 / 4.6 us. Eight wavefronts (two per SIMD):
// 28.5 / 10.6 / 5.0; 8-lane rows (fewer reduction and softmax instructions
// per key, twice the accumulators): 28.0-28.5 / 10.5-10.7 / 4.9-5.0; 3 or 4
// tiles in flight: 27.4-27.5 / 9.9-10.3 / 4.7-4.9. The loop is bound by HBM
// (the K/V stream alone, with the compute removed, runs at the rate of a
// plain read of the same pattern, ~6.2 TB/s), so more work in flight only
// lengthens the latency of each load.
// Head size 64 takes 8-lane rows (one 16-byte run per lane), 256 two runs
// per lane of 16-lane rows.
using SplitCfg = DecodeCfg<4, 16, 2, 2>;
template <int kD>
using SplitCfgD = std::conditional_t<kD == kHeadDim, SplitCfg,
                                     DecodeShape<4, kD == 64 ? 8 : 16, 2, 2, kD>>;
template <int kD, bool kPadD>
using SplitCfgP = std::conditional_t<kPadD, DecodePadShape<4, kD == 64 ? 8 : 16, 2, 2, kD>,
                                     SplitCfgD<kD>>;

template <int G, bool kQ16, bool kO16, int kQsub, int kD = kHeadDim, bool kPadD = false>
static hipError_t launch_g(const DecodeArgs& a, int batch, hipStream_t stream, void* ev_start,
                           void* ev_stop) {
  using C = SplitCfgP<kD, kPadD>;
  dim3 grid((unsigned)a.nsplit, (unsigned)(a.n_kv * kQsub), (unsigned)batch);
  hipError_t e;
  if (ev_start || ev_stop) {
    // Measurement: the runtime records the events when the split kernel
    // starts and when it ends.
    DecodeArgs arg = a;
    void* args[] = {&arg};
    e = hipExtLaunchKernel(reinterpret_cast<const void*>(&decode_split_kernel<G, kQ16, kO16, kQsub, C>),
                           grid, dim3(C::kThreads), args, 0, stream, (hipEvent_t)ev_start,
                           (hipEvent_t)ev_stop, 0);
  } else {
    decode_split_kernel<G, kQ16, kO16, kQsub, C><<<grid, C::kThreads, 0, stream>>>(a);
    e = hipGetLastError();
  }
  if (e != hipSuccess || a.nsplit == 1 || a.fused_merge) return e;
  const dim3 mgrid((unsigned)a.n_heads, (unsigned)batch);
  if constexpr (kPadD)
    decode_merge_pad_kernel<kO16, kD><<<mgrid, 64, 0, stream>>>(a.part_o, a.part_ml, a.out,
                                                                a.n_heads, a.nsplit, a.records,
                                                                a.status, a.head_dim);
  else if constexpr (kD == kHeadDim)
    decode_merge_kernel<kO16><<<mgrid, 64, 0, stream>>>(a.part_o, a.part_ml, a.out, a.n_heads,
                                                        a.nsplit, a.records, a.status);
  else
    decode_merge_hd_kernel<kO16, kD><<<mgrid, 64, 0, stream>>>(a.part_o, a.part_ml, a.out,
                                                               a.n_heads, a.nsplit, a.records,
                                                               a.status);
  return hipGetLastError();
}

template <int G, int kQsub = 1, int kD = kHeadDim, bool kPadD = false>
static hipError_t launch_qo(const Shape& s, const DecodeArgs& a, const DecodeCall& c,
                            hipStream_t st) {
  const int B = c.batch;
  if (s.q16)
    return s.o16 ? launch_g<G, true, true, kQsub, kD, kPadD>(a, B, st, c.ev_start, c.ev_stop)
                 : launch_g<G, true, false, kQsub, kD, kPadD>(a, B, st, c.ev_start, c.ev_stop);
  return s.o16 ? launch_g<G, false, true, kQsub, kD, kPadD>(a, B, st, c.ev_start, c.ev_stop)
               : launch_g<G, false, false, kQsub, kD, kPadD>(a, B, st, c.ev_start, c.ev_stop);
}



// decode_split_kernel launches at head sizes other than 128 (nwd_decode_hd.hip).
hipError_t launch_decode_other(const Shape& s, const DecodeArgs& a, const DecodeCall& c,
                               hipStream_t stream);

}  // namespace nwd
