// nwd_decode.hip — decode GQA attention for gfx950 (split-K + merge).
//
// Replaces kernels/sparse_attn.wgsl main (:31-114). The reference runs one
// 64-thread workgroup per QUERY head (engine/runtime.js:391), so each of the
// G = H/Hkv query heads of a group re-reads the same K/V rows, with one
// thread streaming one whole key row (uncoalesced), and it caps the context
// at 256 keys (:29).
//
// Here one workgroup owns (sequence b, KV head hkv, split s): it loads each
// K/V row of its key range once and serves all G query heads of the group
// from it. When few sequences leave the chip nearly idle, the launch instead
// gives each query head its own workgroups (kQsub = G workgroups per KV head,
// each serving one head), which shortens every workgroup's serial chain
// G-fold.
//
// Mapping inside a wavefront: rows of kLanes lanes (16 or 8); a row owns one
// key at a time and each lane holds 128 / kLanes of its dims (one or two
// 16-byte runs), so one load instruction reads 1 KB of consecutive keys. q.k
// is a packed fp16 dot (v_dot2_f32_f16) or an fp32 FMA chain, summed over the
// row's lanes with DPP moves, so every lane of the row holds the score. Each
// row runs its own online softmax (running max and sum in log2 units, exp2
// on the hardware) and accumulates p * V for its dims in fp32 with no
// cross-lane traffic. The next iteration's K/V loads are issued before the
// current one is computed, unconditionally, so the wait before the compute
// only waits for the older loads; they go through buffer descriptors that
// end at the split's last key, so the prefetch past the end reads zeros
// without a memory round trip, and they are marked non-temporal (each byte
// is read once). At the end the row states are merged (DPP and lane swaps
// inside a wave, LDS across waves) into one record (m, l, o[128]) per query
// head.
//
// With one split the record is normalised and written to `out`. With
// several, records go to the workspace and decode_merge_kernel combines them
// — the partial/merge structure of kernels/argmax_partial.wgsl:16-52 and
// kernels/argmax_merge.wgsl:8-42, with (max, sum, o[D]) records instead of
// (value, index) pairs. Optionally (nwd_set_decode_merge) the merge runs in
// the split kernel itself: records are written through to memory (vector
// stores with the agent-coherent cache policy sc1) and the workgroup that
// takes the last arrival ticket of its (b, hkv) reads them with sc1 loads
// and merges them.
//
// The key range is partitioned from the host's length bound (max_len), not
// from the device position, so a workgroup's first K/V loads do not wait for
// the position load; the position only masks keys and bounds the loop, and
// the last split extends past the bound if the position exceeds it.
//
// Fused append: when new K/V rows are given, the workgroup whose range holds
// the new position writes them into the caches and uses them from registers,
// so an attention-layer step (kv_append x2 + attention in the reference,
// engine/runtime.js:389-391) is one launch.
#include <hip/hip_ext.h>

#include <atomic>
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

// ---------------------------------------------------------------------------
// Matrix-core form of the split workgroup (decode_mfma_kernel). Same
// key-range partition, records and merges as decode_split_kernel; the loop
// runs on fp16 MFMAs instead of VALU dot products, so its work per key does
// not grow with the group size G, while decode_split_kernel's does.
// Decode-only calls, B = 1, 8 KV heads, K/V N(0,1), same box (us,
// dot-product / matrix-core):
//   G = 4: 2K 8.3 / 8.5, 4K 9.2 / 9.5, 16K 16.3 / 17.0, 32K 26.2 / 26.5
//   G = 5: 2K 8.9 / 8.6, 4K 9.9 / 9.6, 16K 17.9 / 17.1, 32K 27.3 / 26.4
//   G = 8: 1K 11.0 / 8.6, 4K 12.2 / 9.9, 16K 23.5 / 17.3, 32K 38.9 / 26.7
// (with 1% of K/V at +-8, whose larger score swings move the dot-product
// kernel's per-row references more often, 32K: 27.0 / 26.3, 28.6 / 26.6,
// 39.0 / 26.8). Batches at G = 4, N(0,1): B 2 x 8K 15.5-16.4 / 15.5-15.8,
// 8 x 16K 98.6 / 89.6, 12 x 8K 65.0 / 61.0, 16 x 256 8.9 / 8.4, 16 x 8K
// 90.3 / 83.4, 64 x 2K 86.8 / 81.3, 64 ragged 512..16K 422 / 409 (ties at
// 4 x 8K, 8 x 4K, 16 x 2K). Timed as append + attend steps at B = 1 and
// G = 4 on two more boxes it led from 16K keys up (16.2 / 20.6 / 25.1
// against 16.8 / 21.1 / 26.2 us at 16K / 24K / 32K on N(0,1) K/V), while
// the dot-product kernel stays ahead at 4K. The launch takes it for
// one-workgroup-per-KV-head calls with G >= 5, or G = 4 with a batch or with
// splits of 512+ keys in one wave (launch_decode); nwd_set_decode_kernel
// forces either.
// Four wavefronts, each owning one 16-key block of every 64-key workgroup
// iteration (keys t0 + 64 it + 16 w ..), independent of each other inside
// the loop:
//   - K: lane (r = lane % 16, q = lane / 16) loads dims 32 db + 8q .. +8 of
//     key r straight into registers (per instruction, one 64-byte run of
//     each of 16 rows): the A operands of S^T = K Q^T on
//     v_mfma_f32_16x16x32_f16;
//   - Q^T, the B operand, holds query head h0 + r in column r (zero for
//     r >= G), so one MFMA serves every head of the group;
//   - V: the wavefront copies its block's V rows into its own LDS ring
//     (buffer_load_dwordx4 with the lds flag, no registers held) and reads
//     the V^T operands with ds_read_b64_tr_b16, as prefill does;
//   - softmax: each lane holds 4 consecutive keys of one head, the B
//     operand layout of v_mfma_f32_16x16x16_f16, which computes O^T += V^T
//     P^T; weights are exp2(s * scale * log2 e - m) in fp32, given to it as
//     fp16 high and low parts (so the result keeps fp32-like precision and
//     does not depend on the split count); the reference m moves only for
//     a head's first keys and when a weight may exceed fp16 (then lazily,
//     by more than kRescaleSlack).
// The loads of block it + 1 are issued before block it is computed. Shape
// of the loop, measured at G = 4, 32K keys (us per call): 16-key blocks
// with two in flight 25.3, three 25.7, four 26.1; 32-key blocks with two in
// flight 26.0, three 26.9 (and staging K through LDS as whole rows too,
// 26.6). K loads use the default cache policy, V copies the non-temporal
// one (non-temporal K: 25.7 against 25.3; default-policy V: 28.9). An fp32
// query is split into fp16 high and low parts (two MFMAs per operand), so
// the scores keep ~22 bits of the query.
// Workgroups of one matrix-core launch that run at once: one per CU (256 CUs).
constexpr int kMOneWave = 256;
constexpr int kMWaves = 4;
constexpr int kMThreads = kMWaves * 64;
constexpr int kMWaveKeys = 16;                           // keys per wavefront per iteration
constexpr int kMBlockKeys = kMWaves * kMWaveKeys;       // keys per workgroup iteration
constexpr int kMSlotBytes = kMWaveKeys * kHeadDim * 2;  // one V block: 4 KB
constexpr int kMDepth = 2;                               // blocks in flight per wavefront
constexpr size_t kMLdsBytes = (size_t)kMWaves * kMDepth * kMSlotBytes;
constexpr int kMBlockLoads = 4 + kMSlotBytes / 1024;  // K fragments + V copies
static_assert(kUnitKeys % kMWaveKeys == 0, "a split's range is whole wavefront blocks");
static_assert(kMBlockLoads * (kMDepth - 1) <= 63, "vmcnt counts at most 63 loads");
static_assert(kMLdsBytes <= 160 * 1024, "LDS of one gfx950 CU");

// Chunk swizzle of the V rows in LDS (16 chunks of 16 bytes per row):
// physical chunk p of row r holds logical chunk p ^ vswz_m(r), so the
// transpose reads (4 rows x 2 chunks per 16 lanes) hit 8 distinct chunks.
__device__ inline int vswz_m(int r) { return (r & 7) << 1; }

// s_waitcnt vmcnt(n) that the compiler keeps in place: memory accesses do
// not move across it.
template <int n>
__device__ inline void wait_vm_keep() {
  static_assert(n == 0 || n == 8, "instantiated counts");
  if constexpr (n == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if constexpr (n == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
}
__device__ inline void compiler_fence() { asm volatile("" ::: "memory"); }

template <int G, bool kQ16, bool kO16>
__global__ __launch_bounds__(kMThreads, 1) void decode_mfma_kernel(const DecodeArgs a) {
  static_assert(G <= 16, "the heads of a group are the MFMA's 16 columns");
  static_assert(kMBlockLoads == 8, "wait counts below assume 8 loads per block");
  static_assert(G * 32 <= kMThreads, "one 4-dim run of each head per thread");
  static_assert((size_t)kMWaves * G * (kHeadDim + 2) * 4 <= kMLdsBytes,
                "the end of the kernel reuses the ring");
  extern __shared__ __attribute__((aligned(16))) f16 dsmem[];
  char* lds = reinterpret_cast<char*>(dsmem);

  const int b = blockIdx.z, hkv = blockIdx.y;
  // The KV head this group of query heads reads (DecodeArgs::kv_rep).
  const int kv_m = a.kv_rep > 1 ? hkv / a.kv_rep : hkv;
  const int nkv_m = a.kv_rep > 1 ? a.n_kv / a.kv_rep : a.n_kv;
  int split = blockIdx.x + (b & 7);  // XCD rotation, as decode_split_kernel
  while (split >= a.nsplit) split -= a.nsplit;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lq = lane >> 4;
  const int nsplit = a.nsplit;

  // Key partition as in decode_split_kernel, in blocks of kMBlockKeys.
  const int units = (a.span + kUnitKeys - 1) / kUnitKeys;
  const int u0 = (int)((int64_t)split * units / nsplit);
  const int u1 = (int)((int64_t)(split + 1) * units / nsplit);
  const int t0 = a.strided ? split * kMBlockKeys : u0 * kUnitKeys;
  const int it_keys = a.strided ? nsplit * kMBlockKeys : kMBlockKeys;
  const int t1h = min(a.span, u1 * kUnitKeys);
  const int64_t slab = (int64_t)(b * nkv_m + kv_m) * a.cap * kHeadDim;
  auto slab_rsrc = [&](f16* cache, int end_key) {
    return __builtin_amdgcn_make_buffer_rsrc(cache + slab, 0, end_key * (kHeadDim * 2),
                                             kBufferWord3);
  };
  char* const ring = lds + wave * (kMDepth * kMSlotBytes);

  struct KFrag {
    f16x8 k[4];  // [32-dim block]
  };
  auto load_k = [&](KFrag& f, const __amdgpu_buffer_rsrc_t rk, int it) {
    const int key0 = t0 + it * it_keys + wave * kMWaveKeys;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const uint32_t off = (uint32_t)(key0 + lr) * (kHeadDim * 2) + db * 64 + lq * 16;
      f.k[db] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
    }
  };
  // The block's 16 V rows into ring slot `slot`: 4 copies of 4 rows (1 KB);
  // lane l fills physical chunk l % 16 of row 4i + l / 16, so it loads the
  // logical chunk the swizzle puts there.
  auto load_v = [&](const __amdgpu_buffer_rsrc_t rv, int it, int slot) {
    const int key0 = t0 + it * it_keys + wave * kMWaveKeys;
    char* dst = ring + slot * kMSlotBytes;
#pragma unroll
    for (int i = 0; i < kMSlotBytes / 1024; ++i) {
      const int row = 4 * i + lq;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rv, (lds_void*)(dst + i * 1024), 16,
          (uint32_t)(key0 + row) * (kHeadDim * 2) + ((lr ^ vswz_m(row)) << 4), 0, 0,
          kStreamPolicy);
    }
  };

  // Fused append: the new rows are requested first (the K chunks this
  // lane's fragments hold, and V logical chunk lr), before the position
  // says which split owns them.
  const bool has_new = a.k_new != nullptr;
  SrcRun nk_raw[4], nv_raw;
  if (has_new) {
    const int64_t src = (int64_t)(b * nkv_m + kv_m) * kHeadDim;
#pragma unroll
    for (int db = 0; db < 4; ++db) nk_raw[db] = load_src_run_raw(a.k_new, src + db * 32 + 8 * lq, a.new16);
    nv_raw = load_src_run_raw(a.v_new, src + 8 * lr, a.new16);
  }

  // The first kMDepth - 1 blocks are requested before the position is
  // known, over the keys this split can own; rows at or past L are zeroed
  // in LDS before use (see below). Each block's copies are kept together,
  // so the wait counts below see whole blocks.
  KFrag kf[kMDepth];
  {
    const int own_end = a.strided || split == nsplit - 1 ? a.cap : t1h;
    const auto ek = slab_rsrc(a.k_cache, own_end), ev = slab_rsrc(a.v_cache, own_end);
#pragma unroll
    for (int t = 0; t < kMDepth - 1; ++t) {
      load_k(kf[t], ek, t);
      load_v(ev, t, t);
      compiler_fence();
    }
  }

  // Q^T: column lr is head h0 + lr; the rows past the group are zero.
  const int h0 = hkv * G;
  f16x8 qh[4], ql[kQ16 ? 1 : 4];
  bool q_range = false;
  {
    const bool qv = lr < G;
    const int64_t qrow = ((int64_t)b * a.n_heads + h0 + (qv ? lr : 0)) * kHeadDim + 8 * lq;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      if constexpr (kQ16) {
        const f16x8 h = *reinterpret_cast<const f16x8*>(static_cast<const f16*>(a.q) + qrow + db * 32);
        qh[db] = qv ? h : f16x8{};
      } else {
        const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(a.q) + qrow + db * 32);
        const f32x4 x0 = p[0], x1 = p[1];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = qv ? (e < 4 ? x0[e] : x1[e - 4]) : 0.f;
          qh[db][e] = (f16)x;
          ql[db][e] = (f16)(x - (float)qh[db][e]);
          q_range |= fabsf(x) > 65504.f;
        }
      }
    }
  }
  if (!kQ16 && q_range && split == 0) atomicOr(a.status, kStatusQueryRange);

  const int pos_raw = a.pos[b];
  const bool pos_ok = pos_raw >= 0 && pos_raw < a.cap;
  if (!pos_ok && tid == 0 && split == 0 && hkv == 0) atomicOr(a.status, kStatusBadPos);
  const int L = pos_ok ? pos_raw + 1 : (pos_raw < 0 ? 1 : a.cap);
  const int t1 = a.strided || split == nsplit - 1 ? L : min(t1h, L);
  const int n_it = t1 > t0 ? (t1 - t0 + it_keys - 1) / it_keys : 0;
  const auto rk = slab_rsrc(a.k_cache, max(t1, 0)), rv = slab_rsrc(a.v_cache, max(t1, 0));

  // Fused append: the wavefront whose block holds the new position writes
  // the new rows to the caches as soon as the position is known (as in
  // decode_split_kernel) and substitutes them (K in its fragments, V in its
  // LDS slot). Its stores are older than the next block's loads, so the
  // block waits below cover them.
  const int pnew = L - 1;
  const bool owns_new =
      has_new && pos_ok && t0 <= pnew && pnew < t1 && (pnew - t0) % it_keys < kMBlockKeys;
  const int it_new = owns_new ? (pnew - t0) / it_keys : -1;
  const int w_new = owns_new ? (pnew - t0) % it_keys / kMWaveKeys : -1;
  const int r_new = (pnew - t0) % kMWaveKeys;
  f16x8 nk[4], nv;
  if (owns_new) {
#pragma unroll
    for (int db = 0; db < 4; ++db) nk[db] = convert_src_run(nk_raw[db], a.new16);
    nv = convert_src_run(nv_raw, a.new16);
    // K chunks 4 db + lq from the lanes of key row 0, V chunk lr from lane
    // group 0
    if (wave == w_new && kv_m * a.kv_rep == hkv) {
      const int64_t at = slab + (int64_t)pnew * kHeadDim;
      const int64_t cache_elems = (int64_t)a.batch * nkv_m * a.cap * kHeadDim;
      if (lr == 0) {
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const int64_t e = at + db * 32 + 8 * lq;
          if (in_bounds(e, 8, cache_elems, a.status)) *reinterpret_cast<f16x8*>(a.k_cache + e) = nk[db];
        }
      }
      if (lq == 0 && in_bounds(at + 8 * lr, 8, cache_elems, a.status))
        *reinterpret_cast<f16x8*>(a.v_cache + at + 8 * lr) = nv;
    }
  }

  const float c = a.qk_scale_log2;
  float m = kNegBig, lsum = 0.f;  // head lr: reference point (log2 units), sum of weights
  f32x4 o[8];                     // O^T: dims 16 dblk + 4 lq .. +4 of head lr
#pragma unroll
  for (int d = 0; d < 8; ++d) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](KFrag& f, int it, int slot) {
    wait_vm_keep<kMBlockLoads * (kMDepth - 1)>();  // block it's K fragments and V rows are in
    const int key0 = t0 + it * it_keys + wave * kMWaveKeys;
    if (key0 >= t1) return;  // nothing of this block is attended
    char* vs = ring + slot * kMSlotBytes;
    const bool partial = key0 + kMWaveKeys > t1;
    if (it == it_new && wave == w_new) {
      const bool sub = lr == r_new;
#pragma unroll
      for (int db = 0; db < 4; ++db) f.k[db] = sub ? nk[db] : f.k[db];
      if (lq == 0) *reinterpret_cast<f16x8*>(vs + r_new * (kHeadDim * 2) + ((lr ^ vswz_m(r_new)) << 4)) = nv;
    }
    if (partial) {
      // Rows at or past t1: zeros past the descriptor's end, or stale cache
      // rows in the blocks requested before the position was known; a stale
      // Inf or NaN times a zero weight would be NaN, so they are zeroed.
#pragma unroll
      for (int i = 0; i < kMSlotBytes / 1024; ++i) {
        const int row = 4 * i + lq;
        if (key0 + row >= t1) *reinterpret_cast<u32x4*>(vs + row * (kHeadDim * 2) + (lr << 4)) = u32x4{0u, 0u, 0u, 0u};
      }
    }
    // S^T: s[e] = q . k for key key0 + 4 lq + e, head lr.
    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      s = mfma16x16x32(f.k[db], qh[db], s);
      if constexpr (!kQ16) s = mfma16x16x32(f.k[db], ql[db], s);
    }
    // V^T operands (dims 16 dblk + lr, keys 4 lq + e), requested before the
    // softmax: the A operands of v_mfma_f32_16x16x16_f16, whose B operand
    // layout (keys 4 lq .. 4 lq + 3 of column lr) is that of S^T, so the
    // weights need no data movement between lanes.
    const int vr0 = 4 * lq + (lr >> 2);
    f16x4 vf[8];
#pragma unroll
    for (int dblk = 0; dblk < 8; ++dblk)
      vf[dblk] = lds_read_tr16_asm(vs + vr0 * (kHeadDim * 2) +
                                   (((2 * dblk + ((lr >> 1) & 1)) ^ vswz_m(vr0)) << 4) + 8 * (lr & 1));
    const float mu = m > kNegBig ? m : 0.f;
    float st[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      st[e] = fmaf(s[e], c, -mu);
      if (partial && key0 + 4 * lq + e >= t1) st[e] = -INFINITY;
    }
    float mu_now = mu;
    auto rescale = [&]() {
      const float mx = fmaxf(fmaxf(st[0], st[1]), fmaxf(st[2], st[3]));
      const float ax = max_xor32(max_xor16(mx)) + mu_now;  // the head's maximum
      if (ax > m + kRescaleSlack) {
        const float al = fast_exp2(m - ax);
        lsum *= al;
#pragma unroll
        for (int d = 0; d < 8; ++d) o[d] *= al;
        m = ax;
        const float dd = mu_now - ax;
#pragma unroll
        for (int e = 0; e < 4; ++e) st[e] += dd;
        mu_now = ax;
      }
    };
    // P^T operands: each fp32 weight w as fp16 hi + lo (w - hi rounded), two
    // PV MFMAs, so the product keeps ~22 bits of w and the result does not
    // depend on where a split's reference point lies.
    f16x4 ph, pl;
    auto weights = [&]() {
      float ls = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float w = fast_exp2(st[e]);
        const f16 h = (f16)w;
        ph[e] = h;
        pl[e] = (f16)(w - (float)h);
        ls += w;
      }
      return ls;
    };
    // The maximum is taken for a head's first keys (so its largest weight
    // is never below 1) and when a weight may exceed fp16 (a lane's sum of
    // 4 weights reaches 65504: the maximum then exceeds m by more than 13,
    // so m moves); both tests are wavefront-wide.
    if (__builtin_amdgcn_ballot_w64(m == kNegBig)) rescale();
    float ls = weights();
    if (__builtin_amdgcn_ballot_w64(ls >= 65504.f)) {
      rescale();
      ls = weights();
    }
    lsum += ls;
    lds_reads_done(vf);
#pragma unroll
    for (int dblk = 0; dblk < 8; ++dblk) {
      o[dblk] = __builtin_amdgcn_mfma_f32_16x16x16f16(vf[dblk], ph, o[dblk], 0, 0, 0);
      o[dblk] = __builtin_amdgcn_mfma_f32_16x16x16f16(vf[dblk], pl, o[dblk], 0, 0, 0);
    }
  };

  for (int it0 = 0; it0 < n_it; it0 += kMDepth) {
#pragma unroll
    for (int t = 0; t < kMDepth; ++t) {
      // The slot copied into next was read by the previous block: its
      // transpose reads are complete before the copy is issued.
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      // The prefetch past the split's last block reads zeros without a
      // memory access (descriptor range) and keeps the wait counts exact.
      load_k(kf[(t + kMDepth - 1) % kMDepth], rk, it0 + t + kMDepth - 1);
      load_v(rv, it0 + t + kMDepth - 1, (t + kMDepth - 1) % kMDepth);
      if (it0 + t < n_it) compute(kf[t], it0 + t, t);
    }
  }
  wait_vm_keep<0>();  // no copy into the ring is in flight when it is reused below

  // Wavefront states to LDS ([kMWaves][G][D] and [kMWaves][G][2]), then the
  // shared end of a split workgroup.
  lsum = sum_xor32(sum_xor16(lsum));  // the head's sum over its 4 lane groups
  __syncthreads();
  float* lds_o = reinterpret_cast<float*>(lds);
  float* lds_ml = lds_o + kMWaves * G * kHeadDim;
  if (lr < G) {
#pragma unroll
    for (int dblk = 0; dblk < 8; ++dblk)
      *reinterpret_cast<f32x4*>(&lds_o[(wave * G + lr) * kHeadDim + dblk * 16 + 4 * lq]) = o[dblk];
    if (lq == 0) {
      lds_ml[(wave * G + lr) * 2] = m;
      lds_ml[(wave * G + lr) * 2 + 1] = lsum;
    }
  }
  __syncthreads();
  const int64_t hrow0 = (int64_t)b * a.n_heads + h0;
  store_split_states<G, kO16, kMWaves>(a, lds_o, lds_ml, hrow0, split);
  if (nsplit == 1 || !a.fused_merge) return;
  merge_on_last_arrival<G, kO16>(a, a.counters + b * a.n_kv + hkv,
                                 hrow0);
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


template <int G, bool kQ16, bool kO16>
static hipError_t launch_mfma_t(const DecodeArgs& a, int batch, hipStream_t stream, void* ev_start,
                                void* ev_stop) {
  auto kern = decode_mfma_kernel<G, kQ16, kO16>;
  // The ring exceeds the 64 KB default of dynamic LDS: raise the kernel's
  // limit once per device (the attribute is per device).
  static std::atomic<uint64_t> attr_set{0};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = 1ull << (dev & 63);
  if (!(attr_set.load() & bit)) {
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMLdsBytes);
    if (e != hipSuccess) return e;
    attr_set.fetch_or(bit);
  }
  const dim3 grid((unsigned)a.nsplit, (unsigned)a.n_kv, (unsigned)batch);
  if (ev_start || ev_stop) {
    DecodeArgs arg = a;
    void* args[] = {&arg};
    e = hipExtLaunchKernel(reinterpret_cast<const void*>(kern), grid, dim3(kMThreads), args,
                           kMLdsBytes, stream, (hipEvent_t)ev_start, (hipEvent_t)ev_stop, 0);
  } else {
    kern<<<grid, kMThreads, kMLdsBytes, stream>>>(a);
    e = hipGetLastError();
  }
  if (e != hipSuccess || a.nsplit == 1 || a.fused_merge) return e;
  decode_merge_kernel<kO16><<<dim3((unsigned)a.n_heads, (unsigned)batch), 64, 0, stream>>>(
      a.part_o, a.part_ml, a.out, a.n_heads, a.nsplit, a.records, a.status);
  return hipGetLastError();
}

template <int G>
static hipError_t launch_mfma(const Shape& s, const DecodeArgs& a, const DecodeCall& c,
                              hipStream_t st) {
  const int B = c.batch;
  if (s.q16)
    return s.o16 ? launch_mfma_t<G, true, true>(a, B, st, c.ev_start, c.ev_stop)
                 : launch_mfma_t<G, true, false>(a, B, st, c.ev_start, c.ev_stop);
  return s.o16 ? launch_mfma_t<G, false, true>(a, B, st, c.ev_start, c.ev_stop)
               : launch_mfma_t<G, false, false>(a, B, st, c.ev_start, c.ev_stop);
}

// Head sizes other than 128 (decode_split_kernel only; the matrix-core
// kernel is built for 128): 64 and 256 as they are, other multiples of 8 up
// to 256 in the padded form of the next of 64, 128, 256. The same
// per-query-head rule, then one workgroup per KV head. Group 8 above 128 is
// not built (its accumulators and query registers would not fit one lane's
// registers) and takes the general-shape kernels.
template <int kD, bool kPadD>
static hipError_t launch_decode_hd(const Shape& s, const DecodeArgs& a, const DecodeCall& c,
                                   hipStream_t stream) {
  if ((int64_t)c.batch * s.n_heads * a.nsplit <= kSubSplitMaxWorkgroups) {
    switch (s.group) {
      case 2: return launch_qo<1, 2, kD, kPadD>(s, a, c, stream);
      case 4: return launch_qo<1, 4, kD, kPadD>(s, a, c, stream);
      case 5: return launch_qo<1, 5, kD, kPadD>(s, a, c, stream);
      case 8:
        if constexpr (kD <= kHeadDim) return launch_qo<1, 8, kD, kPadD>(s, a, c, stream);
        break;
      default: break;
    }
  }
  switch (s.group) {
    case 1: return launch_qo<1, 1, kD, kPadD>(s, a, c, stream);
    case 2: return launch_qo<2, 1, kD, kPadD>(s, a, c, stream);
    case 4: return launch_qo<4, 1, kD, kPadD>(s, a, c, stream);
    case 5: return launch_qo<5, 1, kD, kPadD>(s, a, c, stream);
    case 8:
      if constexpr (kD <= kHeadDim) return launch_qo<8, 1, kD, kPadD>(s, a, c, stream);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

// A larger group runs as groups of the largest built size (8 up to head size
// 128, 5 above), so that each KV head's rows are read as few times as
// possible: kv_rep = ceil(group / largest) reads. A divisor among 8, 5, 4
// that gives that many groups takes the group as it is; otherwise it is
// padded to a multiple of the largest size. Decode calls on MI355X, B = 1,
// 8192 keys: 96q/8kv/d128 (group 12) as 3 groups of 4, 20.6 us, padded to
// 16 as 2 groups of 8, 16.6 (128q/8kv, 2 groups of 8: 12.4; on the general
// kernels 43.3).
int kernel_group(int head_dim, int group, int* kv_rep) {
  *kv_rep = 1;
  const int top = head_dim <= kHeadDim ? 8 : 5;  // group 8 is built up to head size 128
  if (group == 1 || group == 2 || group == 4 || group == 5 || group == top) return group;
  if (group < 8) return 0;  // 3, 6, 7: padded first
  const int reads = (group + top - 1) / top;
  for (int gs : {top, 5, 4}) {
    if (group % gs == 0 && group / gs == reads) {
      *kv_rep = reads;
      return gs;
    }
  }
  return 0;
}

int padded_group(int head_dim, int group) {
  int rep = 0;
  if (kernel_group(head_dim, group, &rep) > 0) return 0;
  if (group == 3) return 4;
  if (group < 8) return 8;
  const int top = head_dim <= kHeadDim ? 8 : 5;
  return (group + top - 1) / top * top;
}

bool split_decode_shape(int head_dim, int group) {
  int rep = 0;
  return head_dim >= 8 && head_dim <= 256 && head_dim % 8 == 0 &&
         kernel_group(head_dim, group, &rep) > 0;
}

hipError_t launch_decode(const Shape& s0, const DecodeCall& c, const Workspace& ws,
                         hipStream_t stream) {
  if (!split_decode_shape(s0.head_dim, s0.group)) return hipErrorInvalidValue;
  // A group the kernels are not built for runs as kv_rep groups of a built
  // size per KV head (kernel_group); the kernels then see n_kv * kv_rep KV
  // heads of that group.
  int kv_rep = 1;
  Shape s = s0;
  s.group = kernel_group(s0.head_dim, s0.group, &kv_rep);
  s.n_kv = s0.n_kv * kv_rep;
  DecodeArgs a;
  a.q = c.q;
  a.k_cache = static_cast<f16*>(c.k_cache);
  a.v_cache = static_cast<f16*>(c.v_cache);
  a.pos = c.pos;
  a.out = c.out;
  a.part_o = ws.part_o;
  a.part_ml = ws.part_ml;
  a.records = ws.records;
  a.k_new = c.k_new;
  a.v_new = c.v_new;
  a.new16 = s.kv16;
  a.batch = c.batch;
  a.n_heads = s.n_heads;
  a.n_kv = s.n_kv;
  a.cap = s.cap;
  a.nsplit = c.nsplit;
  a.span = c.span;
  a.counters = ws.counters;
  a.fused_merge = c.fused_merge;
  a.strided = c.layout == 1;
  a.qk_scale_log2 = s.qk_scale * kLog2e;
  a.status = ws.status;
  a.head_dim = s.head_dim;
  a.kv_rep = kv_rep;
  if (s.head_dim == 64) return launch_decode_hd<64, false>(s, a, c, stream);
  if (s.head_dim == 256) return launch_decode_hd<256, false>(s, a, c, stream);
  if (s.head_dim < 64) return launch_decode_hd<64, true>(s, a, c, stream);
  if (s.head_dim < kHeadDim) return launch_decode_hd<kHeadDim, true>(s, a, c, stream);
  if (s.head_dim > kHeadDim) return launch_decode_hd<256, true>(s, a, c, stream);
  // When one workgroup per (sequence, query head, split) fits the chip, each
  // query head gets its own workgroups: a workgroup's time is its serial
  // chain of key iterations, whose compute grows with the heads it serves,
  // and the G-fold K/V reads are small at the lengths the split rule sends
  // here (per append + attend step, B = 1, G = 4: 4.5 against 6.3 us at 153
  // keys with one split; 6.1 against 8.1 at 832 keys and 6.8 against 8.3 at
  // 1088 with 8 splits). Same bits.
  auto mfma = [&]() -> hipError_t {
    switch (s.group) {
      case 1: return launch_mfma<1>(s, a, c, stream);
      case 2: return launch_mfma<2>(s, a, c, stream);
      case 4: return launch_mfma<4>(s, a, c, stream);
      case 5: return launch_mfma<5>(s, a, c, stream);
      case 8: return launch_mfma<8>(s, a, c, stream);
      default: return hipErrorInvalidValue;
    }
  };
  if (c.kernel == 1) return mfma();  // the caller's choice (nwd_set_decode_kernel)
  if ((int64_t)c.batch * s.n_heads * a.nsplit <= kSubSplitMaxWorkgroups) {
    switch (s.group) {
      case 2: return launch_qo<1, 2>(s, a, c, stream);
      case 4: return launch_qo<1, 4>(s, a, c, stream);
      case 5: return launch_qo<1, 5>(s, a, c, stream);
      case 8: return launch_qo<1, 8>(s, a, c, stream);
      default: break;  // group 1 is already one workgroup per query head
    }
  }
  // One workgroup per KV head: the matrix-core kernel where it measured
  // faster (see decode_mfma_kernel): G >= 5; G = 4 with a batch, or with
  // long splits (at least 512 keys each) whose workgroups all fit the chip at
  // once (B = 1, 32q/8kv, append + attend per step, 16K / 24K / 32K keys:
  // 16.2 / 20.6 / 25.1 against 16.8 / 21.1 / 26.2 us on N(0,1) K/V, and
  // 16.2 / 20.7 / 25.1 against 17.1 / 21.7 / 26.8 with 1% outliers, on two
  // boxes; at 64K keys, 33 splits and 264 workgroups, 62.9 against 60.6).
  const bool long_splits = (int64_t)c.span >= 512LL * c.nsplit &&
                           (int64_t)c.batch * s.n_kv * c.nsplit <= kMOneWave;
  if (c.kernel < 0 && (s.group >= 5 || (s.group == 4 && (c.batch >= 2 || long_splits))))
    return mfma();
  switch (s.group) {
    case 1: return launch_qo<1>(s, a, c, stream);
    case 2: return launch_qo<2>(s, a, c, stream);
    case 4: return launch_qo<4>(s, a, c, stream);
    case 5: return launch_qo<5>(s, a, c, stream);
    case 8: return launch_qo<8>(s, a, c, stream);
    default: return hipErrorInvalidValue;
  }
}

int max_decode_splits(const Shape& s, const Workspace& ws, int batch) {
  const int64_t per = (int64_t)batch * s.n_heads;
  int64_t m = per > 0 ? ws.records / per : 0;
  if (m > 256) m = 256;
  return (int)m;
}

}  // namespace nwd
