// nwd_decode_mfma.h — the matrix-core split workgroup of decode
// (decode_mfma_kernel, and decode_mfma_d64_kernel at head size 64), its
// launcher and the kernel choice at head sizes 128 and 64, shared by
// nwd_decode.hip (groups 1, 2, 4, 5, 8 at 128), nwd_decode_groups.hip
// (groups 3, 6, 7) and nwd_decode_mfma64.hip (head size 64), which
// instantiate disjoint sets of it.
#pragma once

#include <atomic>

#include "nwd_decode.h"

namespace nwd {

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

// The workgroup's shape at head size kD: 128, or 64 (128-byte rows: half
// the K fragments, V copies and O blocks per block, and more blocks in
// flight per wavefront for the same bytes). The head-64 V rows take the
// chunk swizzle of the head-64 prefill: the row index halved, so the 4 rows
// of a transpose read (two per 256 bytes) still hit distinct chunk pairs.
constexpr int kMDepth64 = 4;
template <int kD>
struct MShape {
  static constexpr int kSlot = kMWaveKeys * kD * 2;             // one V block
  static constexpr int kDepth = kD == kHeadDim ? kMDepth : kMDepth64;
  static constexpr int kLoads = kD / 32 + kSlot / 1024;         // K fragments + V copies
  static constexpr size_t kLds = (size_t)kMWaves * kDepth * kSlot;
  static constexpr int kChunks = kD / 8;                        // 16-byte chunks per row
  static constexpr int kCopyRows = 1024 / (kD * 2);             // rows per V copy
};
static_assert(MShape<64>::kLoads * (MShape<64>::kDepth - 1) <= 63, "vmcnt counts at most 63 loads");
template <int kD>
__device__ inline int vswz_md(int r) { return kD == kHeadDim ? vswz_m(r) : ((r >> 1) & 3) << 1; }

// s_waitcnt vmcnt(n) that the compiler keeps in place: memory accesses do
// not move across it.
template <int n>
__device__ inline void wait_vm_keep() {
  static_assert(n == 0 || n == 8 || n == 12, "instantiated counts");
  if constexpr (n == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if constexpr (n == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  if constexpr (n == 12) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
}
__device__ inline void compiler_fence() { asm volatile("" ::: "memory"); }

template <int G, bool kQ16, bool kO16, int kD>
__device__ __forceinline__ void decode_mfma_body(const DecodeArgs a) {
  constexpr int kMSlotBytes = MShape<kD>::kSlot, kMDepth = MShape<kD>::kDepth;
  constexpr int kMBlockLoads = MShape<kD>::kLoads;
  constexpr int kChunks = MShape<kD>::kChunks, kCopyRows = MShape<kD>::kCopyRows;
  constexpr int kDB = kD / 32, kDBlk = kD / 16;
  static_assert(G <= 16, "the heads of a group are the MFMA's 16 columns");
  static_assert(G * 32 <= kMThreads, "one 4-dim run of each head per thread");
  static_assert((size_t)kMWaves * G * (kD + 2) * 4 <= MShape<kD>::kLds,
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
  const int64_t slab = (int64_t)(b * nkv_m + kv_m) * a.cap * kD;
  auto slab_rsrc = [&](f16* cache, int end_key) {
    return __builtin_amdgcn_make_buffer_rsrc(cache + slab, 0, end_key * (kD * 2),
                                             kBufferWord3);
  };
  char* const ring = lds + wave * (kMDepth * kMSlotBytes);

  struct KFrag {
    f16x8 k[kDB];  // [32-dim block]
  };
  auto load_k = [&](KFrag& f, const __amdgpu_buffer_rsrc_t rk, int it) {
    const int key0 = t0 + it * it_keys + wave * kMWaveKeys;
#pragma unroll
    for (int db = 0; db < kDB; ++db) {
      const uint32_t off = (uint32_t)(key0 + lr) * (kD * 2) + db * 64 + lq * 16;
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
      const int row = kCopyRows * i + (kD == kHeadDim ? lq : lane / kChunks);
      const int pc = kD == kHeadDim ? lr : lane % kChunks;  // physical chunk
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rv, (lds_void*)(dst + i * 1024), 16,
          (uint32_t)(key0 + row) * (kD * 2) + ((pc ^ vswz_md<kD>(row)) << 4), 0, 0,
          kStreamPolicy);
    }
  };

  // Fused append: the new rows are requested first (the K chunks this
  // lane's fragments hold, and V logical chunk lr), before the position
  // says which split owns them.
  const bool has_new = a.k_new != nullptr;
  SrcRun nk_raw[kDB], nv_raw;
  if (has_new) {
    const int64_t src = (int64_t)(b * nkv_m + kv_m) * kD;
#pragma unroll
    for (int db = 0; db < kDB; ++db) nk_raw[db] = load_src_run_raw(a.k_new, src + db * 32 + 8 * lq, a.new16);
    nv_raw = load_src_run_raw(a.v_new, src + 8 * (kD == kHeadDim ? lr : lr % kChunks), a.new16);
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
  f16x8 qh[kDB], ql[kQ16 ? 1 : kDB];
  bool q_range = false;
  {
    const bool qv = lr < G;
    const int64_t qrow = ((int64_t)b * a.n_heads + h0 + (qv ? lr : 0)) * kD + 8 * lq;
#pragma unroll
    for (int db = 0; db < kDB; ++db) {
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
  f16x8 nk[kDB], nv;
  if (owns_new) {
#pragma unroll
    for (int db = 0; db < kDB; ++db) nk[db] = convert_src_run(nk_raw[db], a.new16);
    nv = convert_src_run(nv_raw, a.new16);
    // K chunks 4 db + lq from the lanes of key row 0, V chunk lr from lane
    // group 0
    if (wave == w_new && kv_m * a.kv_rep == hkv) {
      const int64_t at = slab + (int64_t)pnew * kD;
      const int64_t cache_elems = (int64_t)a.batch * nkv_m * a.cap * kD;
      if (lr == 0) {
#pragma unroll
        for (int db = 0; db < kDB; ++db) {
          const int64_t e = at + db * 32 + 8 * lq;
          if (in_bounds(e, 8, cache_elems, a.status)) *reinterpret_cast<f16x8*>(a.k_cache + e) = nk[db];
        }
      }
      if (lq == 0 && lr < kChunks && in_bounds(at + 8 * lr, 8, cache_elems, a.status))
        *reinterpret_cast<f16x8*>(a.v_cache + at + 8 * lr) = nv;
    }
  }

  const float c = a.qk_scale_log2;
  float m = kNegBig, lsum = 0.f;  // head lr: reference point (log2 units), sum of weights
  f32x4 o[kDBlk];                 // O^T: dims 16 dblk + 4 lq .. +4 of head lr
#pragma unroll
  for (int d = 0; d < kDBlk; ++d) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](KFrag& f, int it, int slot) {
    wait_vm_keep<kMBlockLoads * (kMDepth - 1)>();  // block it's K fragments and V rows are in
    const int key0 = t0 + it * it_keys + wave * kMWaveKeys;
    if (key0 >= t1) return;  // nothing of this block is attended
    char* vs = ring + slot * kMSlotBytes;
    const bool partial = key0 + kMWaveKeys > t1;
    if (it == it_new && wave == w_new) {
      const bool sub = lr == r_new;
#pragma unroll
      for (int db = 0; db < kDB; ++db) f.k[db] = sub ? nk[db] : f.k[db];
      if (lq == 0 && lr < kChunks)
        *reinterpret_cast<f16x8*>(vs + r_new * (kD * 2) + ((lr ^ vswz_md<kD>(r_new)) << 4)) = nv;
    }
    if (partial) {
      // Rows at or past t1: zeros past the descriptor's end, or stale cache
      // rows in the blocks requested before the position was known; a stale
      // Inf or NaN times a zero weight would be NaN, so they are zeroed.
#pragma unroll
      for (int i = 0; i < kMSlotBytes / 1024; ++i) {
        const int row = kCopyRows * i + (kD == kHeadDim ? lq : lane / kChunks);
        const int pc = kD == kHeadDim ? lr : lane % kChunks;
        if (key0 + row >= t1)
          *reinterpret_cast<u32x4*>(vs + row * (kD * 2) + (pc << 4)) = u32x4{0u, 0u, 0u, 0u};
      }
    }
    // S^T: s[e] = q . k for key key0 + 4 lq + e, head lr.
    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int db = 0; db < kDB; ++db) {
      s = mfma16x16x32(f.k[db], qh[db], s);
      if constexpr (!kQ16) s = mfma16x16x32(f.k[db], ql[db], s);
    }
    // V^T operands (dims 16 dblk + lr, keys 4 lq + e), requested before the
    // softmax: the A operands of v_mfma_f32_16x16x16_f16, whose B operand
    // layout (keys 4 lq .. 4 lq + 3 of column lr) is that of S^T, so the
    // weights need no data movement between lanes.
    const int vr0 = 4 * lq + (lr >> 2);
    f16x4 vf[kDBlk];
#pragma unroll
    for (int dblk = 0; dblk < kDBlk; ++dblk)
      vf[dblk] = lds_read_tr16_asm(vs + vr0 * (kD * 2) +
                                   (((2 * dblk + ((lr >> 1) & 1)) ^ vswz_md<kD>(vr0)) << 4) + 8 * (lr & 1));
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
        for (int d = 0; d < kDBlk; ++d) o[d] *= al;
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
    for (int dblk = 0; dblk < kDBlk; ++dblk) {
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
  float* lds_ml = lds_o + kMWaves * G * kD;
  if (lr < G) {
#pragma unroll
    for (int dblk = 0; dblk < kDBlk; ++dblk)
      *reinterpret_cast<f32x4*>(&lds_o[(wave * G + lr) * kD + dblk * 16 + 4 * lq]) = o[dblk];
    if (lq == 0) {
      lds_ml[(wave * G + lr) * 2] = m;
      lds_ml[(wave * G + lr) * 2 + 1] = lsum;
    }
  }
  __syncthreads();
  const int64_t hrow0 = (int64_t)b * a.n_heads + h0;
  store_split_states<G, kO16, kMWaves, kD>(a, lds_o, lds_ml, hrow0, split);
  if (nsplit == 1 || !a.fused_merge) return;
  merge_on_last_arrival<G, kO16, kD>(a, a.counters + b * a.n_kv + hkv, hrow0);
}

template <int G, bool kQ16, bool kO16>
__global__ __launch_bounds__(kMThreads, 1) void decode_mfma_kernel(const DecodeArgs a) {
  decode_mfma_body<G, kQ16, kO16, kHeadDim>(a);
}
// Head size 64 (nwd_decode_mfma64.hip).
template <int G, bool kQ16, bool kO16>
__global__ __launch_bounds__(kMThreads, 1) void decode_mfma_d64_kernel(const DecodeArgs a) {
  decode_mfma_body<G, kQ16, kO16, 64>(a);
}

template <int G, bool kQ16, bool kO16, int kD = kHeadDim>
static hipError_t launch_mfma_t(const DecodeArgs& a, int batch, hipStream_t stream, void* ev_start,
                                void* ev_stop) {
  constexpr size_t kMLdsBytes = MShape<kD>::kLds;
  auto kern = [] {
    if constexpr (kD == kHeadDim) return decode_mfma_kernel<G, kQ16, kO16>;
    else return decode_mfma_d64_kernel<G, kQ16, kO16>;
  }();
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
  if constexpr (kD == kHeadDim)
    decode_merge_kernel<kO16><<<dim3((unsigned)a.n_heads, (unsigned)batch), 64, 0, stream>>>(
        a.part_o, a.part_ml, a.out, a.n_heads, a.nsplit, a.records, a.status);
  else
    decode_merge_hd_kernel<kO16, kD><<<dim3((unsigned)a.n_heads, (unsigned)batch), 64, 0, stream>>>(
        a.part_o, a.part_ml, a.out, a.n_heads, a.nsplit, a.records, a.status);
  return hipGetLastError();
}

template <int G, int kD = kHeadDim>
static hipError_t launch_mfma(const Shape& s, const DecodeArgs& a, const DecodeCall& c,
                              hipStream_t st) {
  const int B = c.batch;
  if (s.q16)
    return s.o16 ? launch_mfma_t<G, true, true, kD>(a, B, st, c.ev_start, c.ev_stop)
                 : launch_mfma_t<G, true, false, kD>(a, B, st, c.ev_start, c.ev_stop);
  return s.o16 ? launch_mfma_t<G, false, true, kD>(a, B, st, c.ev_start, c.ev_stop)
               : launch_mfma_t<G, false, false, kD>(a, B, st, c.ev_start, c.ev_stop);
}

// The matrix-core kernel at head size 64, groups 1 to 8 (nwd_decode_mfma64.hip).
hipError_t launch_mfma_d64(const Shape& s, const DecodeArgs& a, const DecodeCall& c,
                           hipStream_t stream);

// Kernel choice at head size 128 for groups of G query heads per KV head.
// When one workgroup per (sequence, query head, split) fits the chip, each
// query head gets its own workgroups: a workgroup's time is its serial
// chain of key iterations, whose compute grows with the heads it serves,
// and the G-fold K/V reads are small at the lengths the split rule sends
// here (per append + attend step, B = 1, G = 4: 4.5 against 6.3 us at 153
// keys with one split; 6.1 against 8.1 at 832 keys and 6.8 against 8.3 at
// 1088 with 8 splits). Same bits.
// One workgroup per KV head: the matrix-core kernel where it measured
// faster (see decode_mfma_kernel): G >= 5; G = 4 with a batch, or with long
// splits (at least 512 keys each) whose workgroups all fit the chip at once
// (B = 1, 32q/8kv, append + attend per step, 16K / 24K / 32K keys: 16.2 /
// 20.6 / 25.1 against 16.8 / 21.1 / 26.2 us on N(0,1) K/V, and 16.2 / 20.7
// / 25.1 against 17.1 / 21.7 / 26.8 with 1% outliers, on two boxes; at 64K
// keys, 33 splits and 264 workgroups, 62.9 against 60.6). Groups up to 3
// keep the dot-product kernel (24q/8kv, B = 1, decode call: 24.4 against
// 25.9 us at 32K keys, 7.6 against 8.4 at 4K). nwd_set_decode_kernel forces
// either kernel. Head size 64 takes the same rule (decode calls, B = 1,
// dot-product against matrix-core kernel, us: 32q/8kv at 4K / 16K / 32K
// keys 7.2 / 10.7 / 17.9 against 7.7 / 10.5 / 15.6; 64q/8kv at 16K 14.6
// against 10.7; 40q/8kv 11.3 against 10.6; 16q/8kv 10.1 against 10.4;
// 14q/2kv at 32K 11.9 against 10.6).
inline bool prefer_mfma(int G, const Shape& s, const DecodeCall& c) {
  const bool long_splits = (int64_t)c.span >= 512LL * c.nsplit &&
                           (int64_t)c.batch * s.n_kv * c.nsplit <= kMOneWave;
  return c.kernel < 0 && (G >= 5 || (G == 4 && (c.batch >= 2 || long_splits)));
}

template <int G>
static hipError_t launch_decode_128(const Shape& s, const DecodeArgs& a, const DecodeCall& c,
                                    hipStream_t stream) {
  if (c.kernel == 1) return launch_mfma<G>(s, a, c, stream);
  if constexpr (G > 1) {  // group 1 is already one workgroup per query head
    if ((int64_t)c.batch * s.n_heads * a.nsplit <= kSubSplitMaxWorkgroups)
      return launch_qo<1, G>(s, a, c, stream);
  }
  if (prefer_mfma(G, s, c)) return launch_mfma<G>(s, a, c, stream);
  return launch_qo<G>(s, a, c, stream);
}

// Groups 3, 6 and 7 at head sizes 128 and 64 (nwd_decode_groups.hip).
hipError_t launch_decode_groups(const Shape& s, const DecodeArgs& a, const DecodeCall& c,
                                hipStream_t stream);

}  // namespace nwd
