// nwd_prefill.h — causal chunked-prefill attention on gfx950 fp16 MFMA: the
// kernel, its split merge and launchers, instantiated by nwd_prefill.hip
// (head size 128 and the padded sizes above 64) and nwd_prefill_d64.hip
// (head sizes up to 64).
//
//
// The reference has no prefill kernel: each prompt token runs the whole
// decode step (kv_append, then sparse_attn over keys 0..seq) one at a time
// (engine/runtime.js:640-643). The result of that loop is what this kernel
// computes in one launch: with the n_new new K/V rows already appended at
// tokens pos0 .. pos0+n_new-1, query i attends keys 0 .. pos0+i.
//
// GQA packing: for one KV head the G query heads of the group and the n_new
// queries form n_new*G rows (row R = query R/G, head R%G) that all share the
// same K/V stream. A workgroup (8 wavefronts) owns 128 consecutive rows and
// walks 128-key tiles. Wavefront w computes row group w%4 (32 rows, two
// 16-row MFMA blocks) against key half w/4 (64 keys) of each tile, as one
// 64-key online-softmax step: every K/V fragment read from LDS feeds two
// MFMAs, and two wavefronts share each SIMD. 128 rows per workgroup halve
// the K/V staging per flop against 64 (one tile copy serves twice the rows);
// the 64-key step gives each wavefront 8 independent QK^T accumulator chains
// and one max / rescale per 64 keys (85 us against 103 us for 64-row
// workgroups with 32-key steps, config 5).
//   - K and V rows go from memory straight into LDS (buffer_load_dwordx4
//     with the lds flag, gfx950: one instruction writes 1 KB, lane l's 16
//     bytes at +16l), double-buffered: the next tile's copies are issued
//     between the current tile's K fragment reads and land while it is
//     computed; one wait plus one barrier per tile publish them. Rows are
//     unpadded (256 B at head size 128, 128 B at 64); the 16-byte chunks of
//     a row are XOR-swizzled by the row index so the MFMA operand reads hit
//     distinct banks (each lane fetches the chunk its LDS slot must hold);
//   - S^T = K Q^T on v_mfma_f32_16x16x32_f16 (K from LDS as the A operand,
//     all 16 fragments of a tile read before its MFMAs, the query rows held
//     in registers as the B operand), so each lane holds 4 consecutive keys
//     of ONE row — its own softmax row;
//   - causal mask only on tiles that cross a row's limit; online softmax in
//     log2 units: fp16 query rows enter the MFMAs exact and each score is
//     scaled by scale * log2(e) and moved by -m in one FMA; fp32 rows are
//     pre-scaled and split into fp16 high and low parts (two QK^T MFMAs,
//     the low parts read from LDS) that accumulate onto -m, so each weight
//     is one v_exp of an MFMA output (the softmax's VALU work hides only
//     partly behind the MFMAs, so VALU instructions per score are what the
//     loop minimises); the row
//     maximum is taken only for a row's first keys and when a weight
//     overflows fp16 (seen as an infinite row sum), and the reference point
//     m then moves lazily (only when the row maximum exceeds it by more
//     than 8), so the common tile costs one v_exp per score and the
//     33-multiply rescale of a row block is rare; the row sum is taken over
//     the fp16 weights the PV product uses (v_dot2 with ones, two weights
//     per instruction);
//   - O^T += V^T P^T on the same MFMA, where P^T (fp16) is built in
//     registers from the S^T accumulators with no data movement between
//     lanes, and V^T is read from the row-major V tile with two
//     ds_read_b64_tr_b16 transpose loads per operand (gfx950), all of a
//     tile's requested before its softmax: within a 16-lane group, output
//     lane j element e comes from position j%4 of the 8 bytes lane
//     4e + j/4 addresses, so lanes 4e..4e+3 addressing 16 consecutive dims
//     of key row e give lane j V[key_e][d0 + j];
//   - the two key halves of a row group are merged through LDS at the end;
//     accumulation is fp32 throughout.
// With fewer than 256 row tiles, each row tile's key range is split over
// nsplit workgroups (the decode kernel's split-K): they write (max, sum, o)
// records to the context's workspace (o / sum in fp16 when the output is
// fp16, o in fp32 otherwise), and prefill_merge_kernel combines them; with
// one split the workgroup writes O directly.
// Head size 64 has a form of its own (prefill_d64_kernel): 128-byte rows,
// half the MFMAs and LDS reads per key (the softmax's work per score is the
// same). Other head sizes below 128 (multiples of 8) run the kernel of the
// next of 64 and 128 on rows padded with zeros to its dims
// (prefill_pad_kernel, prefill_d64_kernel with kPadD): the query's and the
// K/V rows' missing 16-byte chunks read as zeros (the copies' offsets pushed
// past the buffer range), so the scores are those of the real dims, the
// padded dims of O come out zero and are not stored.
#pragma once

#include <atomic>

#include "nwd_common.h"
#include "nwd_internal.h"

namespace nwd {

constexpr int kPWaves = 8;
constexpr int kPThreads = kPWaves * 64;
constexpr int kPBM = 128;                   // rows per workgroup
constexpr int kPBN = 128;                   // keys per tile
constexpr int kRB = 2;                      // 16-row MFMA blocks per wavefront
constexpr int kKB = 4;                      // 16-key blocks per wavefront per tile
constexpr float kPSlack = 8.f;              // lazy-rescale slack, log2 units
// Head size 128 (the kernel body takes these from PRow<kD> below):
constexpr int kRowBytes = kHeadDim * 2;     // 256: K/V rows are unpadded in LDS
constexpr int kTileBytes = kPBN * kRowBytes;  // 32 KB
constexpr int kStageInsts = kTileBytes / (kPWaves * 1024);  // 1 KB per wave per load (4)
static_assert(4 * kStageInsts == 4 * kKB, "a tile's K and V copies fit one per two QK^T MFMA steps");
// Chunk swizzles (16 chunks of 16 bytes per row): physical chunk p of LDS
// row r holds logical chunk p ^ kswz(r) of a K row, p ^ vswz(r) of a V row.
// A K operand read (16 rows, one logical chunk) then covers 16 distinct
// chunks, and a transpose read (4 rows x 2 chunks per 16 lanes) 8.
__device__ inline int kswz(int r) { return r & 15; }
__device__ inline int vswz(int r) { return (r & 7) << 1; }
// The same for head size kD (128 or 64). A head-64 row is 128 bytes (8
// chunks), two rows per 256 bytes, so the swizzles take the row index
// halved: the 16 rows of a K operand read still cover 16 distinct 16-byte
// slots of 256 bytes, and the 4 rows of a transpose read 4 distinct chunk
// pairs in those slots.
template <int kD>
struct PRow {
  static constexpr int kBytes = kD * 2;                      // LDS row (unpadded)
  static constexpr int kChunks = kD / 8;                     // 16-byte chunks per row
  static constexpr int kTile = kPBN * kBytes;                // one K or V tile
  static constexpr int kStage = kTile / (kPWaves * 1024);    // 1 KB copies per wave per tile
  static constexpr int kCopyRows = 1024 / kBytes;            // rows per copy
  static constexpr int kDB = kD / 32;                        // 32-dim QK^T steps
  static constexpr int kDBlk = kD / 16;                      // 16-dim blocks of O
};
template <int kD>
__device__ inline int kswz_d(int r) { return kD == kHeadDim ? kswz(r) : (r >> 1) & 7; }
template <int kD>
__device__ inline int vswz_d(int r) { return kD == kHeadDim ? vswz(r) : ((r >> 1) & 3) << 1; }
// Eight query elements as MFMA operands. fp16 queries are taken as they are
// (exact; the scale is applied to the fp32 scores). fp32 queries are scaled
// by s: `hi` is the product rounded to fp16 and `lo` the rounding error
// (x - hi, rounded to fp16), so hi + lo carries ~22 bits of the scaled
// query and the MFMAs leave the scores in log2 units. `range` is set when a
// scaled fp32 element leaves the fp16 range (its hi is then +-inf).
template <bool kQ16>
__device__ inline void load_q8(const void* q, int64_t elem, float s, f16x8& hi, f16x8& lo,
                               bool& range) {
  if constexpr (kQ16) {
    hi = *reinterpret_cast<const f16x8*>(static_cast<const f16*>(q) + elem);
  } else {
    const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(q) + elem);
    const f32x4 a = p[0], b = p[1];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = (e < 4 ? a[e] : b[e - 4]) * s;
      hi[e] = (f16)x;
      lo[e] = (f16)(x - (float)hi[e]);
      range |= fabsf(x) > 65504.f;
    }
  }
}

template <bool kO16>
__device__ inline void store_o4(void* out, int64_t at, f32x4 r) {
  if constexpr (kO16) {
    f16x4 h;
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = (f16)r[e];
    *reinterpret_cast<f16x4*>(static_cast<f16*>(out) + at) = h;
  } else {
    *reinterpret_cast<f32x4*>(static_cast<float*>(out) + at) = r;
  }
}

struct PrefillArgs {
  const void* q;
  const f16* k_cache;
  const f16* v_cache;
  const int32_t* pos0;
  void* out;
  float* part_o;    // [rows][nsplit][D] (nsplit > 1)
  float2* part_ml;  // [rows][nsplit] (max in log2 units, sum)
  int64_t records;  // capacity of part_o / part_ml in records
  int batch, n_heads, n_kv, cap, n_new, mtiles, nsplit;
  float qk_scale_log2;
  int* status;
  int head_dim;     // D (prefill_pad_kernel; 128 in prefill_kernel)
  int kv_rep;       // groups of G query heads per KV head (n_kv counts the groups)
};

// LDS of a workgroup: K0 K1 V0 V1 tiles, 32 KB each at head size 128 (16 KB
// at 64); with fp32 queries also the low halves of the workgroup's 128 query
// rows (one more tile's size, rows swizzled as K rows), which do not fit the
// registers beside the high halves.
template <bool kQ16, int kD = kHeadDim>
constexpr size_t prefill_lds_bytes() { return (size_t)(kQ16 ? 4 : 5) * PRow<kD>::kTile; }

// The body of prefill_kernel (kPadD false: D = 128), prefill_pad_kernel
// (kPadD: D = a.head_dim, a multiple of 8 below 128, rows padded to 128) and
// prefill_d64_kernel (kD = 64: D = 64, or with kPadD a multiple of 8 below
// it, rows padded to 64).
template <int G, bool kQ16, bool kO16, bool kPadD, int kD = kHeadDim>
__device__ __forceinline__ void prefill_body(const PrefillArgs a) {
  extern __shared__ __attribute__((aligned(16))) f16 smem[];
  char* lds = reinterpret_cast<char*>(smem);
  const int D = kPadD ? a.head_dim : kD;
  constexpr int kRowBytes = PRow<kD>::kBytes;
  constexpr int kTileBytes = PRow<kD>::kTile;
  constexpr int kStageInsts = PRow<kD>::kStage;
  constexpr int kQloOffset = 4 * kTileBytes;
  constexpr int kDB = PRow<kD>::kDB, kDBlk = PRow<kD>::kDBlk;
  static_assert(kDB * kKB == 4 * kStageInsts, "a tile's K and V copies fit one per two QK^T MFMA steps");

  const int id = blockIdx.x;
  const int hkv = id % a.n_kv;
  int rest = id / a.n_kv;
  const int split = rest % a.nsplit;
  rest /= a.nsplit;
  const int mt = rest % a.mtiles;
  const int b = rest / a.mtiles;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, lq = lane >> 4;
  const int rh = wave & 3, kh = wave >> 2;  // row group (32 rows), key half (64 keys)

  int P0 = a.pos0[b];
  if (P0 < 0 || P0 > a.cap - a.n_new) {
    if (tid == 0 && mt == 0 && hkv == 0 && split == 0) atomicOr(a.status, kStatusBadPos);
    P0 = P0 < 0 ? 0 : a.cap - a.n_new;
  }
  const int total_rows = a.n_new * G;
  const int r_last = min(mt * kPBM + kPBM, total_rows) - 1;
  const int kend = P0 + r_last / G + 1;  // keys this row tile needs
  const int ntiles_all = (kend + kPBN - 1) / kPBN;
  const int t0 = (int)((int64_t)split * ntiles_all / a.nsplit);
  const int t1 = (int)((int64_t)(split + 1) * ntiles_all / a.nsplit);
  const int kend_s = min(kend, t1 * kPBN);  // keys this split may load

  // Query rows in registers. fp32 rows are pre-scaled by scale * log2(e)
  // (the scores come out of the MFMAs in log2 units), and the key-half-0
  // wavefront of each row group writes their low halves to LDS (published by
  // the barrier before the first tile); fp16 rows stay exact and their
  // scores are scaled after the MFMAs.
  const float c = a.qk_scale_log2;
  const int r0 = mt * kPBM + rh * 32;
  int qi[kRB], gq[kRB], lim[kRB];
  f16x8 qf[kRB][kDB];
  char* const qlo = lds + kQloOffset;
  // LDS address of the low half of row block rb's fragment db (row rh*32 +
  // rb*16 + lr of the workgroup, logical chunk 4 db + lq, K's swizzle)
  auto qlo_at = [&](int rb, int db) {
    return qlo + (rh * 32 + rb * 16 + lr) * kRowBytes + (((4 * db + lq) ^ kswz_d<kD>(lr)) << 4);
  };
  bool q_range = false;
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    const int R = r0 + rb * 16 + lr;
    const bool ok = R < total_rows;
    qi[rb] = ok ? R / G : 0;
    gq[rb] = ok ? R - qi[rb] * G : 0;
    lim[rb] = ok ? P0 + qi[rb] : -1;
    const int64_t qrow = (((int64_t)b * a.n_new + qi[rb]) * a.n_heads + hkv * G + gq[rb]) * D;
#pragma unroll
    for (int db = 0; db < kDB; ++db) {
      f16x8 lo{};
      if (ok && (!kPadD || db * 32 + 8 * lq < D)) {
        load_q8<kQ16>(a.q, qrow + db * 32 + 8 * lq, c, qf[rb][db], lo, q_range);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[rb][db][e] = (f16)0.f;
      }
      if constexpr (!kQ16) {
        if (kh == 0) *reinterpret_cast<f16x8*>(qlo_at(rb, db)) = lo;
      }
    }
  }
  if (q_range) atomicOr(a.status, kStatusQueryRange);
  const bool wave_has_pad = r0 + 31 >= total_rows;
  const int wave_min_lim = P0 + r0 / G;

  // The KV head this group of query heads reads (kv_rep groups per KV head).
  const int kv_m = a.kv_rep > 1 ? hkv / a.kv_rep : hkv;
  const int nkv_m = a.kv_rep > 1 ? a.n_kv / a.kv_rep : a.n_kv;
  const int64_t slab = (int64_t)(b * nkv_m + kv_m) * a.cap * D;
  const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(a.k_cache + slab), 0,
                                                    kend_s * (D * 2), kBufferWord3);
  const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(a.v_cache + slab), 0,
                                                    kend_s * (D * 2), kBufferWord3);
  // Staging: wave w copies rows 16w .. 16w+15 of a tile, 1 KB (4 rows at
  // head size 128, 8 at 64) per instruction: lane l fills physical chunk
  // l % chunks of row 16w + (rows per copy) i + l / chunks and so loads the
  // logical chunk the swizzle puts there. Rows past the
  // split's last key read as zeros (buffer range check), so no LDS row is
  // ever stale.
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const int st_row = 16 * wv + lane / PRow<kD>::kChunks, st_p = lane % PRow<kD>::kChunks;
  // Copy j of this wave's part of tile kt into buffer bb: j < kStageInsts
  // are K rows, the rest V rows. `oob` (0 or 2^31) pushes the offset past
  // the range, which makes the copy a no-op read of zeros.
  // With kPadD a row holds D * 2 bytes in memory, and the chunks at or past
  // it are pushed out of range too (they would read the next row).
  auto stage = [&](int kt, int bb, int j, uint32_t oob) {
    const int i = j % kStageInsts;
    const bool kpart = j < kStageInsts;
    const int row = st_row + PRow<kD>::kCopyRows * i;
    if constexpr (kPadD) {
      char* dst = lds + ((kpart ? 0 : 2) + bb) * kTileBytes + wv * 16 * kRowBytes + i * 1024;
      const int lc = st_p ^ (kpart ? kswz_d<kD>(row) : vswz_d<kD>(row));  // logical chunk
      const uint32_t off = ((uint32_t)(kt * kPBN + row) * (uint32_t)(D * 2) + (lc << 4)) |
                           (8 * lc >= D ? 0x80000000u : oob);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(kpart ? rk : rv, (lds_void*)dst, 16, off, 0, 0, 0);
    } else {
      const uint32_t rb_off = (uint32_t)(kt * kPBN + row) * kRowBytes + oob;
      char* dst = lds + ((kpart ? 0 : 2) + bb) * kTileBytes + wv * 16 * kRowBytes + i * 1024;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(kpart ? rk : rv, (lds_void*)dst, 16,
                                               rb_off + ((st_p ^ (kpart ? kswz_d<kD>(row) : vswz_d<kD>(row))) << 4),
                                               0, 0, 0);
    }
  };
  auto load_tile = [&](int kt, int bb) {
#pragma unroll
    for (int j = 0; j < 2 * kStageInsts; ++j) stage(kt, bb, j, 0u);
  };
  auto wait_tile = [&]() { __builtin_amdgcn_s_waitcnt(0x0F70); };  // vmcnt(0)

  // Per row (lane lr of each row block): the reference point m (log2
  // units; kNegBig until the row has seen a key), the sum of weights and
  // O^T, all relative to m.
  float m[kRB], lsum[kRB];
  f32x4 o[kRB][kDBlk];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    m[rb] = kNegBig;
    lsum[rb] = 0.f;
#pragma unroll
    for (int j = 0; j < kDBlk; ++j) o[rb][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  if (t1 > t0) load_tile(t0, 0);
  wait_tile();
  __syncthreads();  // the first tile and the query low halves are in LDS
  for (int kt = t0; kt < t1; ++kt) {
    const int buf = (kt - t0) & 1;
    const char* ks = lds + buf * kTileBytes + kh * 64 * kRowBytes;
    const char* vs = lds + (2 + buf) * kTileBytes + kh * 64 * kRowBytes;
    const int k0 = kt * kPBN + kh * 64;

    // st[kb][rb][e] = score(key k0 + kb*16 + 4*lq + e, row rb*16 + lr) - mu[rb]
    // in log2 units, mu being the row's reference point (0 before the row
    // has seen a key): fp32 rows' MFMAs accumulate onto -mu, fp16 rows'
    // scores q.k are scaled by c and moved by -mu in one FMA each.
    float mu[kRB];
    f32x4 c0[kRB], st[kKB][kRB];
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) {
      mu[rb] = m[rb] > kNegBig ? m[rb] : 0.f;
      const float init = kQ16 ? 0.f : -mu[rb];
      c0[rb] = f32x4{init, init, init, init};
    }
    // All 16 K fragments of this wavefront's 64 keys are read first (64
    // VGPRs), then the 32 MFMAs run on them: no MFMA waits on a read issued
    // just before it. Tile kt+1 is copied into the other buffer between the
    // reads, one copy per two: issued in one burst after the barrier, a
    // workgroup's 64 copies per tile queued at the address unit for ~680
    // cycles of every tile.
    const int nb = (kt + 1 - t0) & 1;
    const uint32_t oob = kt + 1 < t1 ? 0u : 0x80000000u;
    f16x8 kf[kDB][kKB];
#pragma unroll
    for (int db = 0; db < kDB; ++db) {
#pragma unroll
      for (int kb = 0; kb < kKB; ++kb) {
        if (((db * kKB + kb) & 1) == 0) stage(kt + 1, nb, (db * kKB + kb) >> 1, oob);
        kf[db][kb] = *reinterpret_cast<const f16x8*>(ks + (kb * 16 + lr) * kRowBytes +
                                                     (((4 * db + lq) ^ kswz_d<kD>(lr)) << 4));
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every read ahead of the MFMAs
#pragma unroll
    for (int db = 0; db < kDB; ++db) {
      f16x8 ql[kRB];
      if constexpr (!kQ16) {
#pragma unroll
        for (int rb = 0; rb < kRB; ++rb) ql[rb] = *reinterpret_cast<const f16x8*>(qlo_at(rb, db));
      }
#pragma unroll
      for (int kb = 0; kb < kKB; ++kb)
#pragma unroll
        for (int rb = 0; rb < kRB; ++rb) {
          st[kb][rb] = mfma16x16x32(kf[db][kb], qf[rb][db], db == 0 ? c0[rb] : st[kb][rb]);
          if constexpr (!kQ16) st[kb][rb] = mfma16x16x32(kf[db][kb], ql[rb], st[kb][rb]);
        }
    }
    if constexpr (kQ16) {
#pragma unroll
      for (int kb = 0; kb < kKB; ++kb)
#pragma unroll
        for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
          for (int e = 0; e < 4; ++e) st[kb][rb][e] = fmaf(st[kb][rb][e], c, -mu[rb]);
    }
    // The Vᵀ operands of this tile's PV product do not depend on the
    // softmax: all 16 (32 transpose reads) are requested now, and arrive
    // while the softmax runs.
    const int vr0 = 4 * lq + (lr >> 2);
    auto vaddr = [&](int r, int dblk) {
      return reinterpret_cast<const f16*>(vs + r * kRowBytes +
                                          (((2 * dblk + ((lr >> 1) & 1)) ^ vswz_d<kD>(r)) << 4) + 8 * (lr & 1));
    };
    f16x8 vf[2][kDBlk];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int dblk = 0; dblk < kDBlk; ++dblk) {
        const f16x4 lo = lds_read_tr16(vaddr(h * 32 + vr0, dblk));
        const f16x4 hi = lds_read_tr16(vaddr(h * 32 + 16 + vr0, dblk));
        vf[h][dblk] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    __builtin_amdgcn_sched_barrier(0);
    if (wave_has_pad || k0 + 63 > wave_min_lim) {
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
        for (int kb = 0; kb < kKB; ++kb)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (k0 + kb * 16 + 4 * lq + e > lim[rb]) st[kb][rb][e] = -INFINITY;
    }
    // P^T operands, two per row block: pb[rb][h] element e < 4 is key
    // k0 + 32h + 4*lq + e, e >= 4 is key k0 + 32h + 16 + 4*lq + (e-4).
    f16x8 pb[kRB][2];
    // Row maximum and lazy rescale of row block rb: m moves only when the
    // tile's row maximum exceeds it by more than kPSlack, and the scores are
    // then re-based onto the new m.
    auto rescale = [&](int rb) {
      float mx = st[0][rb][0];
#pragma unroll
      for (int kb = 0; kb < kKB; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) mx = fmaxf(mx, st[kb][rb][e]);
      const float ax = max_xor32(max_xor16(mx)) + mu[rb];
      if (ax > m[rb] + kPSlack) {
        const float alpha = fast_exp2(m[rb] - ax);
        lsum[rb] *= alpha;
#pragma unroll
        for (int j = 0; j < kDBlk; ++j) o[rb][j] *= alpha;
        m[rb] = ax;
        const float d = mu[rb] - ax;
#pragma unroll
        for (int kb = 0; kb < kKB; ++kb)
#pragma unroll
          for (int e = 0; e < 4; ++e) st[kb][rb][e] += d;
        mu[rb] = ax;
      }
    };
    // Weights of row block rb and their per-lane sum, taken over the fp16
    // values the PV product uses (v_dot2 with ones, two per instruction).
    auto weights = [&](int rb) {
#pragma unroll
      for (int kb = 0; kb < kKB; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) pb[rb][kb >> 1][(kb & 1) * 4 + e] = (f16)fast_exp2(st[kb][rb][e]);
      float ls = 0.f;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 8; e += 2)
          ls = dot2(f16x2{pb[rb][h][e], pb[rb][h][e + 1]}, f16x2{(f16)1.f, (f16)1.f}, ls);
      return ls;
    };
    // The row maximum is taken only where it is needed: for a row's first
    // keys (m is set from them, so the largest weight of a row is never
    // below 1) and when a weight overflowed fp16 (m lags the row maximum by
    // 16 or more: the tile's fp16 row sum is then +inf). Otherwise the
    // weights are exponentials of the MFMA outputs as they are: m stays
    // within 16 of the running maximum and every weight is below 2^16. Both
    // tests are taken over the whole wavefront, so the four lanes of a row
    // always take the path together.
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) {
      if (__builtin_amdgcn_ballot_w64(m[rb] == kNegBig && k0 <= lim[rb])) rescale(rb);
      float ls = weights(rb);
      if (__builtin_amdgcn_ballot_w64(__builtin_isinf(ls))) {
        rescale(rb);
        ls = weights(rb);
      }
      lsum[rb] += ls;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int dblk = 0; dblk < kDBlk; ++dblk)
#pragma unroll
        for (int rb = 0; rb < kRB; ++rb) o[rb][dblk] = mfma16x16x32(vf[h][dblk], pb[rb][h], o[rb][dblk]);

    wait_tile();      // this wave's part of tile kt+1 is in LDS
    __syncthreads();  // every part is, and every wave is done with tile kt
  }

  // Merge the two key halves of each row group through LDS: wave (rh, 1)
  // publishes (m, l, o); wave (rh, 0) combines and writes the output or
  // this split's records.
  constexpr int kX = 2 + 4 * kDBlk;
  float* xch = reinterpret_cast<float*>(smem);  // [4 row groups][64 lanes][kRB][kX]
  auto slot = [&](int rb) { return xch + ((rh * 64 + lane) * kRB + rb) * kX; };
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) lsum[rb] = sum_xor32(sum_xor16(lsum[rb]));
  __syncthreads();  // the last tile's LDS reads are done before xch is written
  if (kh == 1) {
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) {
      float* x = slot(rb);
      x[0] = m[rb];
      x[1] = lsum[rb];
#pragma unroll
      for (int j = 0; j < kDBlk; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) x[2 + j * 4 + e] = o[rb][j][e];
    }
  }
  __syncthreads();
  if (kh == 1) return;
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    const int R = r0 + rb * 16 + lr;
    if (R >= total_rows) continue;
    const float* x = slot(rb);
    const float M = fmaxf(m[rb], x[0]);
    const float a0 = fast_exp2(m[rb] - M), a1 = fast_exp2(x[0] - M);
    const float lt = lsum[rb] * a0 + x[1] * a1;
    const int64_t grow = ((int64_t)b * a.n_new + qi[rb]) * a.n_heads + hkv * G + gq[rb];
    const int64_t out_rows = (int64_t)a.batch * a.n_new * a.n_heads;
    if (!in_bounds(grow, 1, out_rows, a.status)) continue;
    if (a.nsplit == 1) {
      const float inv = 1.f / lt;
#pragma unroll
      for (int dblk = 0; dblk < kDBlk; ++dblk) {
        f32x4 r = o[rb][dblk] * a0;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = fmaf(x[2 + dblk * 4 + e], a1, r[e]);
        if (kPadD && dblk * 16 + 4 * lq >= D) continue;  // a padded dim
        store_o4<kO16>(a.out, grow * D + dblk * 16 + 4 * lq, r * inv);
      }
    } else {
      // This split's record: (M, lt) and o. With an fp16 output, o is
      // stored normalised (o / lt, bounded by the largest |V| entry) in
      // fp16: half the record bytes for one more rounding of the output's
      // own precision; with an fp32 output it stays unnormalised fp32.
      const int64_t rec = grow * a.nsplit + split;
      if (!in_bounds(rec, 1, a.records, a.status)) continue;
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
#pragma unroll
      for (int dblk = 0; dblk < kDBlk; ++dblk) {
        f32x4 r = o[rb][dblk] * a0;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = fmaf(x[2 + dblk * 4 + e], a1, r[e]);
        const int64_t at = rec * kHeadDim + dblk * 16 + 4 * lq;
        if constexpr (kO16) store_o4<true>(a.part_o, at, r * inv);
        else *reinterpret_cast<f32x4*>(a.part_o + at) = r;
      }
      if (lq == 0) a.part_ml[rec] = make_float2(M, lt);
    }
  }
}

template <int G, bool kQ16, bool kO16>
__global__ __launch_bounds__(kPThreads, 1) void prefill_kernel(const PrefillArgs a) {
  prefill_body<G, kQ16, kO16, false>(a);
}
template <int G, bool kQ16, bool kO16>
__global__ __launch_bounds__(kPThreads, 1) void prefill_pad_kernel(const PrefillArgs a) {
  prefill_body<G, kQ16, kO16, true>(a);
}
// Head size 64 (kPadD: the multiples of 8 below it, rows padded to 64): half
// the MFMA work and LDS traffic per key of the head-128 kernel on padded rows.
template <int G, bool kQ16, bool kO16, bool kPadD>
__global__ __launch_bounds__(kPThreads, 1) void prefill_d64_kernel(const PrefillArgs a) {
  prefill_body<G, kQ16, kO16, kPadD, 64>(a);
}

// out[row] = sum_s o_s 2^(m_s - M) / sum_s l_s 2^(m_s - M) over the
// row's split records, merged in one pass (online maximum) so every load is
// independent of the others; 32 threads per row, 4 dims each. With kO16 the
// records hold o_s / l_s in fp16 (see prefill_kernel) and are weighted by
// l_s 2^(m_s - M).
// Records hold 128 dims at every head size (zeros past D); the output rows
// hold D.
template <bool kO16, bool kPadD>
__device__ __forceinline__ void prefill_merge_body(const float* __restrict__ part_o,
                                                   const float2* __restrict__ part_ml,
                                                   void* __restrict__ out, int64_t rows, int nsplit,
                                                   int64_t records, int* status, int D) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = t >> 5;
  const int d4 = t & 31;
  if (row >= rows || (kPadD && d4 * 4 >= D)) return;
  if (!in_bounds(row * nsplit, nsplit, records, status)) return;
  float M = kNegBig, L = 0.f;
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int s = 0; s < nsplit; ++s) {
    const int64_t rec = row * nsplit + s;
    const float2 ml = part_ml[rec];
    f32x4 ov;
    if constexpr (kO16) {
      const f16x4 h = *reinterpret_cast<const f16x4*>(reinterpret_cast<const f16*>(part_o) +
                                                     rec * kHeadDim + d4 * 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) ov[e] = (float)h[e];
    } else {
      ov = *reinterpret_cast<const f32x4*>(part_o + rec * kHeadDim + d4 * 4);
    }
    const float Mn = fmaxf(M, ml.x);
    const float sc = fast_exp2(M - Mn);
    float w = fast_exp2(ml.x - Mn);
    if constexpr (kO16) {
      w *= ml.y;
      L = fmaf(L, sc, w);
    } else {
      L = fmaf(L, sc, ml.y * w);
    }
    acc = acc * sc + ov * w;
    M = Mn;
  }
  if (!in_bounds(row * D + d4 * 4, 4, rows * D, status)) return;
  store_o4<kO16>(out, row * D + d4 * 4, acc * (1.f / L));
}

template <bool kO16>
__global__ __launch_bounds__(256) void prefill_merge_kernel(const float* __restrict__ part_o,
                                                            const float2* __restrict__ part_ml,
                                                            void* __restrict__ out, int64_t rows,
                                                            int nsplit, int64_t records,
                                                            int* status) {
  prefill_merge_body<kO16, false>(part_o, part_ml, out, rows, nsplit, records, status, kHeadDim);
}
template <bool kO16>
__global__ __launch_bounds__(256) void prefill_merge_pad_kernel(
    const float* __restrict__ part_o, const float2* __restrict__ part_ml, void* __restrict__ out,
    int64_t rows, int nsplit, int64_t records, int* status, int D) {
  prefill_merge_body<kO16, true>(part_o, part_ml, out, rows, nsplit, records, status, D);
}

static_assert(prefill_lds_bytes<true>() >= (size_t)4 * 64 * kRB * 34 * sizeof(float),
              "merge exchange fits");
static_assert(prefill_lds_bytes<false>() <= 160 * 1024, "LDS of one gfx950 CU");
static_assert(prefill_lds_bytes<true, 64>() >= (size_t)4 * 64 * kRB * 18 * sizeof(float),
              "merge exchange fits at head size 64");

// Splits of each row tile's key range. The launch runs in waves of 256
// workgroups (one per CU), and a partial last wave costs a whole split's
// time, so the split count fills one wave (256 / row tiles splits), or two
// when one wave would hold a single split per row tile and the row tiles
// are long (48+ key tiles); at most 16, at least 3 key tiles per split, and
// as many as the workspace holds records for. Same box, us per call: 512
// tokens onto 8192 at 40q/8kv (160 row tiles), 98.5 with 3 splits (two
// waves) against 130.3 with 2 (the earlier rule, 320 workgroups) and 113.5
// with 1; 256 onto 16384 (80 row tiles), 89.6 with 3 against 127.0 with 4;
// 513 onto 1000 at 40q/8kv, 27.1 with 1 against 39.2 with 2; 128 onto 4096
// at 40q/8kv, 25.3 against 36.1; 512 onto 2048 at 40q/8kv, 37.2 with 1
// against 50.6 with 2 and 43.9 with 3; config 5 (128 row tiles) keeps 2,
// 74.5 (81.3 with 4).
static int prefill_splits(int64_t row_tiles, int64_t rows, int max_len, const Workspace& ws) {
  const int64_t key_tiles = (max_len + kPBN - 1) / kPBN;
  int64_t n = 256 / row_tiles;
  if (n <= 1 && row_tiles > 128 && key_tiles >= 48) n = 512 / row_tiles;
  if (n > 16) n = 16;
  if (n > key_tiles / 3) n = key_tiles / 3;
  while (n > 1 && rows * n > ws.records) --n;
  return n < 1 ? 1 : (int)n;
}

// The kernel of a form, chosen at compile time so that a launcher
// instantiates only its own kernel.
template <int G, bool kQ16, bool kO16, bool kPadD, int kD>
constexpr auto prefill_kernel_for() {
  if constexpr (kD == 64) return prefill_d64_kernel<G, kQ16, kO16, kPadD>;
  else if constexpr (kPadD) return prefill_pad_kernel<G, kQ16, kO16>;
  else return prefill_kernel<G, kQ16, kO16>;
}

template <int G, bool kQ16, bool kO16, bool kPadD, int kD = kHeadDim>
static hipError_t launch_prefill_t(const Shape& s, const void* q, const void* kc, const void* vc,
                                   const int32_t* pos0, void* out, int batch, int n_new,
                                   int max_len, const Workspace& ws, int kv_rep,
                                   hipStream_t stream) {
  auto kern = prefill_kernel_for<G, kQ16, kO16, kPadD, kD>();
  constexpr size_t kPrefillLds = prefill_lds_bytes<kQ16, kD>();
  // The dynamic LDS size exceeds the 64 KB default: raise the kernel's limit
  // once per device (the attribute is per device).
  static std::atomic<uint64_t> attr_set{0};
  int dev = 0;
  hipError_t de = hipGetDevice(&dev);
  if (de != hipSuccess) return de;
  const uint64_t bit = 1ull << (dev & 63);
  if (!(attr_set.load() & bit)) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPrefillLds);
    if (e != hipSuccess) return e;
    attr_set.fetch_or(bit);
  }
  PrefillArgs a;
  a.q = q;
  a.k_cache = static_cast<const f16*>(kc);
  a.v_cache = static_cast<const f16*>(vc);
  a.pos0 = pos0;
  a.out = out;
  a.n_heads = s.n_heads;
  a.n_kv = s.n_kv;
  a.cap = s.cap;
  a.n_new = n_new;
  a.mtiles = (n_new * G + kPBM - 1) / kPBM;
  a.qk_scale_log2 = s.qk_scale * kLog2e;
  a.status = ws.status;
  a.head_dim = s.head_dim;
  a.kv_rep = kv_rep;
  const int64_t row_tiles = (int64_t)a.mtiles * s.n_kv * batch;
  const int64_t rows = (int64_t)n_new * s.n_heads * batch;
  const int nsplit = prefill_splits(row_tiles, rows, max_len, ws);
  a.nsplit = nsplit;
  a.part_o = ws.part_o;
  a.part_ml = ws.part_ml;
  a.records = ws.records;
  a.batch = batch;
  kern<<<(unsigned)(row_tiles * nsplit), kPThreads, kPrefillLds, stream>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || nsplit == 1) return e;
  const unsigned blocks = (unsigned)((rows * 32 + 255) / 256);
  if constexpr (kPadD || kD != kHeadDim)  // records of 128 floats, D of them used
    prefill_merge_pad_kernel<kO16><<<blocks, 256, 0, stream>>>(ws.part_o, ws.part_ml, out, rows,
                                                                nsplit, ws.records, ws.status,
                                                                s.head_dim);
  else
    prefill_merge_kernel<kO16><<<blocks, 256, 0, stream>>>(ws.part_o, ws.part_ml, out, rows, nsplit,
                                                           ws.records, ws.status);
  return hipGetLastError();
}

template <int G, bool kPadD, int kD = kHeadDim>
static hipError_t launch_prefill_p(const Shape& s, const void* q, const void* kc, const void* vc,
                                   const int32_t* pos0, void* out, int batch, int n_new,
                                   int max_len, const Workspace& ws, int r, hipStream_t stream) {
  if (s.q16)
    return s.o16 ? launch_prefill_t<G, true, true, kPadD, kD>(s, q, kc, vc, pos0, out, batch, n_new, max_len, ws, r, stream)
                 : launch_prefill_t<G, true, false, kPadD, kD>(s, q, kc, vc, pos0, out, batch, n_new, max_len, ws, r, stream);
  return s.o16 ? launch_prefill_t<G, false, true, kPadD, kD>(s, q, kc, vc, pos0, out, batch, n_new, max_len, ws, r, stream)
               : launch_prefill_t<G, false, false, kPadD, kD>(s, q, kc, vc, pos0, out, batch, n_new, max_len, ws, r, stream);
}

// Prefill at head sizes up to 64 (nwd_prefill_d64.hip).
hipError_t launch_prefill_d64(const Shape& s, const void* q, const void* k_cache,
                              const void* v_cache, const int32_t* pos0, void* out, int batch,
                              int n_new, int max_len, const Workspace& ws, int kv_rep,
                              hipStream_t stream);

}  // namespace nwd
