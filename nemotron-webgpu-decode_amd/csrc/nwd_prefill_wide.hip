// nwd_prefill_wide.hip — causal chunked prefill at head size 256 (and the
// multiples of 8 between 128 and 256, rows padded to 256 dims) on gfx950
// fp16 MFMA.
//
// The contract is prefill_kernel's (nwd_prefill.hip): the n_new new K/V rows
// are in the caches at pos0 .. pos0 + n_new - 1 and query i attends keys
// 0 .. pos0 + i, the result of the reference's token-by-token prefill
// (engine/runtime.js:640-643) over sparse_attn.wgsl:31-114. The head-128
// kernel holds 32 rows per wavefront and its O accumulators for 128 dims;
// twice the dims do not fit its registers, so this kernel gives each
// wavefront 16 rows and all 64 keys of a tile:
//   - a workgroup (8 wavefronts) owns 128 consecutive GQA-packed rows (row
//     R = query R / G, head R % G of one KV head), wavefront w rows
//     16w .. 16w + 15, and walks 64-key tiles of K and V (32 KB each,
//     double-buffered: 128 KB of LDS), copied from memory straight into LDS
//     (buffer_load ... lds, 2 rows of 512 bytes per instruction), the next
//     tile's copies issued between the current tile's K fragment reads;
//   - S^T = K Q^T on v_mfma_f32_16x16x32_f16 (8 dim steps per 16-key
//     block), so each lane holds 4 consecutive keys of one row; the softmax
//     is prefill_kernel's (log2 units, row maximum only on a row's first
//     keys and on fp16 overflow, lazy rescale);
//   - O^T += V^T P^T in two 32-key steps of 16 dim blocks, V^T read with
//     ds_read_b64_tr_b16 transpose loads (the lane layout prefill_kernel
//     uses), P^T built in registers from the S^T accumulators;
//   - rows of K and V are 32 chunks of 16 bytes in LDS, XOR-swizzled by the
//     row index (K: c ^ (r & 15), V: c ^ ((r & 15) << 1)) so the operand and
//     transpose reads hit distinct banks.
// fp32 queries are scaled and carried as fp16 high and low parts in
// registers (two QK^T MFMAs per step), fp16 queries enter exact. With fewer
// than 256 row tiles the key range is split over workgroups that write
// (max, sum, o[256]) records, merged by prefill_wide_merge_kernel.
#include <atomic>

#include "nwd_common.h"
#include "nwd_internal.h"

namespace nwd {

namespace {

constexpr int kWD = 256;                       // head size of the layout
constexpr int kWWaves = 8;
constexpr int kWThreads = kWWaves * 64;
constexpr int kWBM = 128;                      // rows per workgroup (16 per wavefront)
constexpr int kWBN = 64;                       // keys per tile
constexpr int kWKB = kWBN / 16;                // 16-key blocks per tile (4)
constexpr int kWDB = kWD / 32;                 // 32-dim MFMA steps of QK^T (8)
constexpr int kWOB = kWD / 16;                 // 16-dim blocks of O (16)
constexpr int kWRowBytes = kWD * 2;            // 512
constexpr int kWTileBytes = kWBN * kWRowBytes;  // 32 KB
constexpr int kWStage = kWTileBytes / (kWWaves * 1024);  // copies per wavefront per tile (4)
constexpr size_t kWLds = 4 * (size_t)kWTileBytes;       // K0 K1 V0 V1
constexpr float kWSlack = 8.f;
static_assert(kWLds <= 160 * 1024, "LDS of one gfx950 CU");
static_assert(2 * kWStage * 4 == kWDB * kWKB, "one copy per four QK^T MFMA steps");

__device__ inline int wkswz(int r) { return r & 15; }
__device__ inline int wvswz(int r) { return (r & 15) << 1; }

struct WideArgs {
  const void* q;
  const f16* k_cache;
  const f16* v_cache;
  const int32_t* pos0;
  void* out;
  float* part_o;    // [rows][nsplit][256] (nsplit > 1)
  float2* part_ml;  // [rows][nsplit]
  int64_t records;
  int batch, n_heads, n_kv, cap, n_new, mtiles, nsplit;
  float qk_scale_log2;
  int* status;
  int head_dim;  // D of the rows in memory (256, or fewer in the padded form)
  int kv_rep;    // groups of G query heads per KV head (n_kv counts the groups)
};

template <bool kQ16>
__device__ inline void wide_load_q8(const void* q, int64_t elem, float s, f16x8& hi, f16x8& lo,
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
__device__ inline void wide_store_o4(void* out, int64_t at, f32x4 r) {
  if constexpr (kO16) {
    f16x4 h;
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = (f16)r[e];
    *reinterpret_cast<f16x4*>(static_cast<f16*>(out) + at) = h;
  } else {
    *reinterpret_cast<f32x4*>(static_cast<float*>(out) + at) = r;
  }
}

template <int G, bool kQ16, bool kO16, bool kPadD>
__global__ __launch_bounds__(kWThreads, 1) void prefill_wide_kernel(const WideArgs a) {
  extern __shared__ __attribute__((aligned(16))) f16 wsmem[];
  char* lds = reinterpret_cast<char*>(wsmem);
  const int D = kPadD ? a.head_dim : kWD;

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

  int P0 = a.pos0[b];
  if (P0 < 0 || P0 > a.cap - a.n_new) {
    if (tid == 0 && mt == 0 && hkv == 0 && split == 0) atomicOr(a.status, kStatusBadPos);
    P0 = P0 < 0 ? 0 : a.cap - a.n_new;
  }
  const int total_rows = a.n_new * G;
  const int r_last = min(mt * kWBM + kWBM, total_rows) - 1;
  const int kend = P0 + r_last / G + 1;  // keys this row tile needs
  const int ntiles_all = (kend + kWBN - 1) / kWBN;
  const int t0 = (int)((int64_t)split * ntiles_all / a.nsplit);
  const int t1 = (int)((int64_t)(split + 1) * ntiles_all / a.nsplit);
  const int kend_s = min(kend, t1 * kWBN);

  // This wavefront's 16 rows: lane lr's row R, its query and head.
  const float c = a.qk_scale_log2;
  const int r0 = mt * kWBM + wave * 16;
  const int R = r0 + lr;
  const bool row_ok = R < total_rows;
  const int qi = row_ok ? R / G : 0;
  const int gq = row_ok ? R - qi * G : 0;
  const int lim = row_ok ? P0 + qi : -1;
  const int64_t grow = ((int64_t)b * a.n_new + qi) * a.n_heads + hkv * G + gq;
  f16x8 qf[kWDB], ql[kQ16 ? 1 : kWDB];
  bool q_range = false;
#pragma unroll
  for (int db = 0; db < kWDB; ++db) {
    f16x8 lo{};
    if (row_ok && (!kPadD || db * 32 + 8 * lq < D)) {
      wide_load_q8<kQ16>(a.q, grow * D + db * 32 + 8 * lq, c, qf[db], lo, q_range);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[db][e] = (f16)0.f;
    }
    if constexpr (!kQ16) ql[db] = lo;
  }
  if (q_range) atomicOr(a.status, kStatusQueryRange);
  const bool wave_has_pad = r0 + 15 >= total_rows;
  const int wave_min_lim = P0 + r0 / G;

  const int kv_m = a.kv_rep > 1 ? hkv / a.kv_rep : hkv;
  const int nkv_m = a.kv_rep > 1 ? a.n_kv / a.kv_rep : a.n_kv;
  const int64_t slab = (int64_t)(b * nkv_m + kv_m) * a.cap * D;
  const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(a.k_cache + slab), 0,
                                                    kend_s * (D * 2), kBufferWord3);
  const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(a.v_cache + slab), 0,
                                                    kend_s * (D * 2), kBufferWord3);
  // Staging: wave w copies rows 8w .. 8w+7 of a tile, 2 rows (1 KB) per
  // instruction: lane l fills physical chunk l & 31 of row 8w + 2i + l/32
  // with the logical chunk the swizzle puts there. Rows past the split's
  // last key, and (padded form) chunks past a row's D dims, read as zeros.
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const int st_row = 8 * wv + (lane >> 5), st_p = lane & 31;
  auto stage = [&](int kt, int bb, int j, uint32_t oob) {
    const int i = j % kWStage;
    const bool kpart = j < kWStage;
    const int row = st_row + 2 * i;
    char* dst = lds + ((kpart ? 0 : 2) + bb) * kWTileBytes + wv * 8 * kWRowBytes + i * 1024;
    const int lc = st_p ^ (kpart ? wkswz(row) : wvswz(row));
    uint32_t off = (uint32_t)(kt * kWBN + row) * (uint32_t)(D * 2) + (lc << 4);
    if (kPadD && 8 * lc >= D) off |= 0x80000000u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(kpart ? rk : rv, (lds_void*)dst, 16, off | oob, 0, 0,
                                             0);
  };
  auto wait_tile = [&]() { __builtin_amdgcn_s_waitcnt(0x0F70); };  // vmcnt(0)

  float m = kNegBig, lsum = 0.f;
  f32x4 o[kWOB];
#pragma unroll
  for (int j = 0; j < kWOB; ++j) o[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (t1 > t0) {
#pragma unroll
    for (int j = 0; j < 2 * kWStage; ++j) stage(t0, 0, j, 0u);
  }
  wait_tile();
  __syncthreads();
  for (int kt = t0; kt < t1; ++kt) {
    const int buf = (kt - t0) & 1;
    const char* ks = lds + buf * kWTileBytes;
    const char* vs = lds + (2 + buf) * kWTileBytes;
    const int k0 = kt * kWBN;
    const float mu = m > kNegBig ? m : 0.f;
    const float init = kQ16 ? 0.f : -mu;
    f32x4 st[kWKB];
#pragma unroll
    for (int kb = 0; kb < kWKB; ++kb) st[kb] = f32x4{init, init, init, init};
    // QK^T, one 32-dim step at a time: the step's 4 K fragments are read,
    // then its MFMAs run; tile kt+1 is copied into the other buffer, one
    // copy per four steps.
    const int nb = (kt + 1 - t0) & 1;
    const uint32_t oob = kt + 1 < t1 ? 0u : 0x80000000u;
#pragma unroll
    for (int db = 0; db < kWDB; ++db) {
      f16x8 kf[kWKB];
#pragma unroll
      for (int kb = 0; kb < kWKB; ++kb) {
        if (((db * kWKB + kb) & 3) == 0) stage(kt + 1, nb, (db * kWKB + kb) >> 2, oob);
        kf[kb] = *reinterpret_cast<const f16x8*>(ks + (kb * 16 + lr) * kWRowBytes +
                                                 (((4 * db + lq) ^ lr) << 4));
      }
#pragma unroll
      for (int kb = 0; kb < kWKB; ++kb) {
        st[kb] = mfma16x16x32(kf[kb], qf[db], st[kb]);
        if constexpr (!kQ16) st[kb] = mfma16x16x32(kf[kb], ql[db], st[kb]);
      }
    }
    if constexpr (kQ16) {
#pragma unroll
      for (int kb = 0; kb < kWKB; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) st[kb][e] = fmaf(st[kb][e], c, -mu);
    }
    if (wave_has_pad || k0 + kWBN - 1 > wave_min_lim) {
#pragma unroll
      for (int kb = 0; kb < kWKB; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (k0 + kb * 16 + 4 * lq + e > lim) st[kb][e] = -INFINITY;
    }
    // P^T operands: pb[h] element e < 4 is key k0 + 32h + 4*lq + e, e >= 4
    // is key k0 + 32h + 16 + 4*lq + (e-4).
    f16x8 pb[2];
    float mcur = mu;
    auto rescale = [&]() {
      float mx = st[0][0];
#pragma unroll
      for (int kb = 0; kb < kWKB; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) mx = fmaxf(mx, st[kb][e]);
      const float ax = max_xor32(max_xor16(mx)) + mcur;
      if (ax > m + kWSlack) {
        const float alpha = fast_exp2(m - ax);
        lsum *= alpha;
#pragma unroll
        for (int j = 0; j < kWOB; ++j) o[j] *= alpha;
        m = ax;
        const float d = mcur - ax;
#pragma unroll
        for (int kb = 0; kb < kWKB; ++kb)
#pragma unroll
          for (int e = 0; e < 4; ++e) st[kb][e] += d;
        mcur = ax;
      }
    };
    auto weights = [&]() {
#pragma unroll
      for (int kb = 0; kb < kWKB; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) pb[kb >> 1][(kb & 1) * 4 + e] = (f16)fast_exp2(st[kb][e]);
      float ls = 0.f;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 8; e += 2)
          ls = dot2(f16x2{pb[h][e], pb[h][e + 1]}, f16x2{(f16)1.f, (f16)1.f}, ls);
      return ls;
    };
    if (__builtin_amdgcn_ballot_w64(m == kNegBig && k0 <= lim)) rescale();
    float ls = weights();
    if (__builtin_amdgcn_ballot_w64(__builtin_isinf(ls))) {
      rescale();
      ls = weights();
    }
    lsum += ls;
    // O^T += V^T P^T, 32 keys per step: lanes 4e..4e+3 of a 16-lane group
    // address 16 consecutive dims of key row 4*lq + e (+16), and lane j gets
    // V[key][d0 + j] (the ds_read_b64_tr_b16 layout).
    const int vr0 = 4 * lq + (lr >> 2);
    auto vaddr = [&](int r, int dblk) {
      return reinterpret_cast<const f16*>(vs + r * kWRowBytes +
                                          (((2 * dblk + ((lr >> 1) & 1)) ^ wvswz(r)) << 4) +
                                          8 * (lr & 1));
    };
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      f16x8 vf[kWOB];
#pragma unroll
      for (int dblk = 0; dblk < kWOB; ++dblk) {
        const f16x4 lo = lds_read_tr16(vaddr(h * 32 + vr0, dblk));
        const f16x4 hi = lds_read_tr16(vaddr(h * 32 + 16 + vr0, dblk));
        vf[dblk] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int dblk = 0; dblk < kWOB; ++dblk) o[dblk] = mfma16x16x32(vf[dblk], pb[h], o[dblk]);
    }
    wait_tile();      // this wave's part of tile kt+1 is in LDS
    __syncthreads();  // every part is, and every wave is done with tile kt
  }

  lsum = sum_xor32(sum_xor16(lsum));
  if (!row_ok) return;
  const int64_t out_rows = (int64_t)a.batch * a.n_new * a.n_heads;
  if (!in_bounds(grow, 1, out_rows, a.status)) return;
  if (a.nsplit == 1) {
    const float inv = 1.f / lsum;
#pragma unroll
    for (int dblk = 0; dblk < kWOB; ++dblk) {
      if (kPadD && dblk * 16 + 4 * lq >= D) continue;  // a padded dim
      wide_store_o4<kO16>(a.out, grow * D + dblk * 16 + 4 * lq, o[dblk] * inv);
    }
  } else {
    // This split's record, as prefill_kernel writes them (fp16 o / l with an
    // fp16 output, fp32 o otherwise), 256 dims per record.
    const int64_t rec = grow * a.nsplit + split;
    if (!in_bounds(rec, 1, a.records, a.status)) return;
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
#pragma unroll
    for (int dblk = 0; dblk < kWOB; ++dblk) {
      const int64_t at = rec * kWD + dblk * 16 + 4 * lq;
      if constexpr (kO16) wide_store_o4<true>(a.part_o, at, o[dblk] * inv);
      else *reinterpret_cast<f32x4*>(a.part_o + at) = o[dblk];
    }
    if (lq == 0) a.part_ml[rec] = make_float2(m, lsum);
  }
}

// out[row] = sum_s o_s 2^(m_s - M) / sum_s l_s 2^(m_s - M) over the row's
// split records (256 dims each), one pass with an online maximum; 64
// threads per row, 4 dims each. With kO16 the records hold o_s / l_s in
// fp16 and are weighted by l_s 2^(m_s - M).
template <bool kO16>
__global__ __launch_bounds__(256) void prefill_wide_merge_kernel(
    const float* __restrict__ part_o, const float2* __restrict__ part_ml, void* __restrict__ out,
    int64_t rows, int nsplit, int64_t records, int* status, int D) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = t >> 6;
  const int d4 = t & 63;
  if (row >= rows || d4 * 4 >= D) return;
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
                                                     rec * kWD + d4 * 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) ov[e] = (float)h[e];
    } else {
      ov = *reinterpret_cast<const f32x4*>(part_o + rec * kWD + d4 * 4);
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
  wide_store_o4<kO16>(out, row * D + d4 * 4, acc * (1.f / L));
}

// Split count: the head-128 prefill's rule (whole waves of 256 workgroups,
// at most 16 splits, at least 3 of its 128-key tiles per split, records
// permitting).
int wide_splits(int64_t row_tiles, int64_t rows, int max_len, const Workspace& ws) {
  const int64_t key_tiles = (max_len + 127) / 128;
  int64_t n = 256 / row_tiles;
  if (n <= 1 && row_tiles > 128 && key_tiles >= 48) n = 512 / row_tiles;
  if (n > 16) n = 16;
  if (n > key_tiles / 3) n = key_tiles / 3;
  while (n > 1 && rows * n > ws.records) --n;
  return n < 1 ? 1 : (int)n;
}

template <int G, bool kQ16, bool kO16, bool kPadD>
hipError_t launch_wide_t(const Shape& s, const void* q, const void* kc, const void* vc,
                         const int32_t* pos0, void* out, int batch, int n_new, int max_len,
                         const Workspace& ws, int kv_rep, hipStream_t stream) {
  auto kern = prefill_wide_kernel<G, kQ16, kO16, kPadD>;
  static std::atomic<uint64_t> attr_set{0};
  int dev = 0;
  hipError_t de = hipGetDevice(&dev);
  if (de != hipSuccess) return de;
  const uint64_t bit = 1ull << (dev & 63);
  if (!(attr_set.load() & bit)) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kWLds);
    if (e != hipSuccess) return e;
    attr_set.fetch_or(bit);
  }
  WideArgs a;
  a.q = q;
  a.k_cache = static_cast<const f16*>(kc);
  a.v_cache = static_cast<const f16*>(vc);
  a.pos0 = pos0;
  a.out = out;
  a.n_heads = s.n_heads;
  a.n_kv = s.n_kv;
  a.cap = s.cap;
  a.n_new = n_new;
  a.mtiles = (n_new * G + kWBM - 1) / kWBM;
  a.qk_scale_log2 = s.qk_scale * kLog2e;
  a.status = ws.status;
  a.head_dim = s.head_dim;
  a.kv_rep = kv_rep;
  const int64_t row_tiles = (int64_t)a.mtiles * s.n_kv * batch;
  const int64_t rows = (int64_t)n_new * s.n_heads * batch;
  const int nsplit = wide_splits(row_tiles, rows, max_len, ws);
  a.nsplit = nsplit;
  a.part_o = ws.part_o;
  a.part_ml = ws.part_ml;
  a.records = ws.records;
  a.batch = batch;
  kern<<<(unsigned)(row_tiles * nsplit), kWThreads, kWLds, stream>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || nsplit == 1) return e;
  const unsigned blocks = (unsigned)((rows * 64 + 255) / 256);
  prefill_wide_merge_kernel<kO16><<<blocks, 256, 0, stream>>>(ws.part_o, ws.part_ml, out, rows,
                                                              nsplit, ws.records, ws.status,
                                                              s.head_dim);
  return hipGetLastError();
}

template <int G, bool kPadD>
hipError_t launch_wide_p(const Shape& s, const void* q, const void* kc, const void* vc,
                         const int32_t* pos0, void* out, int batch, int n_new, int max_len,
                         const Workspace& ws, int r, hipStream_t stream) {
  if (s.q16)
    return s.o16 ? launch_wide_t<G, true, true, kPadD>(s, q, kc, vc, pos0, out, batch, n_new, max_len, ws, r, stream)
                 : launch_wide_t<G, true, false, kPadD>(s, q, kc, vc, pos0, out, batch, n_new, max_len, ws, r, stream);
  return s.o16 ? launch_wide_t<G, false, true, kPadD>(s, q, kc, vc, pos0, out, batch, n_new, max_len, ws, r, stream)
               : launch_wide_t<G, false, false, kPadD>(s, q, kc, vc, pos0, out, batch, n_new, max_len, ws, r, stream);
}

template <int G>
hipError_t launch_wide_g(const Shape& s, const void* q, const void* kc, const void* vc,
                         const int32_t* pos0, void* out, int batch, int n_new, int max_len,
                         const Workspace& ws, int r, hipStream_t stream) {
  if (s.head_dim == kWD)
    return launch_wide_p<G, false>(s, q, kc, vc, pos0, out, batch, n_new, max_len, ws, r, stream);
  return launch_wide_p<G, true>(s, q, kc, vc, pos0, out, batch, n_new, max_len, ws, r, stream);
}

}  // namespace

bool prefill_wide_head_dim(int head_dim) {
  return head_dim > kHeadDim && head_dim <= kWD && head_dim % 8 == 0;
}

hipError_t launch_prefill_wide(const Shape& s0, const void* q, const void* k_cache,
                               const void* v_cache, const int32_t* pos0, void* out, int batch,
                               int n_new, int max_len, const Workspace& ws, hipStream_t stream) {
  if (!prefill_wide_head_dim(s0.head_dim)) return hipErrorInvalidValue;
  int r = 1;
  Shape s = s0;
  s.group = kernel_group(s0.head_dim, s0.group, &r);
  s.n_kv = s0.n_kv * r;
  switch (s.group) {
    case 1: return launch_wide_g<1>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    case 2: return launch_wide_g<2>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    case 4: return launch_wide_g<4>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    case 5: return launch_wide_g<5>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    case 3:  // built at head size 256 only
      if (s.head_dim != kWD) return hipErrorInvalidValue;
      return launch_wide_p<3, false>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace nwd
