// nwd_prefill.hip — causal chunked-prefill attention on gfx950 fp16 MFMA.
//
// The reference has no prefill kernel: each prompt token runs the whole
// decode step (kv_append, then sparse_attn over keys 0..seq) one at a time
// (engine/runtime.js:640-643). The result of that loop is what this kernel
// computes in one launch: with the n_new new K/V rows already appended at
// tokens pos0 .. pos0+n_new-1, query i attends keys 0 .. pos0+i.
//
// GQA packing: for one KV head the G query heads of the group and the n_new
// queries form n_new*G rows (row R = query R/G, head R%G) that all share the
// same K/V stream. A workgroup (8 wavefronts) owns 64 consecutive rows and
// walks 128-key tiles. Wavefront w computes row group w%2 (32 rows, two
// 16-row MFMA blocks) against key quarter w/2 (32 keys) of each tile: every
// K/V fragment read from LDS feeds two MFMAs, which halves LDS traffic per
// flop against 16-row waves, and two wavefronts share each SIMD so the
// matrix cores always have a second wavefront to issue from.
//   - K and V rows go from memory straight into LDS (buffer_load_dwordx4
//     with the lds flag, gfx950: one instruction writes 1 KB, lane l's 16
//     bytes at +16l), double-buffered: the next tile's copies land while the
//     current tile is computed, and one wait plus one barrier per tile
//     publish them. Rows are unpadded (256 B); the 16-byte chunks of a row
//     are XOR-swizzled by the row index so the MFMA operand reads hit
//     distinct banks (each lane fetches the chunk its LDS slot must hold);
//   - S^T = K Q^T on v_mfma_f32_16x16x32_f16 (K from LDS as the A operand,
//     the query rows held in registers as the B operand), so each lane holds
//     4 consecutive keys of ONE row — its own softmax row;
//   - causal mask only on tiles that cross a row's limit; online softmax in
//     log2 units with the scale folded into the exp2 argument (one FMA per
//     score), the row sum taken over the fp16 weights the PV product uses
//     (v_dot2 with ones, two weights per instruction); O^T += V^T P^T on the same MFMA, where P^T (fp16) is built in
//     registers from the S^T accumulators with no data movement between
//     lanes, and V^T is read from the row-major V tile with two
//     ds_read_b64_tr_b16 transpose loads per operand (gfx950): within a
//     16-lane group, output lane j element e comes from position j%4 of the
//     8 bytes lane 4e + j/4 addresses, so lanes 4e..4e+3 addressing 16
//     consecutive dims of key row e give lane j V[key_e][d0 + j];
//   - the four key quarters of a row group are merged through LDS at the
//     end; accumulation is fp32 throughout and O is normalised once.
#include "nwd_common.h"
#include "nwd_internal.h"

namespace nwd {

constexpr int kPWaves = 8;
constexpr int kPThreads = kPWaves * 64;
constexpr int kPBM = 64;                    // rows per workgroup
constexpr int kPBN = 128;                   // keys per tile
constexpr int kRowBytes = kHeadDim * 2;     // 256: K/V rows are unpadded in LDS
constexpr int kTileBytes = kPBN * kRowBytes;  // 32 KB
constexpr int kStageInsts = kTileBytes / (kPWaves * 1024);  // 1 KB per wave per copy (4)
// Chunk swizzles (16 chunks of 16 bytes per row): physical chunk p of LDS
// row r holds logical chunk p ^ kswz(r) of a K row, p ^ vswz(r) of a V row.
// A K operand read (16 rows, one logical chunk) then covers 16 distinct
// chunks, and a transpose read (4 rows x 2 chunks per 16 lanes) 8.
__device__ inline int kswz(int r) { return r & 15; }
__device__ inline int vswz(int r) { return (r & 7) << 1; }
typedef __attribute__((address_space(3))) void lds_void;

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Transpose load of 4 fp16 values (see the header comment for the lanes).
__device__ inline f16x4 lds_read_tr16(const f16* p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  return __builtin_bit_cast(f16x4, v);
}

__device__ inline f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

template <bool kQ16>
__device__ inline f16x8 load_q8(const void* q, int64_t elem) {
  if constexpr (kQ16) {
    return *reinterpret_cast<const f16x8*>(static_cast<const f16*>(q) + elem);
  } else {
    const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(q) + elem);
    f32x4 a = p[0], c = p[1];
    f16x8 r;
    r[0] = (f16)a[0]; r[1] = (f16)a[1]; r[2] = (f16)a[2]; r[3] = (f16)a[3];
    r[4] = (f16)c[0]; r[5] = (f16)c[1]; r[6] = (f16)c[2]; r[7] = (f16)c[3];
    return r;
  }
}

// grid: one workgroup per (row tile, kv head, sequence), kv head fastest so
// that the workgroups the dispatcher sends to one XCD share a KV head and its
// K/V stream in that XCD's L2.
template <int G, bool kQ16, bool kO16>
__global__ __launch_bounds__(kPThreads, 1) void prefill_kernel(
    const void* __restrict__ q, const f16* __restrict__ k_cache,
    const f16* __restrict__ v_cache, const int32_t* __restrict__ pos0,
    void* __restrict__ out, int n_heads, int n_kv, int cap, int n_new,
    int mtiles, float qk_scale_log2, int* __restrict__ status) {
  constexpr int RB = 2;  // 16-row MFMA blocks per wavefront
  extern __shared__ __attribute__((aligned(16))) f16 smem[];
  char* lds = reinterpret_cast<char*>(smem);  // K0 K1 V0 V1, 32 KB each

  const int id = blockIdx.x;
  const int hkv = id % n_kv;
  const int rest = id / n_kv;
  const int mt = rest % mtiles;
  const int b = rest / mtiles;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, lq = lane >> 4;
  const int rg = wave & 1, kq = wave >> 1;  // row group (32 rows), key quarter (32 keys)

  int P0 = pos0[b];
  if (P0 < 0 || P0 > cap - n_new) {
    if (tid == 0 && mt == 0 && hkv == 0) atomicOr(status, kStatusBadPos);
    P0 = P0 < 0 ? 0 : cap - n_new;
  }
  const int total_rows = n_new * G;
  const int r_last = min(mt * kPBM + kPBM, total_rows) - 1;
  const int kend = P0 + r_last / G + 1;  // keys this workgroup needs
  const int ntiles = (kend + kPBN - 1) / kPBN;

  // This wave's rows: R = mt*64 + rg*32 + rb*16 + lr. Query rows are the B
  // operand of S^T = K Q^T: lane holds Q[row][db*32 + 8*lq .. +7].
  const int r0 = mt * kPBM + rg * 32;
  int qi[RB], gq[RB], lim[RB];
  f16x8 qf[RB][4];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int R = r0 + rb * 16 + lr;
    const bool ok = R < total_rows;
    qi[rb] = ok ? R / G : 0;
    gq[rb] = ok ? R - qi[rb] * G : 0;
    lim[rb] = ok ? P0 + qi[rb] : -1;  // last key this row attends
    const int64_t qrow = ((int64_t)(b * n_new + qi[rb]) * n_heads + hkv * G + gq[rb]) * kHeadDim;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      if (ok) {
        qf[rb][db] = load_q8<kQ16>(q, qrow + db * 32 + 8 * lq);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[rb][db][e] = (f16)0.f;
      }
    }
  }
  // Keys at or below every row limit of this wave need no mask.
  const bool wave_has_pad = r0 + 31 >= total_rows;
  const int wave_min_lim = P0 + r0 / G;

  const int64_t slab = (int64_t)(b * n_kv + hkv) * cap * kHeadDim;
  const f16* kb_ptr = k_cache + slab;
  const f16* vb_ptr = v_cache + slab;

  const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(kb_ptr), 0,
                                                    kend * (kHeadDim * 2), kBufferWord3);
  const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(vb_ptr), 0,
                                                    kend * (kHeadDim * 2), kBufferWord3);
  // Wave w copies rows 16w .. 16w+15 of a tile, 4 rows (1 KB) per
  // instruction: lane l fills physical chunk l & 15 of row 16w + 4i + l/16.
  // Rows past kend read as zeros (buffer range check), so no LDS row is
  // ever stale.
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const int st_row = 16 * wv + (lane >> 4), st_p = lane & 15;
  auto load_tile = [&](int kt, int bb) {
    char* kdst = lds + bb * kTileBytes + wv * 16 * kRowBytes;
    char* vdst = lds + (2 + bb) * kTileBytes + wv * 16 * kRowBytes;
#pragma unroll
    for (int i = 0; i < kStageInsts; ++i) {
      const int row = st_row + 4 * i;
      const uint32_t rb_off = (uint32_t)(kt * kPBN + row) * kRowBytes;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(kdst + i * 1024), 16,
                                               rb_off + ((st_p ^ kswz(row)) << 4), 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(vdst + i * 1024), 16,
                                               rb_off + ((st_p ^ vswz(row)) << 4), 0, 0, 0);
    }
  };
  auto wait_tile = [&]() { __builtin_amdgcn_s_waitcnt(0x0F70); };  // vmcnt(0)

  // Running max of the raw scores (log2 units after scaling) and sums.
  float m[RB], lsum[RB];
  f32x4 o[RB][8];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    m[rb] = kNegBig;
    lsum[rb] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[rb][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const float c = qk_scale_log2;

  // Prologue: tile 0 into LDS, tile 1 in flight.
  load_tile(0, 0);
  wait_tile();
  __syncthreads();
  load_tile(1, 1);

  for (int kt = 0; kt < ntiles; ++kt) {
    const int buf = kt & 1;
    const char* ks = lds + buf * kTileBytes + kq * 32 * kRowBytes;
    const char* vs = lds + (2 + buf) * kTileBytes + kq * 32 * kRowBytes;
    // transpose reads: lane 4e+c of a 16-lane group reads dims 4c..4c+3 (of
    // each 16-dim block) of key row 4*lq + e (+16 for the second half of the
    // operand); those dims are logical chunk 2*dblk + c/2, bytes 8*(c&1).
    const int vr0 = 4 * lq + (lr >> 2);
    auto vaddr = [&](int r, int dblk) {
      return reinterpret_cast<const f16*>(vs + r * kRowBytes +
                                          (((2 * dblk + ((lr >> 1) & 1)) ^ vswz(r)) << 4) + 8 * (lr & 1));
    };
    const int k0 = kt * kPBN + kq * 32;

    // st[kb][rb][e] = raw score(key k0 + kb*16 + 4*lq + e, row rb*16 + lr)
    f32x4 st[2][RB];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) st[kb][rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const f16x8 a = *reinterpret_cast<const f16x8*>(ks + (kb * 16 + lr) * kRowBytes +
                                                        (((4 * db + lq) ^ lr) << 4));
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) st[kb][rb] = mfma16x16x32(a, qf[rb][db], st[kb][rb]);
      }
    }

    if (wave_has_pad || k0 + 31 > wave_min_lim) {  // this tile crosses a row limit
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (k0 + kb * 16 + 4 * lq + e > lim[rb]) st[kb][rb][e] = -INFINITY;
    }

    f16x8 pb[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float mx = fmaxf(fmaxf(fmaxf(st[0][rb][0], st[0][rb][1]), fmaxf(st[0][rb][2], st[0][rb][3])),
                       fmaxf(fmaxf(st[1][rb][0], st[1][rb][1]), fmaxf(st[1][rb][2], st[1][rb][3])));
      mx = max_xor32(max_xor16(mx));
      if (mx > m[rb]) {  // rescale only when the running max moves
        const float alpha = fast_exp2((m[rb] - mx) * c);
        lsum[rb] *= alpha;
#pragma unroll
        for (int j = 0; j < 8; ++j) o[rb][j] *= alpha;
        m[rb] = mx;
      }
      const float mc = m[rb] * c;
      // P^T operand (32 keys): element e < 4 is key k0 + 4*lq + e, element
      // e >= 4 is key k0 + 16 + 4*lq + (e-4); V^T is read in the same order.
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p = fast_exp2(fmaf(st[kb][rb][e], c, -mc));
          pb[rb][kb * 4 + e] = (f16)p;
        }
      // the row sum of the fp16 weights the PV product uses
#pragma unroll
      for (int e = 0; e < 8; e += 2)
        lsum[rb] = dot2(f16x2{pb[rb][e], pb[rb][e + 1]}, f16x2{(f16)1.f, (f16)1.f}, lsum[rb]);
    }

#pragma unroll
    for (int dblk = 0; dblk < 8; ++dblk) {
      const f16x4 lo = lds_read_tr16(vaddr(vr0, dblk));
      const f16x4 hi = lds_read_tr16(vaddr(16 + vr0, dblk));
      const f16x8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) o[rb][dblk] = mfma16x16x32(a, pb[rb], o[rb][dblk]);
    }

    wait_tile();      // this wave's part of tile kt+1 is in LDS
    __syncthreads();  // every part is, and every wave is done with tile kt
    if (kt + 2 < ntiles) load_tile(kt + 2, buf);  // nothing lands in LDS after the loop
  }

  // Row totals of this key quarter, then merge the quarters through LDS:
  // quarters 1..3 publish (m, l, o); quarter 0 combines and writes O.
  constexpr int kX = 2 + 32;  // floats per (rb) state: m, l, o[8][4]
  float* xch = reinterpret_cast<float*>(smem);  // [3 quarters][2 row groups][64 lanes][RB][kX]
  auto slot = [&](int qq, int rb) { return xch + ((((qq - 1) * 2 + rg) * 64 + lane) * RB + rb) * kX; };
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    lsum[rb] = sum_xor32(sum_xor16(lsum[rb]));
  }
  if (kq > 0) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float* x = slot(kq, rb);
      x[0] = m[rb];
      x[1] = lsum[rb];
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) x[2 + j * 4 + e] = o[rb][j][e];
    }
  }
  __syncthreads();
  if (kq > 0) return;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int R = r0 + rb * 16 + lr;
    if (R >= total_rows) continue;
    float M = m[rb];
#pragma unroll
    for (int qq = 1; qq < 4; ++qq) M = fmaxf(M, slot(qq, rb)[0]);
    const float a0 = fast_exp2((m[rb] - M) * c);
    float lt = lsum[rb] * a0;
    float w[3];
#pragma unroll
    for (int qq = 1; qq < 4; ++qq) {
      w[qq - 1] = fast_exp2((slot(qq, rb)[0] - M) * c);
      lt = fmaf(slot(qq, rb)[1], w[qq - 1], lt);
    }
    const float inv = 1.f / lt;
    // o[rb][dblk][e] = O^T[d = dblk*16 + 4*lq + e][row R]
    const int64_t orow = ((int64_t)(b * n_new + qi[rb]) * n_heads + hkv * G + gq[rb]) * kHeadDim;
#pragma unroll
    for (int dblk = 0; dblk < 8; ++dblk) {
      f32x4 r = o[rb][dblk] * a0;
#pragma unroll
      for (int qq = 1; qq < 4; ++qq)
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = fmaf(slot(qq, rb)[2 + dblk * 4 + e], w[qq - 1], r[e]);
      r *= inv;
      const int64_t at = orow + dblk * 16 + 4 * lq;
      if constexpr (kO16) {
        f16x4 h;
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = (f16)r[e];
        *reinterpret_cast<f16x4*>(static_cast<f16*>(out) + at) = h;
      } else {
        *reinterpret_cast<f32x4*>(static_cast<float*>(out) + at) = r;
      }
    }
  }
}

constexpr size_t kPrefillLds = (size_t)4 * kTileBytes;
static_assert(kPrefillLds >= (size_t)3 * 2 * 64 * 2 * 34 * sizeof(float), "merge exchange fits");
static_assert(kPrefillLds <= 160 * 1024, "LDS of one gfx950 CU");

template <int G, bool kQ16, bool kO16>
static hipError_t launch_prefill_t(const Shape& s, const void* q, const void* kc, const void* vc,
                                   const int32_t* pos0, void* out, int batch, int n_new,
                                   const Workspace& ws, hipStream_t stream) {
  auto kern = prefill_kernel<G, kQ16, kO16>;
  static bool attr_set = false;  // the dynamic LDS size exceeds the 64 KB default
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPrefillLds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int mtiles = (n_new * G + kPBM - 1) / kPBM;
  const unsigned blocks = (unsigned)(mtiles * s.n_kv * batch);
  kern<<<blocks, kPThreads, kPrefillLds, stream>>>(
      q, static_cast<const f16*>(kc), static_cast<const f16*>(vc), pos0, out, s.n_heads, s.n_kv,
      s.cap, n_new, mtiles, s.qk_scale * kLog2e, ws.status);
  return hipGetLastError();
}

template <int G>
static hipError_t launch_prefill_g(const Shape& s, const void* q, const void* kc, const void* vc,
                                   const int32_t* pos0, void* out, int batch, int n_new,
                                   const Workspace& ws, hipStream_t stream) {
  if (s.q16)
    return s.o16 ? launch_prefill_t<G, true, true>(s, q, kc, vc, pos0, out, batch, n_new, ws, stream)
                 : launch_prefill_t<G, true, false>(s, q, kc, vc, pos0, out, batch, n_new, ws, stream);
  return s.o16 ? launch_prefill_t<G, false, true>(s, q, kc, vc, pos0, out, batch, n_new, ws, stream)
               : launch_prefill_t<G, false, false>(s, q, kc, vc, pos0, out, batch, n_new, ws, stream);
}

hipError_t launch_prefill(const Shape& s, const void* q, const void* k_cache,
                          const void* v_cache, const int32_t* pos0, void* out,
                          int batch, int n_new, int max_len, const Workspace& ws,
                          hipStream_t stream) {
  (void)max_len;
  switch (s.group) {
    case 1: return launch_prefill_g<1>(s, q, k_cache, v_cache, pos0, out, batch, n_new, ws, stream);
    case 2: return launch_prefill_g<2>(s, q, k_cache, v_cache, pos0, out, batch, n_new, ws, stream);
    case 4: return launch_prefill_g<4>(s, q, k_cache, v_cache, pos0, out, batch, n_new, ws, stream);
    case 5: return launch_prefill_g<5>(s, q, k_cache, v_cache, pos0, out, batch, n_new, ws, stream);
    case 8: return launch_prefill_g<8>(s, q, k_cache, v_cache, pos0, out, batch, n_new, ws, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace nwd
