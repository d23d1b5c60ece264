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
// same K/V stream. A workgroup owns 64*RB consecutive rows (4 wavefronts of
// 16*RB rows) and walks 64-key tiles:
//   - the tile's K rows are staged in LDS row-major and its V rows in LDS
//     transposed (V^T[d][key]), both with padding against bank conflicts;
//     the next tile's loads are in flight while the current one computes;
//   - S^T = K Q^T on v_mfma_f32_16x16x32_f16 (K from LDS as the A operand,
//     the query rows held in registers as the B operand), so each lane ends
//     up with 4 consecutive keys of ONE row — its own softmax row;
//   - scale, causal mask, online softmax in log2 units (exp2), then
//     O^T += V^T P^T on the same MFMA, where P^T (fp16) is built in
//     registers from the S^T accumulators with no data movement between
//     lanes, and V^T comes from LDS with two 8-byte reads per operand;
//   - accumulation is fp32 throughout; O is normalised once at the end.
#include "nwd_common.h"
#include "nwd_internal.h"

namespace nwd {

constexpr int kPWaves = 4;
constexpr int kPThreads = kPWaves * 64;
constexpr int kPBN = 64;                   // keys per tile
constexpr int kKsStride = kHeadDim + 8;    // halves per K row in LDS (272 B)
constexpr int kVtStride = kPBN + 8;        // halves per V^T row in LDS (144 B)

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
// consecutive workgroups (which the dispatcher spreads over the XCDs) of one
// XCD share a KV head and its K/V stream in that XCD's L2.
template <int G, int RB, bool kQ16, bool kO16>
__global__ __launch_bounds__(kPThreads, 2) void prefill_kernel(
    const void* __restrict__ q, const f16* __restrict__ k_cache,
    const f16* __restrict__ v_cache, const int32_t* __restrict__ pos0,
    void* __restrict__ out, int n_heads, int n_kv, int cap, int n_new,
    int mtiles, float qk_scale_log2, int* __restrict__ status) {
  constexpr int kWaveRows = 16 * RB;
  constexpr int kBM = kPWaves * kWaveRows;

  __shared__ __attribute__((aligned(16))) f16 Ks[kPBN * kKsStride];
  __shared__ __attribute__((aligned(16))) f16 Vt[kHeadDim * kVtStride];

  const int id = blockIdx.x;
  const int hkv = id % n_kv;
  const int rest = id / n_kv;
  const int mt = rest % mtiles;
  const int b = rest / mtiles;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, lq = lane >> 4;

  int P0 = pos0[b];
  if (P0 < 0 || P0 > cap - n_new) {
    if (tid == 0 && mt == 0 && hkv == 0) atomicOr(status, kStatusBadPos);
    P0 = P0 < 0 ? 0 : cap - n_new;
  }
  const int total_rows = n_new * G;
  const int row_base = mt * kBM + wave * kWaveRows;
  const int r_last = min(mt * kBM + kBM, total_rows) - 1;
  const int kend = P0 + r_last / G + 1;  // keys this workgroup needs
  const int ntiles = (kend + kPBN - 1) / kPBN;

  // Query rows as the B operand of S^T = K Q^T: lane holds
  // Q[row rb*16+lr][db*32 + 8*lq .. +7].
  f16x8 qf[RB][4];
  int lim[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int R = row_base + rb * 16 + lr;
    const bool ok = R < total_rows;
    const int qi = ok ? R / G : 0, g = ok ? R - (R / G) * G : 0;
    lim[rb] = ok ? P0 + qi : -1;
    const int64_t qrow = ((int64_t)(b * n_new + qi) * n_heads + hkv * G + g) * kHeadDim;
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

  const int64_t slab = (int64_t)(b * n_kv + hkv) * cap * kHeadDim;
  const f16* kb_ptr = k_cache + slab;
  const f16* vb_ptr = v_cache + slab;

  // Staging registers. K: 16 threads per key row, 4 instructions cover the
  // 64 keys. V: lane = key, wave w takes dim runs 4w..4w+3 (written
  // transposed into LDS, one 64-key row segment per store).
  f16x8 kr[4], vr[4];
  auto load_tile = [&](int kt) {
    const int k0 = kt * kPBN;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = min(k0 + i * 16 + (tid >> 4), kend - 1);
      kr[i] = *reinterpret_cast<const f16x8*>(kb_ptr + (int64_t)key * kHeadDim + (tid & 15) * 8);
    }
    const int vkey = min(k0 + lane, kend - 1);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      vr[i] = *reinterpret_cast<const f16x8*>(vb_ptr + (int64_t)vkey * kHeadDim + (wave * 4 + i) * 8);
  };

  float m[RB], lsum[RB];
  f32x4 o[RB][8];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    m[rb] = kNegBig;
    lsum[rb] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[rb][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  if (ntiles > 0) load_tile(0);
  for (int kt = 0; kt < ntiles; ++kt) {
    __syncthreads();  // the previous tile's LDS reads are done
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<f16x8*>(&Ks[(i * 16 + (tid >> 4)) * kKsStride + (tid & 15) * 8]) = kr[i];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) Vt[((wave * 4 + i) * 8 + e) * kVtStride + lane] = vr[i][e];
    __syncthreads();
    if (kt + 1 < ntiles) load_tile(kt + 1);

    // S^T tile: st[kb][rb][e] = score(key k0 + kb*16 + 4*lq + e, row rb*16 + lr)
    f32x4 st[4][RB];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) st[kb][rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const f16x8 a = *reinterpret_cast<const f16x8*>(&Ks[(kb * 16 + lr) * kKsStride + db * 32 + 8 * lq]);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) st[kb][rb] = mfma16x16x32(a, qf[rb][db], st[kb][rb]);
      }
    }

    const int k0 = kt * kPBN;
    f16x8 pb[RB][2];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float mx = kNegBig;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key = k0 + kb * 16 + 4 * lq + e;
          const float s = key <= lim[rb] ? st[kb][rb][e] * qk_scale_log2 : -INFINITY;
          st[kb][rb][e] = s;
          mx = fmaxf(mx, s);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mnew = fmaxf(m[rb], mx);
      const float alpha = fast_exp2(m[rb] - mnew);
      m[rb] = mnew;
      lsum[rb] *= alpha;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[rb][j] *= alpha;
      float ps = 0.f;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p = fast_exp2(st[kb][rb][e] - mnew);
          st[kb][rb][e] = p;
          ps += p;
        }
      lsum[rb] += ps;
      // P^T operand for k-block h (32 keys): element e < 4 is key
      // h*32 + 4*lq + e, element e >= 4 is key h*32 + 16 + 4*lq + (e-4).
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pb[rb][h][e] = (f16)st[2 * h][rb][e];
          pb[rb][h][4 + e] = (f16)st[2 * h + 1][rb][e];
        }
    }

    // O^T[d][row] += V^T[d][keys] P^T[keys][row], keys in the same order.
#pragma unroll
    for (int dblk = 0; dblk < 8; ++dblk) {
      const f16* vrow = &Vt[(dblk * 16 + lr) * kVtStride + 4 * lq];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const f16x4 lo = *reinterpret_cast<const f16x4*>(vrow + h * 32);
        const f16x4 hi = *reinterpret_cast<const f16x4*>(vrow + h * 32 + 16);
        const f16x8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) o[rb][dblk] = mfma16x16x32(a, pb[rb][h], o[rb][dblk]);
      }
    }
  }

  // o[rb][dblk][e] = O^T[d = dblk*16 + 4*lq + e][row rb*16 + lr]
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    float lt = lsum[rb];
    lt += __shfl_xor(lt, 16);
    lt += __shfl_xor(lt, 32);
    const int R = row_base + rb * 16 + lr;
    if (R >= total_rows) continue;
    const float inv = 1.f / lt;
    const int qi = R / G, g = R - (R / G) * G;
    const int64_t orow = ((int64_t)(b * n_new + qi) * n_heads + hkv * G + g) * kHeadDim;
#pragma unroll
    for (int dblk = 0; dblk < 8; ++dblk) {
      const int64_t at = orow + dblk * 16 + 4 * lq;
      if constexpr (kO16) {
        f16x4 r;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = (f16)(o[rb][dblk][e] * inv);
        *reinterpret_cast<f16x4*>(static_cast<f16*>(out) + at) = r;
      } else {
        f32x4 r = o[rb][dblk] * inv;
        *reinterpret_cast<f32x4*>(static_cast<float*>(out) + at) = r;
      }
    }
  }
}

template <int G, int RB>
static void launch_prefill_rb(const Shape& s, const void* q, const void* kc, const void* vc,
                              const int32_t* pos0, void* out, int batch, int n_new,
                              const Workspace& ws, hipStream_t stream) {
  constexpr int kBM = kPWaves * 16 * RB;
  const int mtiles = (n_new * G + kBM - 1) / kBM;
  const unsigned blocks = (unsigned)(mtiles * s.n_kv * batch);
  const float sl = s.qk_scale * kLog2e;
  const f16* k = static_cast<const f16*>(kc);
  const f16* v = static_cast<const f16*>(vc);
  if (s.q16) {
    if (s.o16)
      prefill_kernel<G, RB, true, true><<<blocks, kPThreads, 0, stream>>>(
          q, k, v, pos0, out, s.n_heads, s.n_kv, s.cap, n_new, mtiles, sl, ws.status);
    else
      prefill_kernel<G, RB, true, false><<<blocks, kPThreads, 0, stream>>>(
          q, k, v, pos0, out, s.n_heads, s.n_kv, s.cap, n_new, mtiles, sl, ws.status);
  } else {
    if (s.o16)
      prefill_kernel<G, RB, false, true><<<blocks, kPThreads, 0, stream>>>(
          q, k, v, pos0, out, s.n_heads, s.n_kv, s.cap, n_new, mtiles, sl, ws.status);
    else
      prefill_kernel<G, RB, false, false><<<blocks, kPThreads, 0, stream>>>(
          q, k, v, pos0, out, s.n_heads, s.n_kv, s.cap, n_new, mtiles, sl, ws.status);
  }
}

template <int G>
static void launch_prefill_g(const Shape& s, const void* q, const void* kc, const void* vc,
                             const int32_t* pos0, void* out, int batch, int n_new,
                             const Workspace& ws, hipStream_t stream) {
  // Two row blocks per wavefront when that still gives a workgroup per CU.
  const int big_tiles = (n_new * G + 127) / 128;
  if ((int64_t)big_tiles * s.n_kv * batch >= 256)
    launch_prefill_rb<G, 2>(s, q, kc, vc, pos0, out, batch, n_new, ws, stream);
  else
    launch_prefill_rb<G, 1>(s, q, kc, vc, pos0, out, batch, n_new, ws, stream);
}

hipError_t launch_prefill(const Shape& s, const void* q, const void* k_cache,
                          const void* v_cache, const int32_t* pos0, void* out,
                          int batch, int n_new, int max_len, const Workspace& ws,
                          hipStream_t stream) {
  (void)max_len;
  switch (s.group) {
    case 1: launch_prefill_g<1>(s, q, k_cache, v_cache, pos0, out, batch, n_new, ws, stream); break;
    case 2: launch_prefill_g<2>(s, q, k_cache, v_cache, pos0, out, batch, n_new, ws, stream); break;
    case 4: launch_prefill_g<4>(s, q, k_cache, v_cache, pos0, out, batch, n_new, ws, stream); break;
    case 5: launch_prefill_g<5>(s, q, k_cache, v_cache, pos0, out, batch, n_new, ws, stream); break;
    case 8: launch_prefill_g<8>(s, q, k_cache, v_cache, pos0, out, batch, n_new, ws, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace nwd
