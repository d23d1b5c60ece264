// nwd_append.hip — fused K+V cache append for gfx950.
//
// Replaces kernels/kv_append.wgsl main (:12-18), which the reference
// dispatches twice per attention layer, once for K and once for V with a
// shared uniform (engine/runtime.js:183,331-332,389-390). One launch here
// writes both caches. Each thread moves one run of a K row and the same run
// of the V row: 8 fp16 values (16-byte stores, a wavefront writes 1 KB of
// each cache) when the head size D is a multiple of 8, as at D = 128, and
// single values otherwise (the reference takes any head size, hd in its
// Params, kernels/kv_append.wgsl:1-6).
#include "nwd_common.h"
#include "nwd_internal.h"

namespace nwd {

constexpr int kAppendThreads = 256;

template <bool kSrc16, int R>
__device__ inline void load_run(const void* src, int64_t elem, f16 (&r)[R]) {
  if constexpr (R == 8) {
    f16x8 v;
    if constexpr (kSrc16) {
      v = *reinterpret_cast<const f16x8*>(static_cast<const f16*>(src) + elem);
    } else {
      const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(src) + elem);
      const f32x4 a = p[0], b = p[1];
      // v_cvt_f16_f32 rounds to nearest even (the default rounding mode).
      v[0] = (f16)a[0]; v[1] = (f16)a[1]; v[2] = (f16)a[2]; v[3] = (f16)a[3];
      v[4] = (f16)b[0]; v[5] = (f16)b[1]; v[6] = (f16)b[2]; v[7] = (f16)b[3];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = v[e];
  } else {
    r[0] = kSrc16 ? static_cast<const f16*>(src)[elem] : (f16) static_cast<const float*>(src)[elem];
  }
}

template <int R>
__device__ inline void store_run(f16* dst, const f16 (&r)[R]) {
  if constexpr (R == 8) {
    f16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = r[e];
    *reinterpret_cast<f16x8*>(dst) = v;
  } else {
    dst[0] = r[0];
  }
}

// grid: (ceil(n_tokens * Hkv * D / R / 256), batch). Source rows are
// [batch][n_tokens][Hkv][D]; token j of sequence b lands at pos[b] + j.
template <bool kSrc16, int R>
__global__ __launch_bounds__(kAppendThreads) void kv_append_kernel(
    const void* __restrict__ k_new, const void* __restrict__ v_new,
    f16* __restrict__ k_cache, f16* __restrict__ v_cache,
    const int32_t* __restrict__ pos, int n_tokens, int n_kv, int D, int cap,
    int* __restrict__ status) {
  const int b = blockIdx.y;
  const int runs_per_row = D / R;
  // 64-bit run index: n_tokens * n_kv * runs can exceed 2^31 at the largest
  // capacities.
  const int64_t runs_per_token = (int64_t)n_kv * runs_per_row;
  const int64_t i = (int64_t)blockIdx.x * kAppendThreads + threadIdx.x;
  if (i >= (int64_t)n_tokens * runs_per_token) return;
  const int j = (int)(i / runs_per_token);
  const int rem = (int)(i - j * runs_per_token);
  const int h = rem / runs_per_row;
  const int run = rem - h * runs_per_row;
  const int64_t p = (int64_t)pos[b] + j;
  if (p < 0 || p >= cap) {  // the reference host throws here (runtime.js:448)
    atomicOr(status, kStatusBadPos);
    return;
  }
  const int64_t src = (((int64_t)b * n_tokens + j) * n_kv + h) * D + run * R;
  const int64_t dst = cache_index_d(b, (int)p, h, run * R, n_kv, cap, D);
  f16 kr[R], vr[R];
  load_run<kSrc16, R>(k_new, src, kr);
  load_run<kSrc16, R>(v_new, src, vr);
  if (!in_bounds(dst, R, (int64_t)gridDim.y * n_kv * cap * D, status)) return;
  store_run<R>(k_cache + dst, kr);
  store_run<R>(v_cache + dst, vr);
}

template <int R>
hipError_t launch_kv_append_r(const Shape& s, const void* k_new, const void* v_new,
                              void* k_cache, void* v_cache, const int32_t* pos, int batch,
                              int n_tokens, int* status, hipStream_t stream) {
  const int64_t runs = (int64_t)n_tokens * s.n_kv * (s.head_dim / R);
  const int64_t blocks = (runs + kAppendThreads - 1) / kAppendThreads;
  if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;  // beyond the grid's x range
  dim3 grid((unsigned)blocks, (unsigned)batch);
  f16* kc = static_cast<f16*>(k_cache);
  f16* vc = static_cast<f16*>(v_cache);
  if (s.kv16)
    kv_append_kernel<true, R><<<grid, kAppendThreads, 0, stream>>>(
        k_new, v_new, kc, vc, pos, n_tokens, s.n_kv, s.head_dim, s.cap, status);
  else
    kv_append_kernel<false, R><<<grid, kAppendThreads, 0, stream>>>(
        k_new, v_new, kc, vc, pos, n_tokens, s.n_kv, s.head_dim, s.cap, status);
  return hipGetLastError();
}

hipError_t launch_kv_append(const Shape& s, const void* k_new, const void* v_new,
                            void* k_cache, void* v_cache, const int32_t* pos,
                            int batch, int n_tokens, int* status,
                            hipStream_t stream) {
  if (s.head_dim % 8 == 0)
    return launch_kv_append_r<8>(s, k_new, v_new, k_cache, v_cache, pos, batch, n_tokens, status, stream);
  return launch_kv_append_r<1>(s, k_new, v_new, k_cache, v_cache, pos, batch, n_tokens, status, stream);
}

}  // namespace nwd
