// nwd_append.hip — fused K+V cache append for gfx950.
//
// Replaces kernels/kv_append.wgsl main (:12-18), which the reference
// dispatches twice per attention layer, once for K and once for V with a
// shared uniform (engine/runtime.js:183,331-332,389-390). One launch here
// writes both caches. Each thread moves one 16-byte run (8 fp16 values) of a
// K row and the same run of the V row, so a wavefront writes 1 KB of each
// cache with 16-byte stores.
#include "nwd_common.h"
#include "nwd_internal.h"

namespace nwd {

constexpr int kAppendThreads = 256;
constexpr int kRunsPerRow = kHeadDim / 8;  // 16 runs of 8 values per head row

template <bool kSrc16>
__device__ inline f16x8 load_run(const void* src, int64_t elem) {
  if constexpr (kSrc16) {
    return *reinterpret_cast<const f16x8*>(static_cast<const f16*>(src) + elem);
  } else {
    const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(src) + elem);
    f32x4 a = p[0], b = p[1];
    f16x8 r;
    // v_cvt_f16_f32 rounds to nearest even (the default rounding mode).
    r[0] = (f16)a[0]; r[1] = (f16)a[1]; r[2] = (f16)a[2]; r[3] = (f16)a[3];
    r[4] = (f16)b[0]; r[5] = (f16)b[1]; r[6] = (f16)b[2]; r[7] = (f16)b[3];
    return r;
  }
}

// grid: (ceil(n_tokens * Hkv * 16 / 256), batch). Source rows are
// [batch][n_tokens][Hkv][D]; token j of sequence b lands at pos[b] + j.
template <bool kSrc16>
__global__ __launch_bounds__(kAppendThreads) void kv_append_kernel(
    const void* __restrict__ k_new, const void* __restrict__ v_new,
    f16* __restrict__ k_cache, f16* __restrict__ v_cache,
    const int32_t* __restrict__ pos, int n_tokens, int n_kv, int cap,
    int* __restrict__ status) {
  const int b = blockIdx.y;
  // 64-bit run index: n_tokens * n_kv * 16 can exceed 2^31 at the largest
  // capacities.
  const int64_t runs_per_token = (int64_t)n_kv * kRunsPerRow;
  const int64_t i = (int64_t)blockIdx.x * kAppendThreads + threadIdx.x;
  if (i >= (int64_t)n_tokens * runs_per_token) return;
  const int j = (int)(i / runs_per_token);
  const int rem = (int)(i - j * runs_per_token);
  const int h = rem / kRunsPerRow;
  const int run = rem - h * kRunsPerRow;
  const int64_t p = (int64_t)pos[b] + j;
  if (p < 0 || p >= cap) {  // the reference host throws here (runtime.js:448)
    atomicOr(status, kStatusBadPos);
    return;
  }
  const int64_t src = (((int64_t)b * n_tokens + j) * n_kv + h) * kHeadDim + run * 8;
  const int64_t dst = cache_index(b, (int)p, h, run * 8, n_kv, cap);
  f16x8 kr = load_run<kSrc16>(k_new, src);
  f16x8 vr = load_run<kSrc16>(v_new, src);
  if (!in_bounds(dst, 8, (int64_t)gridDim.y * n_kv * cap * kHeadDim, status)) return;
  *reinterpret_cast<f16x8*>(k_cache + dst) = kr;
  *reinterpret_cast<f16x8*>(v_cache + dst) = vr;
}

hipError_t launch_kv_append(const Shape& s, const void* k_new, const void* v_new,
                            void* k_cache, void* v_cache, const int32_t* pos,
                            int batch, int n_tokens, int* status,
                            hipStream_t stream) {
  const int64_t runs = (int64_t)n_tokens * s.n_kv * kRunsPerRow;
  const int64_t blocks = (runs + kAppendThreads - 1) / kAppendThreads;
  if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;  // beyond the grid's x range
  dim3 grid((unsigned)blocks, (unsigned)batch);
  if (s.kv16) {
    kv_append_kernel<true><<<grid, kAppendThreads, 0, stream>>>(
        k_new, v_new, static_cast<f16*>(k_cache), static_cast<f16*>(v_cache), pos,
        n_tokens, s.n_kv, s.cap, status);
  } else {
    kv_append_kernel<false><<<grid, kAppendThreads, 0, stream>>>(
        k_new, v_new, static_cast<f16*>(k_cache), static_cast<f16*>(v_cache), pos,
        n_tokens, s.n_kv, s.cap, status);
  }
  return hipGetLastError();
}

}  // namespace nwd
