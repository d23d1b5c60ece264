// nwd_argmax.hip — the greedy token pick (argmax) for gfx950.
//
// Replaces kernels/argmax_partial.wgsl (:16-52, 256 workgroups) and
// kernels/argmax_merge.wgsl (:8-42, one workgroup), dispatched at
// engine/runtime.js:398-399. The reference's tie order is reproduced
// exactly through the (value, key) encoding of nwd_argmax.h, so the chunks
// here need not match its slices: each 256-thread workgroup reduces 4096
// logits (16 per thread, coalesced) to one 64-bit record with an LDS
// atomic maximum, and a merge workgroup per row reduces the records and
// decodes the index. The same merge serves the lm_head GEMV, whose
// workgroups write one record per 16 logits (nwd_q4.hip).
#include "nwd_argmax.h"
#include "nwd_common.h"
#include "nwd_internal.h"

namespace nwd {

constexpr int kArgmaxThreads = 256;
constexpr int kArgmaxPerThread = 16;
constexpr int kArgmaxChunk = kArgmaxThreads * kArgmaxPerThread;

__global__ __launch_bounds__(kArgmaxThreads) void argmax_partial_kernel(
    const float* __restrict__ x, uint32_t n, unsigned long long* __restrict__ records) {
  __shared__ unsigned long long best;
  const int t = threadIdx.x;
  if (t == 0) best = 0ull;
  __syncthreads();
  const ArgmaxShape s = argmax_shape(n);
  const float* row = x + (int64_t)blockIdx.y * n;
  const uint32_t base = blockIdx.x * (uint32_t)kArgmaxChunk + t;
  unsigned long long e = 0ull;
#pragma unroll
  for (int m = 0; m < kArgmaxPerThread; ++m) {
    const uint32_t i = base + m * kArgmaxThreads;
    if (i < n) {
      const unsigned long long c = argmax_enc(row[i], i, s);
      e = c > e ? c : e;
    }
  }
  e = wave_max_u64(e);
  if ((t & 63) == 0) atomicMax(&best, e);
  __syncthreads();
  if (t == 0) records[(int64_t)blockIdx.y * gridDim.x + blockIdx.x] = best;
}

// One workgroup per row. A 131072-token vocabulary leaves 8192 records per
// row (64 KiB): 1024 threads each issue all their loads (8 per pass) before
// the first comparison, so a row costs about one memory round trip. Loads
// past the row's end return 0 through the buffer descriptor's range, which
// is the encoding of "no candidate".
constexpr int kMergeThreads = 1024;
constexpr int kMergeLoads = 8;

__global__ __launch_bounds__(kMergeThreads) void argmax_merge_kernel(
    const unsigned long long* __restrict__ records, int n_records, uint32_t n,
    uint32_t* __restrict__ out) {
  __shared__ unsigned long long best;
  const int t = threadIdx.x;
  if (t == 0) best = 0ull;
  const auto rr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<unsigned long long*>(records + (int64_t)blockIdx.x * n_records), 0,
      n_records * 8, kBufferWord3);
  unsigned long long e = 0ull;
  for (int base = 0; base < n_records; base += kMergeThreads * kMergeLoads) {
    unsigned long long v[kMergeLoads];
#pragma unroll
    for (int u = 0; u < kMergeLoads; ++u)
      v[u] = __builtin_bit_cast(unsigned long long, __builtin_amdgcn_raw_buffer_load_b64(
                                   rr, (base + u * kMergeThreads + t) * 8, 0, 0));
#pragma unroll
    for (int u = 0; u < kMergeLoads; ++u) e = v[u] > e ? v[u] : e;
  }
  e = wave_max_u64(e);
  __syncthreads();
  if ((t & 63) == 0) atomicMax(&best, e);
  __syncthreads();
  if (t == 0) out[blockIdx.x] = argmax_decode(best, argmax_shape(n));
}

int argmax_records_per_row(int n) { return (n + kArgmaxChunk - 1) / kArgmaxChunk; }

hipError_t launch_argmax(const float* x, int n, uint32_t* out, int batch,
                         unsigned long long* records, hipStream_t stream) {
  const int per_row = argmax_records_per_row(n);
  argmax_partial_kernel<<<dim3(per_row, batch), kArgmaxThreads, 0, stream>>>(x, n, records);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_argmax_merge(records, per_row, n, out, batch, stream);
}

hipError_t launch_argmax_merge(const unsigned long long* records, int per_row, int n,
                               uint32_t* out, int batch, hipStream_t stream) {
  argmax_merge_kernel<<<batch, kMergeThreads, 0, stream>>>(records, per_row, n, out);
  return hipGetLastError();
}

}  // namespace nwd
