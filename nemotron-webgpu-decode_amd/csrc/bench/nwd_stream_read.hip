// nwd_stream_read.hip — the read ceiling of the decode access pattern
// (measurement only; built into lib/libnwd_bench.so, not the product library).
//
// Reads exactly the bytes a decode call reads, the way decode_split_kernel
// reads them, and does nothing else: one 256-thread workgroup per (KV head
// slab, split), each streaming its own contiguous key range of the K slab and
// of the V slab with 16-byte buffer loads (one load instruction = 1 KB of 4
// consecutive keys), two iterations of 32 keys in flight, the non-temporal
// cache policy. Its time for the decode-32k caches is the floor a decode call
// over the same 134 MB could reach on the box.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kRowBytes = 256;      // one fp16 key row of head_dim 128
constexpr int kIterKeys = 32;       // keys per workgroup iteration (4 waves x 8)
constexpr int kBufferWord3 = 0x00020000;
constexpr int kNonTemporal = 2;

__global__ __launch_bounds__(kThreads) void stream_read_kernel(const char* __restrict__ k,
                                                               const char* __restrict__ v,
                                                               int cap, int keys, int splits,
                                                               float* __restrict__ out) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int split = blockIdx.x, slab = blockIdx.y;
  const int units = (keys + 127) / 128;  // 128-key units spread evenly, as the decode does
  const int t0 = (int)((int64_t)split * units / splits) * 128;
  const int t1 = min(keys, (int)((int64_t)(split + 1) * units / splits) * 128);
  const int n = t1 > t0 ? t1 - t0 : 0;
  const int64_t base = ((int64_t)slab * cap + t0) * kRowBytes;
  // Descriptors end at the range's last key: loads past it return zeros
  // without a memory access.
  const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(k + base), 0, n * kRowBytes,
                                                    kBufferWord3);
  const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(v + base), 0, n * kRowBytes,
                                                    kBufferWord3);
  const int n_it = (n + kIterKeys - 1) / kIterKeys;
  // wave iteration: 8 keys = 2 KB per array, 1 KB per load instruction
  auto off = [&](int it, int j) {
    return (uint32_t)((it * kIterKeys + wave * 8 + j * 4) * kRowBytes + lane * 16);
  };
  f32x4 a[4], b[4];
  auto issue = [&](f32x4* t, int it) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      t[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, off(it, j), 0, kNonTemporal));
      t[2 + j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, off(it, j), 0, kNonTemporal));
    }
  };
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  issue(a, 0);
  for (int it = 0; it < n_it; it += 2) {
    issue(b, it + 1);
    acc += a[0] + a[1] + a[2] + a[3];
    issue(a, it + 2);
    acc += b[0] + b[1] + b[2] + b[3];
  }
  out[((int64_t)slab * splits + split) * kThreads + tid] = acc[0] + acc[1] + acc[2] + acc[3];
}

}  // namespace

// Reads keys [0, keys) of `slabs` K and V slabs of `cap` fp16 rows each
// (head-major caches, one slab per KV head) with `splits` workgroups per
// slab. out needs slabs * splits * 256 floats. Returns a hipError_t code.
extern "C" int nwd_bench_stream_read(const void* k, const void* v, int slabs, int cap, int keys,
                                     int splits, float* out, void* stream) {
  if (!k || !v || !out || slabs < 1 || cap < 1 || keys < 1 || keys > cap || splits < 1 ||
      (int64_t)cap * kRowBytes > 0x7FFFFFFF)
    return (int)hipErrorInvalidValue;
  stream_read_kernel<<<dim3((unsigned)splits, (unsigned)slabs), kThreads, 0, (hipStream_t)stream>>>(
      static_cast<const char*>(k), static_cast<const char*>(v), cap, keys, splits, out);
  return (int)hipGetLastError();
}
