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

// ---------------------------------------------------------------------------
// A plain read of the same bytes with none of the decode's structure: the
// 2 x slabs key ranges (K and V of each slab, keys [0, keys)) are cut into
// chunks of kU x threads x 16 bytes, and a grid of `grid` workgroups walks
// the chunks with a grid stride, each thread issuing its kU 16-byte loads of
// a chunk at once (one 1 KB run per wavefront instruction) and summing them.
// Occupancy, not software pipelining, keeps loads in flight: the launch
// shape (threads per workgroup, workgroups, loads per thread) is free, so a
// sweep of it gives a read ceiling that does not share the decode's grid.
namespace {

template <int kU, int kPolicy>
__global__ void plain_read_kernel(const char* __restrict__ k, const char* __restrict__ v,
                                  int64_t slab_stride, int64_t range_bytes, int64_t chunks_per_range,
                                  int64_t chunks, float* __restrict__ out, int per_range) {
  const int tid = threadIdx.x, nt = blockDim.x;
  const int64_t chunk_bytes = (int64_t)kU * nt * 16;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  // per_range: the workgroups are dealt to the 2 x slabs ranges (workgroup w
  // reads range w % ranges only), each range swept by its own workgroups
  // with a grid stride, so that as many regions are read at once as the
  // decode reads (K and V of every KV head); otherwise one sweep of all.
  const int64_t ranges = chunks / chunks_per_range;
  const int64_t g_per = gridDim.x / ranges;
  const int64_t c0 = per_range ? (blockIdx.x % ranges) * chunks_per_range + blockIdx.x / ranges
                               : (int64_t)blockIdx.x;
  const int64_t c_end = per_range ? (blockIdx.x % ranges + 1) * chunks_per_range : chunks;
  const int64_t c_step = per_range ? g_per : (int64_t)gridDim.x;
  for (int64_t c = c0; c < c_end; c += c_step) {
    const int64_t range = c / chunks_per_range;  // 2 * slab + (0: K, 1: V)
    const int64_t in_range = (c - range * chunks_per_range) * chunk_bytes;
    const char* base = ((range & 1) ? v : k) + (range >> 1) * slab_stride + in_range;
    const int64_t left = range_bytes - in_range;  // > 0
    const auto r = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), 0,
                                                     (int)(left < chunk_bytes ? left : chunk_bytes),
                                                     kBufferWord3);
    f32x4 t[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u)
      t[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                           r, (uint32_t)((u * nt + tid) * 16), 0, kPolicy));
#pragma unroll
    for (int u = 0; u < kU; ++u) acc += t[u];
  }
  out[(int64_t)blockIdx.x * nt + tid] = acc[0] + acc[1] + acc[2] + acc[3];
}

template <int kU>
hipError_t launch_plain(int nt_policy, dim3 grid, int threads, hipStream_t s, const char* k,
                        const char* v, int64_t slab_stride, int64_t range_bytes, int64_t cpr,
                        int64_t chunks, float* out, int per_range) {
  if (nt_policy)
    plain_read_kernel<kU, kNonTemporal><<<grid, threads, 0, s>>>(k, v, slab_stride, range_bytes,
                                                                 cpr, chunks, out, per_range);
  else
    plain_read_kernel<kU, 0><<<grid, threads, 0, s>>>(k, v, slab_stride, range_bytes, cpr, chunks,
                                                      out, per_range);
  return hipGetLastError();
}

}  // namespace

// Reads keys [0, keys) of `slabs` K and V slabs of `cap` fp16 rows each with
// `grid` workgroups of `threads` threads, `unroll` 16-byte loads per thread
// and chunk (1, 2, 4, 8 or 16), the non-temporal policy if `nt`; with
// per_range, grid must be a multiple of 2 x slabs and each workgroup sweeps
// one range. out needs grid * threads floats. Returns a hipError_t code.
extern "C" int nwd_bench_plain_read(const void* k, const void* v, int slabs, int cap, int keys,
                                    int threads, int unroll, int grid, int nt, float* out,
                                    void* stream, int per_range) {
  if (!k || !v || !out || slabs < 1 || cap < 1 || keys < 1 || keys > cap || grid < 1 ||
      threads < 64 || threads > 1024 || threads % 64 != 0 ||
      (int64_t)cap * kRowBytes > 0x7FFFFFFF || (per_range && grid % (2 * slabs) != 0))
    return (int)hipErrorInvalidValue;
  const int64_t chunk_bytes = (int64_t)unroll * threads * 16;
  const int64_t range_bytes = (int64_t)keys * kRowBytes;
  const int64_t cpr = (range_bytes + chunk_bytes - 1) / chunk_bytes;
  const int64_t chunks = cpr * 2 * slabs;
  const int64_t slab_stride = (int64_t)cap * kRowBytes;
  const char* kp = static_cast<const char*>(k);
  const char* vp = static_cast<const char*>(v);
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)grid);
  switch (unroll) {
    case 1: return (int)launch_plain<1>(nt, g, threads, s, kp, vp, slab_stride, range_bytes, cpr, chunks, out, per_range);
    case 2: return (int)launch_plain<2>(nt, g, threads, s, kp, vp, slab_stride, range_bytes, cpr, chunks, out, per_range);
    case 4: return (int)launch_plain<4>(nt, g, threads, s, kp, vp, slab_stride, range_bytes, cpr, chunks, out, per_range);
    case 8: return (int)launch_plain<8>(nt, g, threads, s, kp, vp, slab_stride, range_bytes, cpr, chunks, out, per_range);
    case 16: return (int)launch_plain<16>(nt, g, threads, s, kp, vp, slab_stride, range_bytes, cpr, chunks, out, per_range);
    default: return (int)hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------
// The cost of a kernel launch itself: a kernel whose workgroups do nothing
// but one store per workgroup, launched back to back. Its time per launch in
// a HIP graph is the dispatch-to-dispatch floor any kernel boundary pays
// (end of the previous kernel, cache release, dispatch of the next).
namespace {
__global__ void empty_kernel(int* __restrict__ sink) {
  if (threadIdx.x == 0 && sink) sink[blockIdx.x] = (int)blockIdx.x;
}
}  // namespace

// `workgroups` workgroups of `threads` threads; sink (optional) needs
// `workgroups` ints. Returns a hipError_t code.
extern "C" int nwd_bench_empty(int workgroups, int threads, int* sink, void* stream) {
  if (workgroups < 1 || threads < 64 || threads > 1024 || threads % 64 != 0)
    return (int)hipErrorInvalidValue;
  empty_kernel<<<workgroups, threads, 0, (hipStream_t)stream>>>(sink);
  return (int)hipGetLastError();
}
