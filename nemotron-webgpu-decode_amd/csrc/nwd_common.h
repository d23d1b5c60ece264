// nwd_common.h — device helpers shared by the gfx950 kernels of libnwd_attn.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nwd {

typedef _Float16 f16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kHeadDim = 128;  // D of the benchmark shapes, the matrix-core and prefill kernels
// Largest cache capacity in tokens: a (sequence, kv head) slab is then at most
// 1 GiB, so 32-bit byte offsets into it, including those of the few tiles
// requested past a range's end, stay below 2^31.
constexpr int kMaxSeq = 1 << 22;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -3.4028234663852886e38f;  // finite "minus infinity"
// Buffer descriptor word 3 for gfx9-family raw (stride 0) buffers: loads at
// or past the descriptor's byte count return zeros without a memory access.
constexpr int kBufferWord3 = 0x00020000;
// Cache policy of the K/V stream loads: non-temporal (the nt bit). Each K/V
// byte is read once per call, and marking the reads as streaming raised the
// read rate of the decode access pattern (256 workgroups, each streaming its
// own contiguous K and V ranges, 134 MB per launch) from 5.5 to 6.2 TB/s on
// MI355X; sc0 / sc1 changed nothing.
constexpr int kStreamPolicy = 2;

// Status bits written by kernels into the context's device status word.
constexpr int kStatusBadPos = 1;
constexpr int kStatusOutOfBounds = 2;  // set only by bounds-checked builds
// A query element of a matrix-core kernel left the fp16 range of its operand
// (|q| scale log2(e) > 65504 in the prefill, |q| > 65504 for an fp32 query of
// the matrix-core decode): those scores are not finite.
constexpr int kStatusQueryRange = 4;

// Bounds-checked builds (compiled with -DNWD_CHECK) check every kernel
// store into an output, a cache or the split-K workspace, and the merges'
// reads of the workspace: the element range [at, at + n) must lie in
// [0, size), the size the call's shape (or the workspace's capacity)
// implies. An access outside it is skipped and sets kStatusOutOfBounds;
// other builds compile the check away.
#ifdef NWD_CHECK
constexpr bool kCheckBounds = true;
#else
constexpr bool kCheckBounds = false;
#endif
__device__ inline bool in_bounds(int64_t at, int64_t n, int64_t size, int* status) {
  if constexpr (!kCheckBounds) return true;
  if (at >= 0 && at + n <= size) return true;
  atomicOr(status, kStatusOutOfBounds);
  return false;
}

// Element index of (b, t, h, d) in a cache: each (sequence, kv head) owns a
// contiguous [cap][D] fp16 slab, so the keys a workgroup streams are one run.
__host__ __device__ inline int64_t cache_index(int b, int t, int h, int d,
                                               int n_kv, int cap) {
  return ((int64_t)(b * n_kv + h) * cap + t) * kHeadDim + d;
}
// The same for a head size D known at run time (the general-shape kernels).
__host__ __device__ inline int64_t cache_index_d(int b, int t, int h, int d, int n_kv, int cap,
                                                 int D) {
  return ((int64_t)(b * n_kv + h) * cap + t) * D + d;
}

// DPP lane moves inside a row of 16 lanes (data-parallel primitives, no LDS).
template <int kCtrl>
__device__ inline float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl,
                                                    0xF, 0xF, false));
}
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;   // lane i <- lane 7-i within 8 lanes
constexpr int kDppRowMirror = 0x140;    // lane i <- lane 15-i within 16 lanes
constexpr int kDppRowRor8 = 0x128;      // lane i <- lane (i+8)%16 within 16 lanes (xor 8)

// Sum over each aligned group of 8 lanes; every lane of the group gets it.
__device__ inline float sum8(float x) {
  x += dpp_mov<kDppQuadXor1>(x);
  x += dpp_mov<kDppQuadXor2>(x);
  x += dpp_mov<kDppHalfMirror>(x);
  return x;
}

// Max over each aligned group of 8 lanes.
__device__ inline float max8(float x) {
  x = fmaxf(x, dpp_mov<kDppQuadXor1>(x));
  x = fmaxf(x, dpp_mov<kDppQuadXor2>(x));
  x = fmaxf(x, dpp_mov<kDppHalfMirror>(x));
  return x;
}

// Cross-row exchanges on gfx950 without the LDS crossbar: with the same value
// in both operands, v_permlane16_swap returns the lane's own value and that of
// lane ^ 16 (in row-parity order), v_permlane32_swap the same for lane ^ 32,
// so max / sum of the two halves is the xor-16 / xor-32 reduction step.
__device__ inline float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Max / sum over each aligned group of 32 lanes (4 DPP steps inside 16
// lanes, then the lane ^ 16 exchange), and sum over the whole wavefront;
// every lane of the group gets the result.
__device__ inline float max32(float x) {
  x = max8(x);
  x = fmaxf(x, dpp_mov<kDppRowMirror>(x));
  return max_xor16(x);
}
__device__ inline float sum32(float x) {
  x = sum8(x);
  x += dpp_mov<kDppRowMirror>(x);
  return sum_xor16(x);
}
__device__ inline float sum64(float x) { return sum_xor32(sum32(x)); }

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

typedef __attribute__((address_space(3))) void lds_void;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// LDS byte address of a pointer into LDS.
__device__ inline uint32_t lds_address(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// ds_read_b64_tr_b16 (gfx950): within each 16-lane group, output lane j
// element e comes from position j % 4 of the 8 bytes that lane 4e + j / 4
// addresses.
__device__ inline f16x4 lds_read_tr16(const f16* p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  return __builtin_bit_cast(f16x4, v);
}

// The same read as inline assembly. While LDS copies
// (buffer_load ... lds) are in flight, the compiler puts a wait for every
// global load in flight (vmcnt(0)) before each builtin transpose read, as it
// cannot tell which LDS bytes a copy writes; in a loop that keeps the next
// block's copies in flight that wait drains them every block. The compiler
// does not track this form: the caller makes its results wait for it with
// lds_reads_done before using them.
__device__ inline f16x4 lds_read_tr16_asm(const void* p) {
  f16x4 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(lds_address(p)));
  return r;
}

// s_waitcnt lgkmcnt(0), ordered before every later use of v (taken as
// in-out operands): every LDS access issued before it is complete.
__device__ inline void lds_reads_done(f16x4 (&v)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]),
                 "+v"(v[6]), "+v"(v[7])
               :
               : "memory");
}
__device__ inline void lds_reads_done(f16x4 (&v)[4]) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]) : : "memory");
}

// D = A B + C on v_mfma_f32_16x16x32_f16: lane (r = lane % 16, q = lane / 16)
// holds A[r][8q .. 8q+7], B[8q .. 8q+7][r] and D[4q .. 4q+3][r].
__device__ inline f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ inline float dot2(f16x2 a, f16x2 b, float c) {
  return __builtin_amdgcn_fdot2(a, b, c, false);
}

}  // namespace nwd
