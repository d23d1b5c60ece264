// nwd_mfma_ceiling.hip — what the matrix cores and the vector ALUs of gfx950
// deliver under a full load (measurement only; built into
// lib/libnwd_bench.so, not the product library).
//
// 256 workgroups of 512 threads (two wavefronts per SIMD, as the prefill
// kernel runs) each run `iters` rounds of one of:
//   mode 0: 32 v_mfma_f32_16x16x32_f16 per wavefront (8 independent chains);
//   mode 1: 16 v_exp_f32 per wavefront (8 independent chains), the prefill
//           kernel's one exponential per score at its ratio of two MFMAs per
//           exponential;
//   mode 2: modes 0 and 1 in the same round;
//   mode 3: 32 v_fma_f32 per wavefront (8 independent chains), about the
//           prefill's ordinary VALU work (conversions, row sums, address
//           arithmetic) per MFMA;
//   mode 4: modes 0 and 3 in the same round.
// Mode 0's FLOP rate is the MFMA ceiling under load; the time of modes 2
// and 4 against their parts says how much of each kind of vector work hides
// under the MFMAs.
// Thread 0 of workgroup 0 also reads the shader clock counter (s_memtime)
// and the 100 MHz constant clock (s_memrealtime) around its rounds, so the
// clock the chip runs at under each load is known.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 512;
constexpr int kBlocks = 256;

template <int kMode>
__global__ __launch_bounds__(kThreads) void ceiling_kernel(int iters, float* __restrict__ out,
                                                           unsigned long long* __restrict__ clk) {
  const int t = threadIdx.x;
  f16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = (f16)((t + i) * 1e-3f);
    b[i] = (f16)((t - i) * 1e-3f);
  }
  f32x4 acc[8];
  float x[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    x[i] = -(t + i) * 1e-4f;
  }
  const unsigned long long c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
    if constexpr (kMode == 0 || kMode == 2 || kMode == 4) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[i], 0, 0, 0);
    }
    if constexpr (kMode == 1 || kMode == 2) {
      // exp2 of a value in (-1, 0] stays in (0.5, 1]; minus 1 keeps the
      // chain's argument in (-0.5, 0].
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = __builtin_amdgcn_exp2f(x[i]) - 1.f;
    }
    if constexpr (kMode == 3 || kMode == 4) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = fmaf(x[i], 0.999f, 1e-3f);
    }
  }
  const unsigned long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  float r = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) r += x[i] + acc[i][0] + acc[i][1] + acc[i][2] + acc[i][3];
  out[blockIdx.x * kThreads + t] = r;
  if (blockIdx.x == 0 && t == 0) {
    clk[0] = c1 - c0;
    clk[1] = r1 - r0;
  }
}

}  // namespace

// Runs one launch of mode 0 .. 4 (see above) with `iters` rounds. out
// needs 256 * 512 floats, clk 2 values (shader-clock ticks and 100 MHz
// ticks of workgroup 0's rounds). Returns a hipError_t code.
extern "C" int nwd_bench_mfma_ceiling(int mode, int iters, float* out, unsigned long long* clk,
                                      void* stream) {
  if (!out || !clk || iters < 1 || mode < 0 || mode > 4) return (int)hipErrorInvalidValue;
  const hipStream_t s = (hipStream_t)stream;
  if (mode == 0) ceiling_kernel<0><<<kBlocks, kThreads, 0, s>>>(iters, out, clk);
  if (mode == 1) ceiling_kernel<1><<<kBlocks, kThreads, 0, s>>>(iters, out, clk);
  if (mode == 2) ceiling_kernel<2><<<kBlocks, kThreads, 0, s>>>(iters, out, clk);
  if (mode == 3) ceiling_kernel<3><<<kBlocks, kThreads, 0, s>>>(iters, out, clk);
  if (mode == 4) ceiling_kernel<4><<<kBlocks, kThreads, 0, s>>>(iters, out, clk);
  return (int)hipGetLastError();
}
