/*
 * q4_oracle.c — CPU restatement of the reference's 4-bit GEMV.
 *
 * TEST INFRASTRUCTURE ONLY. The HIP library's results are checked against it:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it, and never as the thing measured or shipped. The product path
 * (libnwd_attn.so) does not link, load or call it.
 *
 * What it restates (citations are to the reference repository):
 *   oracle_q4_gemv_f32   kernels/matmul_nbits_sg.wgsl:81-137, op for op in
 *                        f32: one 256-thread workgroup per 4 output columns
 *                        (dispatch ceil(N/4), engine/runtime.js:359-361),
 *                        thread tid accumulating blocks tid, tid+256, ...;
 *                        dequant_dot (:29-64) as written; the 32-lane
 *                        subgroup butterfly sg_sum_v4 (:66-74) in lane order;
 *                        the 8 subgroup partials summed by thread 0 in order
 *                        (:119-124); epilogue 1 = relu2 (:76-79, :125-127).
 *                        The subgroup size is 32, as the kernel's
 *                        sg_partials[8] and `tid >> 5` assume.
 *   oracle_q4_dequant    the dequantised weight (nib - zp) * scale of every
 *                        element, [N][K], as dequant_dot forms it.
 *
 * Weight format (engine/weights.js:99-104, engine/weight-index.json): for a
 * [K -> N] projection, quant is uint8 [N][n_blocks][16] (block = 32 weights
 * along K, element 2j in the low nibble of byte j, 2j+1 in the high nibble),
 * scales float32 [N][n_blocks], zp 4-bit zero points packed in order of the
 * flat index col * n_blocks + blk (low nibble first) — load_zp (:24-27).
 *
 * How each function is pinned (tests/test_q4_oracle.py): against an
 * independent numpy float64 dequantise-and-multiply; with one-hot
 * activations (the output is exactly (nib - zp) * scale of that element,
 * which fixes the nibble order, the block index and the zero-point index);
 * zero points equal to every nibble give exactly 0; relu2 is the square of
 * the clamped plain result; N not a multiple of 4 and n_blocks above 256
 * (the strided block loop).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

typedef struct {
  float x, y, z, w;
} v4;

static v4 v4_add(v4 a, v4 b) { return (v4){a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w}; }

/* WGSL dot(a, b): a.x*b.x + a.y*b.y + a.z*b.z + a.w*b.w, left to right. */
static float dot4(v4 a, v4 b) {
  float s = a.x * b.x;
  s = s + a.y * b.y;
  s = s + a.z * b.z;
  s = s + a.w * b.w;
  return s;
}

static uint32_t word_le(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* load_zp (:24-27): nibble col * n_blocks + blk of the packed array. The
 * WGSL reads it from little-endian u32 words, (zp[nib / 8] >> (nib % 8) * 4)
 * & 15, which is byte nib / 2, low nibble for even nib; reading the byte
 * avoids touching the padding the reference's 4-byte-aligned buffer has. */
static float load_zp(const uint8_t* zp, uint32_t col, uint32_t blk, uint32_t n_blocks) {
  const uint32_t nib = col * n_blocks + blk;
  const uint32_t byte = zp[nib / 2u];
  return (float)((nib & 1u) ? (byte >> 4) : (byte & 15u));
}

/* One 32-bit word of packed nibbles -> the two dequantised vec4s d0, d1
 * (:38-42): lo = unpack4xU8(w & 0x0F0F0F0F), hi = unpack4xU8((w >> 4) &
 * 0x0F0F0F0F), d0 = (lo.x, hi.x, lo.y, hi.y), d1 = (lo.z, hi.z, lo.w, hi.w),
 * each (v - z) * s. */
static void dequant_word(uint32_t w, float s, float z, v4* d0, v4* d1) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  const float l0 = (float)(lo & 255u), l1 = (float)((lo >> 8) & 255u);
  const float l2 = (float)((lo >> 16) & 255u), l3 = (float)((lo >> 24) & 255u);
  const float h0 = (float)(hi & 255u), h1 = (float)((hi >> 8) & 255u);
  const float h2 = (float)((hi >> 16) & 255u), h3 = (float)((hi >> 24) & 255u);
  *d0 = (v4){(l0 - z) * s, (h0 - z) * s, (l1 - z) * s, (h1 - z) * s};
  *d1 = (v4){(l2 - z) * s, (h2 - z) * s, (l3 - z) * s, (h3 - z) * s};
}

/* dequant_dot (:29-64): four words, each `acc += dot(a_even, d0) +
 * dot(a_odd, d1)`. */
static float dequant_dot(const uint8_t* packed, float scale, float zero, const float* a) {
  float acc = 0.0f;
  for (int k = 0; k < 4; ++k) {
    v4 d0, d1;
    dequant_word(word_le(packed + 4 * k), scale, zero, &d0, &d1);
    const v4 ae = {a[8 * k + 0], a[8 * k + 1], a[8 * k + 2], a[8 * k + 3]};
    const v4 ao = {a[8 * k + 4], a[8 * k + 5], a[8 * k + 6], a[8 * k + 7]};
    acc = acc + (dot4(ae, d0) + dot4(ao, d1));
  }
  return acc;
}

static float relu2(float v) {
  const float r = v > 0.0f ? v : 0.0f;
  return r * r;
}

/* One workgroup (4 columns) of matmul_nbits_sg.wgsl main. */
static void gemv_workgroup(const float* A, const uint8_t* quant, const float* scales,
                           const uint8_t* zp, float* Y, uint32_t N, uint32_t n_blocks,
                           uint32_t epilogue, uint32_t wg) {
  enum { WG = 256, N_COLS = 4, SG = 32 };
  const uint32_t col0 = wg * N_COLS;
  v4 acc[WG];
  for (uint32_t tid = 0; tid < WG; ++tid) {
    v4 a = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t blk = tid; blk < n_blocks; blk += WG) {
      const float* ab = A + (size_t)blk * 32u;
      for (uint32_t r = 0; r < N_COLS; ++r) {
        const uint32_t col = col0 + r;
        if (col < N) {
          const size_t cb = (size_t)col * n_blocks + blk;
          const float d = dequant_dot(quant + cb * 16u, scales[cb], load_zp(zp, col, blk, n_blocks), ab);
          if (r == 0) a.x = a.x + d;
          else if (r == 1) a.y = a.y + d;
          else if (r == 2) a.z = a.z + d;
          else a.w = a.w + d;
        }
      }
    }
    acc[tid] = a;
  }
  /* sg_sum_v4: x = x + shuffleXor(x, m) for m = 1, 2, 4, 8, 16, every lane
   * of a 32-lane subgroup at once. */
  for (uint32_t m = 1; m < SG; m <<= 1) {
    v4 nxt[WG];
    for (uint32_t t = 0; t < WG; ++t) nxt[t] = v4_add(acc[t], acc[t ^ m]);
    memcpy(acc, nxt, sizeof acc);
  }
  v4 tot = {0.0f, 0.0f, 0.0f, 0.0f};
  for (uint32_t i = 0; i < WG / SG; ++i) tot = v4_add(tot, acc[i * SG]);
  if (epilogue == 1u) tot = (v4){relu2(tot.x), relu2(tot.y), relu2(tot.z), relu2(tot.w)};
  if (col0 + 0u < N) Y[col0 + 0u] = tot.x;
  if (col0 + 1u < N) Y[col0 + 1u] = tot.y;
  if (col0 + 2u < N) Y[col0 + 2u] = tot.z;
  if (col0 + 3u < N) Y[col0 + 3u] = tot.w;
}

/* Y[N] = epilogue(dequant(W)[N][K] . A[K]), K = 32 * n_blocks. Returns 0, or
 * -1 if K is not 32 * n_blocks. `threads` > 1 runs workgroups in parallel
 * (each output column is computed by exactly one workgroup, so the result
 * does not depend on it). */
int oracle_q4_gemv_f32(const float* A, const uint8_t* quant, const float* scales,
                       const uint8_t* zp, float* Y, uint32_t K, uint32_t N, uint32_t n_blocks,
                       uint32_t epilogue, int threads) {
  if (K != 32u * n_blocks) return -1;
  const int64_t n_wg = ((int64_t)N + 3) / 4;
#ifdef _OPENMP
  if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) num_threads(threads)
#else
  (void)threads;
#endif
  for (int64_t wg = 0; wg < n_wg; ++wg)
    gemv_workgroup(A, quant, scales, zp, Y, N, n_blocks, epilogue, (uint32_t)wg);
  return 0;
}

/* W[N][K] = (nib - zp) * scale, as dequant_dot forms each element. */
void oracle_q4_dequant(const uint8_t* quant, const float* scales, const uint8_t* zp, float* W,
                       uint32_t N, uint32_t n_blocks) {
  const uint32_t K = 32u * n_blocks;
  for (uint32_t col = 0; col < N; ++col)
    for (uint32_t blk = 0; blk < n_blocks; ++blk) {
      const size_t cb = (size_t)col * n_blocks + blk;
      const float s = scales[cb], z = load_zp(zp, col, blk, n_blocks);
      for (int k = 0; k < 4; ++k) {
        v4 d0, d1;
        dequant_word(word_le(quant + cb * 16u + 4 * k), s, z, &d0, &d1);
        float* w = W + (size_t)col * K + blk * 32u + 8 * k;
        w[0] = d0.x; w[1] = d0.y; w[2] = d0.z; w[3] = d0.w;
        w[4] = d1.x; w[5] = d1.y; w[6] = d1.z; w[7] = d1.w;
      }
    }
}
