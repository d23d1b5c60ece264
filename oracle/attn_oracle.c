/*
 * attn_oracle.c — CPU restatement of the reference decode-attention path.
 *
 * TEST INFRASTRUCTURE ONLY. The HIP library's results are checked against it:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it, and never as the thing measured or shipped. The product path
 * (libnwd_attn.so) does not link, load or call it.
 *
 * What it restates (citations are to the reference repository):
 *   oracle_sparse_attn_f32  kernels/sparse_attn.wgsl:31-114, op for op, in
 *                           f32, emulating the 64-thread workgroup's
 *                           reduction order; the 256-key cap (:29) removed.
 *   oracle_kv_append_f32    kernels/kv_append.wgsl:12-18.
 *   oracle_attn_f64         the same attention in double precision, written
 *                           from the definition softmax(q.K^T*scale).V; used
 *                           as the truth the f32 restatement is pinned to.
 *   oracle_f16_to_f32 /
 *   oracle_f32_to_f16       IEEE-754 binary16 widening (exact) and
 *                           round-to-nearest-even narrowing, written from the
 *                           format definition; the harness widens the fp16
 *                           inputs with these to feed the f32 restatement.
 *
 * Layout follows the reference: Q and O are [n_heads][head_dim]; K and V are
 * token-major [seq][n_kv_heads][head_dim] (kernels/sparse_attn.wgsl:49,107).
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp). Contraction is
 * off so every `a * b + c` of the WGSL rounds twice, as written.
 *
 * How each function is pinned (tests/test_oracle.py):
 *   - oracle_f32_to_f16 / oracle_f16_to_f32: all 65536 fp16 bit patterns
 *     round-trip; narrowing matches numpy's float16 cast on random and edge
 *     values (ties, subnormals, overflow, NaN).
 *   - oracle_kv_append_f32: closed form (bitwise copy into row `seq`,
 *     canary rows untouched).
 *   - oracle_attn_f64: brute force against an independent numpy float64
 *     einsum/softmax; L = 1 gives V[0]; constant V gives that constant;
 *     Q = 0 gives the mean of V; a dominant key selects its V row; joint
 *     permutation of (K, V) rows leaves O unchanged; GQA heads with equal
 *     queries give equal outputs.
 *   - oracle_sparse_attn_f32: within 1e-5 of oracle_attn_f64 at every
 *     length 1..600 tested, and the same special cases.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- fp16 -- */

static float bits_to_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint32_t f32_to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* binary16 -> binary32, exact for every input. */
static float half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ff;
  if (exp == 0x1f) { /* inf / nan: keep the payload in the top bits */
    return bits_to_f32(sign | 0x7f800000u | (man << 13));
  }
  if (exp == 0) {
    if (man == 0) return bits_to_f32(sign);
    /* subnormal: value = man * 2^-24, exact in f32 */
    float v = (float)man * 5.9604644775390625e-08f; /* 2^-24 */
    return sign ? -v : v;
  }
  return bits_to_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

/* binary32 -> binary16, round to nearest, ties to even. */
static uint16_t float_to_half(float f) {
  uint32_t u = f32_to_bits(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t exp = (u >> 23) & 0xff;
  uint32_t man = u & 0x7fffffu;
  if (exp == 0xff) { /* inf or nan (quiet the nan, keep it a nan) */
    if (man == 0) return sign | 0x7c00u;
    return sign | 0x7e00u | (uint16_t)(man >> 13);
  }
  int32_t e = (int32_t)exp - 127; /* unbiased */
  if (e > 15) return sign | 0x7c00u; /* overflow: |f| >= 2^16 */
  if (e >= -14) {
    /* normal range: 10 kept bits, 13 dropped bits */
    uint32_t m = man;
    uint32_t kept = m >> 13;
    uint32_t rest = m & 0x1fffu;
    uint32_t hexp = (uint32_t)(e + 15);
    uint32_t r = (hexp << 10) | kept;
    if (rest > 0x1000u || (rest == 0x1000u && (kept & 1u))) r += 1; /* may carry into exp / inf */
    return sign | (uint16_t)r;
  }
  /* subnormal or zero: value = m24 * 2^(e-23) with the implicit bit */
  if (e < -25) return sign; /* below half of the smallest subnormal */
  uint32_t m24 = man | 0x800000u;
  /* result units are 2^-24; shift = (-24) - (e - 23) = -1 - e */
  int shift = -1 - e; /* 14 .. 24 */
  uint32_t kept = m24 >> shift;
  uint32_t rest = m24 & ((1u << shift) - 1u);
  uint32_t half = 1u << (shift - 1);
  if (rest > half || (rest == half && (kept & 1u))) kept += 1; /* may become the smallest normal */
  return sign | (uint16_t)kept;
}

void oracle_f16_to_f32(const uint16_t* src, float* dst, int64_t n) {
  for (int64_t i = 0; i < n; i++) dst[i] = half_to_float(src[i]);
}

void oracle_f32_to_f16(const float* src, uint16_t* dst, int64_t n) {
  for (int64_t i = 0; i < n; i++) dst[i] = float_to_half(src[i]);
}

/* ----------------------------------------------------------- kv_append -- */

/* kernels/kv_append.wgsl:12-18: cache[seq * n + i] = src[i], n = n_kv * hd.
 * The reference's f32 copy is a bit copy. */
void oracle_kv_append_f32(const float* src, float* cache, uint32_t seq,
                          uint32_t n_kv, uint32_t hd) {
  uint32_t n = n_kv * hd;
  for (uint32_t i = 0; i < n; i++) cache[(uint64_t)seq * n + i] = src[i];
}

/* ---------------------------------------------------- attention, f32 ---- */

#define ORACLE_WG 64u
static const float ORACLE_NEG_INF = -3.4028234663852886e38f; /* sparse_attn.wgsl:26 */

/* One workgroup of kernels/sparse_attn.wgsl:31-114 (query head h). `scores`
 * holds seq floats (the WGSL array is capped at 256, :29; here it is not). */
static void sparse_attn_head(const float* Q, const float* K, const float* V,
                             float* O, uint32_t n_heads, uint32_t n_kv_heads,
                             uint32_t hd, uint32_t seq, uint32_t h,
                             float* scores) {
  float red[ORACLE_WG];
  uint32_t group = n_heads / n_kv_heads;  /* :38 */
  uint32_t hkv = h / group;               /* :39 */
  float scale = 1.0f / sqrtf((float)hd);  /* :42 inverseSqrt(f32(hd)) */
  uint32_t qOff = h * hd;                 /* :43 */

  /* phase 1, :45-58: each "thread" tid scores keys t = tid, tid+64, ... */
  for (uint32_t t = 0; t < seq; t++) {
    float dot = 0.0f;
    uint32_t kOff = (t * n_kv_heads + hkv) * hd; /* :49 */
    for (uint32_t d = 0; d < hd; d++) dot = dot + Q[qOff + d] * K[kOff + d];
    scores[t] = dot * scale; /* :56 */
  }

  /* phase 2, :61-77: per-thread strided max, then the LDS tree 32 -> 1 */
  for (uint32_t tid = 0; tid < ORACLE_WG; tid++) {
    float m = ORACLE_NEG_INF;
    for (uint32_t t = tid; t < seq; t += ORACLE_WG) m = fmaxf(m, scores[t]);
    red[tid] = m;
  }
  for (uint32_t stride = ORACLE_WG / 2; stride > 0; stride /= 2)
    for (uint32_t tid = 0; tid < stride; tid++)
      red[tid] = fmaxf(red[tid], red[tid + stride]);
  float row_max = red[0];

  /* phase 3, :80-98: p = exp(s - max) stored back; strided sums; tree */
  for (uint32_t tid = 0; tid < ORACLE_WG; tid++) {
    float s = 0.0f;
    for (uint32_t t = tid; t < seq; t += ORACLE_WG) {
      float p = expf(scores[t] - row_max);
      scores[t] = p;
      s = s + p;
    }
    red[tid] = s;
  }
  for (uint32_t stride = ORACLE_WG / 2; stride > 0; stride /= 2)
    for (uint32_t tid = 0; tid < stride; tid++)
      red[tid] = red[tid] + red[tid + stride];
  float inv_sum = 1.0f / red[0]; /* :98 */

  /* phase 4, :100-113: O[h][d] = sum_t (p_t * inv_sum) * V[t][hkv][d] */
  for (uint32_t d = 0; d < hd; d++) {
    float acc = 0.0f;
    for (uint32_t tt = 0; tt < seq; tt++) {
      uint32_t vOff = (tt * n_kv_heads + hkv) * hd; /* :107 */
      acc = acc + scores[tt] * inv_sum * V[vOff + d]; /* :108, left to right */
    }
    O[qOff + d] = acc; /* :111 */
  }
}

/* kernels/sparse_attn.wgsl main dispatched with n_heads workgroups
 * (engine/runtime.js:391). Returns 0, or -1 if seq == 0 or the head counts
 * do not divide (the WGSL would divide by zero / mis-index there). */
int oracle_sparse_attn_f32(const float* Q, const float* K, const float* V,
                           float* O, uint32_t n_heads, uint32_t n_kv_heads,
                           uint32_t head_dim, uint32_t seq) {
  if (seq == 0 || n_kv_heads == 0 || n_heads % n_kv_heads != 0) return -1;
  float* scores = (float*)malloc(sizeof(float) * seq);
  if (!scores) return -1;
  for (uint32_t h = 0; h < n_heads; h++)
    sparse_attn_head(Q, K, V, O, n_heads, n_kv_heads, head_dim, seq, h, scores);
  free(scores);
  return 0;
}

/* Same result, workgroups spread over `threads` OpenMP threads (0 = all).
 * Used to time the reference algorithm on all host cores. */
int oracle_sparse_attn_f32_mt(const float* Q, const float* K, const float* V,
                              float* O, uint32_t n_heads, uint32_t n_kv_heads,
                              uint32_t head_dim, uint32_t seq, int threads) {
  if (seq == 0 || n_kv_heads == 0 || n_heads % n_kv_heads != 0) return -1;
  int bad = 0;
#ifdef _OPENMP
  if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for num_threads(threads) schedule(static) reduction(| : bad)
#endif
  for (int32_t h = 0; h < (int32_t)n_heads; h++) {
    float* scores = (float*)malloc(sizeof(float) * seq);
    if (!scores) {
      bad |= 1;
      continue;
    }
    sparse_attn_head(Q, K, V, O, n_heads, n_kv_heads, head_dim, seq,
                     (uint32_t)h, scores);
    free(scores);
  }
  (void)threads;
  return bad ? -1 : 0;
}

int oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ---------------------------------------------------- attention, f64 ---- */

/* Textbook definition in double: O[h] = sum_t softmax_t(scale * q_h . k_t) v_t
 * with q_h = Q[h], k_t = K[t][h / (H/Hkv)], v_t = V[t][h / (H/Hkv)].
 * `scale` <= 0 means 1/sqrt(head_dim). */
int oracle_attn_f64(const float* Q, const float* K, const float* V, double* O,
                    uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                    uint32_t seq, double scale) {
  if (seq == 0 || n_kv_heads == 0 || n_heads % n_kv_heads != 0) return -1;
  if (scale <= 0.0) scale = 1.0 / sqrt((double)head_dim);
  double* s = (double*)malloc(sizeof(double) * seq);
  if (!s) return -1;
  uint32_t group = n_heads / n_kv_heads;
  for (uint32_t h = 0; h < n_heads; h++) {
    uint32_t hkv = h / group;
    const float* q = Q + (uint64_t)h * head_dim;
    double mx = -INFINITY;
    for (uint32_t t = 0; t < seq; t++) {
      const float* k = K + ((uint64_t)t * n_kv_heads + hkv) * head_dim;
      double dot = 0.0;
      for (uint32_t d = 0; d < head_dim; d++) dot += (double)q[d] * (double)k[d];
      s[t] = dot * scale;
      if (s[t] > mx) mx = s[t];
    }
    double sum = 0.0;
    for (uint32_t t = 0; t < seq; t++) {
      s[t] = exp(s[t] - mx);
      sum += s[t];
    }
    double* o = O + (uint64_t)h * head_dim;
    for (uint32_t d = 0; d < head_dim; d++) o[d] = 0.0;
    for (uint32_t t = 0; t < seq; t++) {
      const float* v = V + ((uint64_t)t * n_kv_heads + hkv) * head_dim;
      double w = s[t] / sum;
      for (uint32_t d = 0; d < head_dim; d++) o[d] += w * (double)v[d];
    }
  }
  free(s);
  return 0;
}
