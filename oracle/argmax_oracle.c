/*
 * argmax_oracle.c — CPU restatement of the reference's greedy token pick.
 *
 * TEST INFRASTRUCTURE ONLY. The HIP library's results are checked against it:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it, and never as the thing measured or shipped. The product path
 * (libnwd_attn.so) does not link, load or call it.
 *
 * What it restates (citations are to the reference repository):
 *   oracle_argmax_ref    kernels/argmax_partial.wgsl:16-52 dispatched as 256
 *                        workgroups of 256 threads over slices of
 *                        n_slice = ceil(n / 256) logits (engine/runtime.js:
 *                        209,398), then kernels/argmax_merge.wgsl:8-42 over
 *                        the 256 (value, index) partials (:399). Op for op:
 *                        each thread walks i = start + tid, + 256, ... keeping
 *                        the first value strictly greater than its running
 *                        best (initially -3.402823466e38 at index `start`);
 *                        the workgroup tree keeps the lower thread on ties;
 *                        the merge starts from (-3.402823466e38, 0), reads one
 *                        partial per thread and reduces the same way.
 *
 * Consequences the tests check independently (tests/test_argmax_oracle.py,
 * tests/argmax_cases.py): the result is the index of the largest value
 * strictly above -3.402823466e38 (NaN never wins), or 0 if no value
 * qualifies. Ties go to the smaller step within a thread, and in the two
 * left-preferring trees to the smaller bit-reversed thread / workgroup
 * position (two tied entries meet at their lowest differing position bit).
 */
#include <stdint.h>
#include <string.h>

static const float kNegFltMax = -3.402823466e38f;

/* argmax_partial.wgsl main for workgroup `wg`. */
static void partial(const float* X, uint32_t n, uint32_t n_slice, uint32_t wg, float* out_v,
                    uint32_t* out_i) {
  enum { WG = 256 };
  float best_v[WG];
  uint32_t best_i[WG];
  const uint32_t start = wg * n_slice;
  const uint32_t end = (start + n_slice < n) ? start + n_slice : n;
  for (uint32_t tid = 0; tid < WG; ++tid) {
    float bv = kNegFltMax;
    uint32_t bi = start;
    for (uint32_t i = start + tid; i < end; i += WG) {
      const float v = X[i];
      if (v > bv) {
        bv = v;
        bi = i;
      }
    }
    best_v[tid] = bv;
    best_i[tid] = bi;
  }
  for (uint32_t stride = WG / 2; stride > 0; stride /= 2)
    for (uint32_t tid = 0; tid < stride; ++tid)
      if (best_v[tid + stride] > best_v[tid]) {
        best_v[tid] = best_v[tid + stride];
        best_i[tid] = best_i[tid + stride];
      }
  *out_v = best_v[0];
  *out_i = best_i[0];
}

/* The token index the reference picks for logits X[n] (n >= 1). */
uint32_t oracle_argmax_ref(const float* X, uint32_t n) {
  enum { WG = 256, N_WG = 256 };
  const uint32_t n_slice = (n + N_WG - 1) / N_WG;
  float pv[N_WG];
  uint32_t pi[N_WG];
  for (uint32_t wg = 0; wg < N_WG; ++wg) partial(X, n, n_slice, wg, &pv[wg], &pi[wg]);
  /* argmax_merge.wgsl main: thread tid reads partial tid (s < 256). */
  float best_v[WG];
  uint32_t best_i[WG];
  for (uint32_t tid = 0; tid < WG; ++tid) {
    float bv = kNegFltMax;
    uint32_t bi = 0;
    const float v = pv[tid];
    if (v > bv) {
      bv = v;
      bi = pi[tid];
    }
    best_v[tid] = bv;
    best_i[tid] = bi;
  }
  for (uint32_t stride = WG / 2; stride > 0; stride /= 2)
    for (uint32_t tid = 0; tid < stride; ++tid)
      if (best_v[tid + stride] > best_v[tid]) {
        best_v[tid] = best_v[tid + stride];
        best_i[tid] = best_i[tid + stride];
      }
  return best_i[0];
}
