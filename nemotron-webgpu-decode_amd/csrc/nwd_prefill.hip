// nwd_prefill.hip — the prefill launch (nwd_prefill.h): the kernels of head
// size 128 and of the multiples of 8 between 64 and 128 on rows padded to
// 128; head sizes up to 64 go to nwd_prefill_d64.hip and those above 128 to
// nwd_prefill_wide.hip.
#include "nwd_prefill.h"

namespace nwd {

template <int G>
static hipError_t launch_prefill_g(const Shape& s, const void* q, const void* kc, const void* vc,
                                   const int32_t* pos0, void* out, int batch, int n_new,
                                   int max_len, const Workspace& ws, int r, hipStream_t stream) {
  if (s.head_dim == kHeadDim)
    return launch_prefill_p<G, false>(s, q, kc, vc, pos0, out, batch, n_new, max_len, ws, r, stream);
  return launch_prefill_p<G, true>(s, q, kc, vc, pos0, out, batch, n_new, max_len, ws, r, stream);
}

bool prefill_head_dim(int head_dim) {
  return head_dim >= 8 && head_dim <= 256 && head_dim % 8 == 0;
}

hipError_t launch_prefill(const Shape& s0, const void* q, const void* k_cache,
                          const void* v_cache, const int32_t* pos0, void* out,
                          int batch, int n_new, int max_len, const Workspace& ws,
                          hipStream_t stream) {
  if (!prefill_head_dim(s0.head_dim)) return hipErrorInvalidValue;
  if (prefill_wide_head_dim(s0.head_dim))  // above 128 (nwd_prefill_wide.hip)
    return launch_prefill_wide(s0, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws,
                               stream);
  // A group the kernel is not built for runs as r groups of a built size per
  // KV head (kernel_group): n_kv * r KV heads of that group, each group's
  // workgroups reading its KV head's rows.
  int r = 1;
  Shape s = s0;
  s.group = kernel_group(s0.head_dim, s0.group, &r);
  s.n_kv = s0.n_kv * r;
  if (s.head_dim <= 64)  // nwd_prefill_d64.hip
    return launch_prefill_d64(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r,
                              stream);
  switch (s.group) {
    case 1: return launch_prefill_g<1>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    case 2: return launch_prefill_g<2>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    case 4: return launch_prefill_g<4>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    case 5: return launch_prefill_g<5>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    case 8: return launch_prefill_g<8>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    default: break;
  }
  if (s.head_dim != kHeadDim) return hipErrorInvalidValue;
  switch (s.group) {  // built at head size 128 (and 64, above)
    case 3: return launch_prefill_p<3, false>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    case 6: return launch_prefill_p<6, false>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    case 7: return launch_prefill_p<7, false>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace nwd
