// nwd_prefill_d64.hip — the prefill at head sizes up to 64: the kernel of
// nwd_prefill.h built for 64-dim rows (prefill_d64_kernel), on rows padded
// with zeros to 64 dims below it. A translation unit of its own, so that
// these kernels and the head-128 ones compile side by side.
#include "nwd_prefill.h"

namespace nwd {

template <int G>
static hipError_t launch_prefill_64g(const Shape& s, const void* q, const void* kc, const void* vc,
                                     const int32_t* pos0, void* out, int batch, int n_new,
                                     int max_len, const Workspace& ws, int r, hipStream_t stream) {
  if (s.head_dim == 64)
    return launch_prefill_p<G, false, 64>(s, q, kc, vc, pos0, out, batch, n_new, max_len, ws, r, stream);
  return launch_prefill_p<G, true, 64>(s, q, kc, vc, pos0, out, batch, n_new, max_len, ws, r, stream);
}

hipError_t launch_prefill_d64(const Shape& s, const void* q, const void* k_cache,
                              const void* v_cache, const int32_t* pos0, void* out, int batch,
                              int n_new, int max_len, const Workspace& ws, int r,
                              hipStream_t stream) {
  if (s.head_dim > 64 || s.head_dim < 8 || s.head_dim % 8 != 0) return hipErrorInvalidValue;
  switch (s.group) {
    case 1: return launch_prefill_64g<1>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    case 2: return launch_prefill_64g<2>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    case 3: return launch_prefill_64g<3>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    case 4: return launch_prefill_64g<4>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    case 5: return launch_prefill_64g<5>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    case 6: return launch_prefill_64g<6>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    case 7: return launch_prefill_64g<7>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    case 8: return launch_prefill_64g<8>(s, q, k_cache, v_cache, pos0, out, batch, n_new, max_len, ws, r, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace nwd
