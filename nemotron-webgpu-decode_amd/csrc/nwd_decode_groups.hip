// nwd_decode_groups.hip — decode for groups of 3, 6 and 7 query heads per
// KV head, at head size 128 (e.g. Qwen2.5-7B's 28q/4kv) on the same two
// split kernels as the other groups, the dot-product one of nwd_decode.h and
// the matrix-core one of nwd_decode_mfma.h (whose MFMA columns past the
// group hold zero queries), at head size 64 (e.g. Qwen2.5-0.5B's 14q/2kv)
// on both kernels built for that size, and group 3 at head size 256 on the
// dot-product kernel built for it. A translation unit
// of its own, so that these kernels and the other groups' compile side by
// side.
#include "nwd_decode_mfma.h"

namespace nwd {

// Head size 64: the per-query-head form when it fits the chip, else one
// workgroup per KV head, on the matrix-core kernel where prefer_mfma says
// so, as for the other groups there (nwd_decode_hd.hip).
template <int G>
static hipError_t launch_decode_64(const Shape& s, const DecodeArgs& a, const DecodeCall& c,
                                   hipStream_t stream) {
  if (c.kernel == 1) return launch_mfma_d64(s, a, c, stream);  // nwd_set_decode_kernel
  if ((int64_t)c.batch * s.n_heads * a.nsplit <= kSubSplitMaxWorkgroups)
    return launch_qo<1, G, 64, false>(s, a, c, stream);
  if (prefer_mfma(G, s, c)) return launch_mfma_d64(s, a, c, stream);
  return launch_qo<G, 1, 64, false>(s, a, c, stream);
}

hipError_t launch_decode_groups(const Shape& s, const DecodeArgs& a, const DecodeCall& c,
                                hipStream_t stream) {
  if (s.head_dim == 256) {  // group 3, on the dot-product kernel built for 256
    if (s.group != 3) return hipErrorInvalidValue;
    if ((int64_t)c.batch * s.n_heads * a.nsplit <= kSubSplitMaxWorkgroups)
      return launch_qo<1, 3, 256, false>(s, a, c, stream);
    return launch_qo<3, 1, 256, false>(s, a, c, stream);
  }
  if (s.head_dim == 64) {
    switch (s.group) {
      case 3: return launch_decode_64<3>(s, a, c, stream);
      case 6: return launch_decode_64<6>(s, a, c, stream);
      case 7: return launch_decode_64<7>(s, a, c, stream);
      default: return hipErrorInvalidValue;
    }
  }
  if (s.head_dim != kHeadDim) return hipErrorInvalidValue;
  switch (s.group) {
    case 3: return launch_decode_128<3>(s, a, c, stream);
    case 6: return launch_decode_128<6>(s, a, c, stream);
    case 7: return launch_decode_128<7>(s, a, c, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace nwd
