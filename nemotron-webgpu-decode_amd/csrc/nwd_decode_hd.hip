// nwd_decode_hd.hip — decode at head sizes other than 128: the split
// workgroup of nwd_decode.h built for head sizes 64 and 256, and its padded
// form (rows of fewer dims, a multiple of 8, on the kernel of the next of
// 64, 128, 256). A translation unit of its own, so that its kernels and
// the head-128 ones compile side by side.
#include "nwd_decode.h"
#include "nwd_decode_mfma.h"

namespace nwd {

// Head sizes other than 128: 64 and 256 as they are, other multiples of 8
// up to 256 in the padded form of the next of 64, 128, 256. The same
// per-query-head rule, then one workgroup per KV head, at head size 64 on
// the matrix-core kernel where prefer_mfma says so (nwd_decode_mfma64.hip),
// otherwise on decode_split_kernel. Group 8 above 128 is
// not built (its accumulators and query registers would not fit one lane's
// registers; kernel_group runs it as two groups of 4). Groups 3, 6 and 7 at
// head size 64, and 3 at 256, are built in nwd_decode_groups.hip.
template <int kD, bool kPadD>
static hipError_t launch_decode_hd(const Shape& s, const DecodeArgs& a, const DecodeCall& c,
                                   hipStream_t stream) {
  if constexpr (kD == 64 && !kPadD) {
    if (c.kernel == 1) return launch_mfma_d64(s, a, c, stream);  // nwd_set_decode_kernel
  }
  if ((int64_t)c.batch * s.n_heads * a.nsplit <= kSubSplitMaxWorkgroups) {
    switch (s.group) {
      case 2: return launch_qo<1, 2, kD, kPadD>(s, a, c, stream);
      case 4: return launch_qo<1, 4, kD, kPadD>(s, a, c, stream);
      case 5: return launch_qo<1, 5, kD, kPadD>(s, a, c, stream);
      case 8:
        if constexpr (kD <= kHeadDim) return launch_qo<1, 8, kD, kPadD>(s, a, c, stream);
        break;
      default: break;
    }
  }
  if constexpr (kD == 64 && !kPadD) {  // groups 3, 6, 7: launch_decode_groups
    if (s.group != 3 && s.group != 6 && s.group != 7 && prefer_mfma(s.group, s, c))
      return launch_mfma_d64(s, a, c, stream);
  }
  switch (s.group) {
    case 1: return launch_qo<1, 1, kD, kPadD>(s, a, c, stream);
    case 2: return launch_qo<2, 1, kD, kPadD>(s, a, c, stream);
    case 4: return launch_qo<4, 1, kD, kPadD>(s, a, c, stream);
    case 5: return launch_qo<5, 1, kD, kPadD>(s, a, c, stream);
    case 8:
      if constexpr (kD <= kHeadDim) return launch_qo<8, 1, kD, kPadD>(s, a, c, stream);
      return hipErrorInvalidValue;
    default:
      if constexpr ((kD == 64 || kD == 256) && !kPadD) return launch_decode_groups(s, a, c, stream);
      return hipErrorInvalidValue;
  }
}

hipError_t launch_decode_other(const Shape& s, const DecodeArgs& a, const DecodeCall& c,
                               hipStream_t stream) {
  if (s.head_dim == 64) return launch_decode_hd<64, false>(s, a, c, stream);
  if (s.head_dim == 256) return launch_decode_hd<256, false>(s, a, c, stream);
  if (s.head_dim < 64) return launch_decode_hd<64, true>(s, a, c, stream);
  if (s.head_dim < kHeadDim) return launch_decode_hd<kHeadDim, true>(s, a, c, stream);
  if (s.head_dim > kHeadDim) return launch_decode_hd<256, true>(s, a, c, stream);
  return hipErrorInvalidValue;
}

}  // namespace nwd
