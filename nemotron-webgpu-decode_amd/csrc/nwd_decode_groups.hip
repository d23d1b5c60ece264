// nwd_decode_groups.hip — decode at head size 128 for groups of 3, 6 and 7
// query heads per KV head (e.g. Qwen2.5-7B's 28q/4kv), on the same two split
// kernels as the other groups: the dot-product one of nwd_decode.h and the
// matrix-core one of nwd_decode_mfma.h, whose MFMA columns past the group
// hold zero queries. A translation unit of its own, so that these kernels
// and the other groups' compile side by side.
#include "nwd_decode_mfma.h"

namespace nwd {

hipError_t launch_decode_groups(const Shape& s, const DecodeArgs& a, const DecodeCall& c,
                                hipStream_t stream) {
  switch (s.group) {
    case 3: return launch_decode_128<3>(s, a, c, stream);
    case 6: return launch_decode_128<6>(s, a, c, stream);
    case 7: return launch_decode_128<7>(s, a, c, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace nwd
