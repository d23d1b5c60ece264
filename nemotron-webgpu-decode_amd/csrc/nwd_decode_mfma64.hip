// nwd_decode_mfma64.hip — the matrix-core split kernel of nwd_decode_mfma.h
// at head size 64 (decode_mfma_d64_kernel), groups 1 to 8. A translation
// unit of its own, so that these kernels and the others compile side by
// side.
#include "nwd_decode_mfma.h"

namespace nwd {

hipError_t launch_mfma_d64(const Shape& s, const DecodeArgs& a, const DecodeCall& c,
                           hipStream_t stream) {
  if (s.head_dim != 64) return hipErrorInvalidValue;
  switch (s.group) {
    case 1: return launch_mfma<1, 64>(s, a, c, stream);
    case 2: return launch_mfma<2, 64>(s, a, c, stream);
    case 3: return launch_mfma<3, 64>(s, a, c, stream);
    case 4: return launch_mfma<4, 64>(s, a, c, stream);
    case 5: return launch_mfma<5, 64>(s, a, c, stream);
    case 6: return launch_mfma<6, 64>(s, a, c, stream);
    case 7: return launch_mfma<7, 64>(s, a, c, stream);
    case 8: return launch_mfma<8, 64>(s, a, c, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace nwd
