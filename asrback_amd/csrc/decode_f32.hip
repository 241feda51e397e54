// Decoder-step kernels for fp32 caches (head_dim 64, 128, 256).
#include "decode_kernels.hpp"

namespace asrattn {

hipError_t launch_decode_f32(const DecodeArgs& a, int head_dim, int group, int waves, bool append,
                             hipStream_t stream) {
  switch (head_dim) {
    case 64: return launch_hd<float, 64>(a, group, waves, append, stream);
    case 128: return launch_hd<float, 128>(a, group, waves, append, stream);
    case 256: return launch_hd<float, 256>(a, group, waves, append, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace asrattn
