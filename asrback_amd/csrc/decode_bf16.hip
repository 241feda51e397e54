// Decoder-step kernels for bf16 caches (head_dim 64, 128, 256, 512).
#include "decode_kernels.hpp"

namespace asrattn {

hipError_t launch_decode_bf16(const DecodeArgs& a, int head_dim, int group, int waves, bool append,
                              hipStream_t stream) {
  switch (head_dim) {
    case 64: return launch_hd<bf16_raw, 64>(a, group, waves, append, stream);
    case 128: return launch_hd<bf16_raw, 128>(a, group, waves, append, stream);
    case 256: return launch_hd<bf16_raw, 256>(a, group, waves, append, stream);
    case 512: return launch_hd<bf16_raw, 512>(a, group, waves, append, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace asrattn
