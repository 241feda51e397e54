// Launchers of the attention kernels; the C ABI (api.hip) validates the
// parameters before calling them.
#pragma once

#include <hip/hip_runtime.h>

#include "asrattn.h"

namespace asrattn {

// Decoder step: split-K pass (and, for num_splits > 1, the combine pass).
// ws_o / ws_ml are the workspace: float[batch][heads_q][splits][head_dim] and
// float[batch][heads_q][splits][2].
hipError_t launch_decode(const asrattn_decode_params& p, int splits, float* ws_o, float* ws_ml,
                         hipStream_t stream);
bool decode_supported(int dtype, int head_dim, int group);

// Multi-row forward on matrix cores (bf16, head_dim 64 or 128).
hipError_t launch_fwd_mfma(const asrattn_fwd_params& p, hipStream_t stream);
bool fwd_mfma_supported(int dtype, int head_dim);

// Multi-row forward on the vector ALUs (fp32 or bf16, head_dim 64 or 128):
// the fp32 path and the reference-precision check of the matrix-core kernel.
hipError_t launch_fwd_valu(const asrattn_fwd_params& p, hipStream_t stream);
bool fwd_valu_supported(int dtype, int head_dim);

}  // namespace asrattn
