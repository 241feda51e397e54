// Arguments of the decoder-step kernels (decode_kernels.hpp), shared by the
// per-dtype launch units.
#pragma once

#include "common.hpp"

namespace asrattn {

struct DecodeArgs {
  asrattn_decode_params p;
  asrattn_append_params ap;  // the fused prologue (append variant only)
  asrattn_paged_kv pk;       // the page table (paged variant only)
  int page_shift;            // log2(pk.page_size)
  float* ws_o;   // [batch][heads_q][splits][head_dim]
  float* ws_ml;  // [batch][heads_q][splits][2]
  int splits;
  float c;  // scale * log2(e)
};

// Launch units, one per element type: head_dim, query heads per kv head and
// waves per workgroup select the kernel.
hipError_t launch_decode_bf16(const DecodeArgs& a, int head_dim, int group, int waves, bool append,
                              hipStream_t stream);
hipError_t launch_decode_f32(const DecodeArgs& a, int head_dim, int group, int waves, bool append,
                             hipStream_t stream);

}  // namespace asrattn
