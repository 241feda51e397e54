// Launchers of the attention kernels; the C ABI (api.hip) validates the
// parameters before calling them.
#pragma once

#include <hip/hip_runtime.h>

#include "asrattn.h"
#include "fsmn.hpp"

namespace asrattn {

// Decoder step over `splits` workgroups per (sequence, kv head); for
// splits > 1 the workspace holds the partial outputs
// float[batch][heads_q][splits][head_dim] and (max, sum) pairs
// float[batch][heads_q][splits][2], merged by a second kernel.
// append: the fused prologue of asrattn_decode_append, or null; paged: the
// page table of asrattn_decode_paged, or null.
hipError_t launch_decode(const asrattn_decode_params& p, const asrattn_append_params* append,
                         const asrattn_paged_kv* paged, int splits, float* ws_o, float* ws_ml, hipStream_t stream);
// Waves per workgroup (page_size 0: not paged) and key rows one wave load
// covers.
int decode_waves(const asrattn_decode_params& p, int splits, int page_size);
int decode_keys_per_wave(int dtype, int head_dim);
bool decode_supported(int dtype, int head_dim, int group);

// Multi-row forward on matrix cores with K/V streamed into an LDS ring by
// DMA (bf16, head_dim 64 or 128, K/V spans addressable with 32-bit offsets).
// fsmn (or null): the FSMN memory computed in the same launch (kernel size
// at most kFsmnFusedKernel).
hipError_t launch_fwd_ring(const asrattn_fwd_params& p, const FsmnArgs* fsmn, hipStream_t stream);
bool fwd_ring_supported(const asrattn_fwd_params& p);

// Greedy choice per row of fp32 logits: argmax (first index on ties) and its
// log-probability; suppress (uint8 per vocabulary entry) may be null.
// Splits per row of the two-launch choice (1: one workgroup per row).
int choose_splits(int64_t rows, int64_t vocab);
// Workspace bytes of the split form (0 when one workgroup per row is used).
size_t choose_workspace_bytes(int64_t rows, int64_t vocab);
// workspace: at least choose_workspace_bytes, or null for one workgroup per row.
hipError_t launch_choose(const float* logits, int64_t rows, int64_t vocab, int64_t row_stride, const uint8_t* suppress,
                         int64_t* token, float* logprob, void* workspace, hipStream_t stream);

// Multi-row forward in fp32 on the matrix cores (head_dim 64 or 128, no
// sliding window, K/V spans addressable with 32-bit offsets).
hipError_t launch_fwd_f32mm(const asrattn_fwd_params& p, hipStream_t stream);
bool fwd_f32mm_supported(const asrattn_fwd_params& p);

// Multi-row forward on the vector ALUs (fp32 or bf16, head_dim 64 or 128):
// the fp32 path, the fallback for bf16 layouts the matrix-core kernel does
// not address, and the reference-precision check of that kernel.
hipError_t launch_fwd_valu(const asrattn_fwd_params& p, hipStream_t stream);
bool fwd_valu_supported(int dtype, int head_dim);

// Blocked local attention with relative position scores (asrattn_local),
// and the LDS it stages per workgroup.
hipError_t launch_local(const asrattn_local_params& p, hipStream_t stream);
size_t local_lds_bytes(const asrattn_local_params& p);

// SAN-M's FSMN memory on its own (fp32 or bf16, head_dim 64 or 128, kernel
// size at most kFsmnMaxKernel) for the padded layout of p (values p.v, frame
// counts p.seqused_k).
hipError_t launch_fsmn(const asrattn_fwd_params& p, const FsmnArgs& f, hipStream_t stream);

}  // namespace asrattn
