// Sequence geometry shared by the multi-row forward kernels.
#pragma once

#include "common.hpp"
#include "fsmn.hpp"

namespace asrattn {

struct FwdArgs {
  asrattn_fwd_params p;
  float c;  // scale * log2(e)
  FsmnArgs f;  // the fused FSMN memory (f.memory null: none)
};

// Resolved geometry of one (sequence, head): element offsets of its first
// query / key / value / output token and its lengths.
struct SeqView {
  int64_t q_off, k_off, v_off, o_off;
  int len_q, len_k, n_k;
};

__device__ __forceinline__ SeqView seq_view(const asrattn_fwd_params& p, int b, int hq, int hkv) {
  SeqView s;
  int64_t qtok = 0, ktok = 0;
  if (p.cu_seqlens_q != nullptr) {
    qtok = p.cu_seqlens_q[b];
    s.len_q = p.cu_seqlens_q[b + 1] - p.cu_seqlens_q[b];
    s.q_off = qtok * p.q_token_stride;
    s.o_off = qtok * p.o_token_stride;
  } else {
    s.len_q = p.max_len_q;
    s.q_off = (int64_t)b * p.q_batch_stride;
    s.o_off = (int64_t)b * p.o_batch_stride;
  }
  if (p.cu_seqlens_k != nullptr) {
    ktok = p.cu_seqlens_k[b];
    s.len_k = p.cu_seqlens_k[b + 1] - p.cu_seqlens_k[b];
    s.k_off = ktok * p.k_token_stride;
    s.v_off = ktok * p.v_token_stride;
  } else {
    s.len_k = p.max_len_k;
    s.k_off = (int64_t)b * p.k_batch_stride;
    s.v_off = (int64_t)b * p.v_batch_stride;
  }
  s.len_q = min(max(s.len_q, 0), p.max_len_q);
  s.len_k = min(max(s.len_k, 0), p.max_len_k);
  s.n_k = s.len_k;
  if (p.seqused_k != nullptr) s.n_k = min(s.n_k, max(p.seqused_k[b], 0));
  s.q_off += (int64_t)hq * p.q_head_stride;
  s.o_off += (int64_t)hq * p.o_head_stride;
  s.k_off += (int64_t)hkv * p.k_head_stride;
  s.v_off += (int64_t)hkv * p.v_head_stride;
  return s;
}

// Keys query row r of a sequence sees are j < visible_keys(r).
__device__ __forceinline__ int visible_keys(const asrattn_fwd_params& p, const SeqView& s, int r) {
  if (p.causal == ASRATTN_CAUSAL_NONE) return s.n_k;
  const int shift = p.causal == ASRATTN_CAUSAL_BOTTOM_RIGHT ? s.n_k - s.len_q : 0;
  return max(0, min(s.n_k, r + 1 + shift));
}

// The first key query row r of a sequence sees (window > 0, causal): keys
// first_key(r) <= j < visible_keys(r).
__device__ __forceinline__ int first_key(const asrattn_fwd_params& p, const SeqView& s, int r) {
  if (p.window <= 0 || p.causal == ASRATTN_CAUSAL_NONE) return 0;
  const int shift = p.causal == ASRATTN_CAUSAL_BOTTOM_RIGHT ? s.n_k - s.len_q : 0;
  return max(0, r + 1 + shift - p.window);
}

}  // namespace asrattn
