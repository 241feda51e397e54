/*
 * asrattn.h -- C ABI of the MI355X (gfx950) attention library behind the
 * asrback attention modules.
 *
 * The reference (sjjeong94/asrback) has no native code and no FFI: its
 * attention is reached through two PyTorch ops called from plain-PyTorch
 * modules.  Every entry point below replaces a group of those op calls; the
 * reference call sites are cited as path:line relative to the reference repo.
 *
 * Conventions
 *   - Tensors are passed as device pointers plus element strides (elements,
 *     not bytes).  The head_dim axis must have unit stride; every other axis
 *     may be strided (views of fused projections, cache slices, ...).
 *   - dtype is ASRATTN_F32 or ASRATTN_BF16 and applies to q, k, v and out.
 *     Arithmetic is always fp32 (bf16 operands, fp32 accumulation).
 *   - Per-sequence lengths live in device memory, so a call can be captured
 *     in a HIP graph and replayed while the lengths change.
 *   - stream is a hipStream_t (passed as void*); every launch goes there.
 *   - No entry point allocates device memory or synchronizes.  Scratch space
 *     comes from the caller (asrattn_decode's workspace), except for
 *     asrattn_decode_noalloc, which uses a static device array.
 *   - Every entry point returns ASRATTN_OK (0) or an error code; the message
 *     of the last error on the calling thread is asrattn_last_error().
 *     Nothing aborts the process.
 */
#ifndef ASRATTN_H
#define ASRATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ASRATTN_ABI_VERSION 11

enum asrattn_status {
  ASRATTN_OK = 0,
  ASRATTN_ERR_INVALID = 1,      /* bad argument (shape, stride, pointer) */
  ASRATTN_ERR_UNSUPPORTED = 2,  /* valid request the library has no kernel for */
  ASRATTN_ERR_HIP = 3,          /* the HIP runtime reported an error */
  ASRATTN_ERR_WORKSPACE = 4     /* workspace missing or too small */
};

enum asrattn_dtype { ASRATTN_F32 = 0, ASRATTN_BF16 = 1 };

/* asrattn_fwd_params.flags: run the vector-ALU kernel (fp32 arithmetic on
   the vector units) even where a matrix-core kernel applies -- the bf16 one,
   or the fp32 one at head_dim 64/128 -- as the exact-arithmetic twin, for
   checks. */
#define ASRATTN_FWD_FORCE_VALU 1
/* asrattn_fwd_params.flags: padded layout (cu_seqlens NULL), non-causal,
   seqused_k given: query rows t >= seqused_k[b] are not computed and get
   zeros.  Rows t < seqused_k[b] are unchanged.  For callers whose padded
   rows never reach a valid row (SenseVoice's encoder: every later op on a
   padded frame is row-local or masked, sensevoice.py:97-107, :115-125). */
#define ASRATTN_FWD_ZERO_PADDED_ROWS 2

enum asrattn_causal {
  ASRATTN_CAUSAL_NONE = 0,
  /* query i sees keys j <= i (torch SDPA is_causal=True, top-left aligned) */
  ASRATTN_CAUSAL_TOP_LEFT = 1,
  /* query i sees keys j <= i + (keys - queries) (flash varlen
     window_size=(-1, 0), bottom-right aligned) */
  ASRATTN_CAUSAL_BOTTOM_RIGHT = 2
};

/*
 * Multi-query-row attention: encoder self-attention, causal prompt prefill,
 * packed variable-length sequences, grouped-query attention.
 *
 *   out[b, i, h, :] = softmax_j(scale * q[b, i, h, :] . k[b, j, h / g, :]) v[b, j, h / g, :]
 *   with g = heads_q / heads_kv and j over the keys sequence b uses.
 *
 * Sequence layout: with cu_seqlens_q == NULL, sequence b's query token t is
 * at q + b * q_batch_stride + t * q_token_stride and every sequence has
 * max_len_q queries (likewise keys with cu_seqlens_k / max_len_k).  With
 * cu_seqlens_q != NULL (int32[batch + 1], device) sequences are packed: token
 * t of sequence b is at q + (cu_seqlens_q[b] + t) * q_token_stride, the batch
 * stride is ignored and the sequence has cu_seqlens_q[b+1] - cu_seqlens_q[b]
 * queries (at most max_len_q).  seqused_k (int32[batch], device, optional)
 * caps the keys sequence b uses.  A query with no visible key gets zeros.
 * head_dim 64, 128, 256 or 512 (256 and 512: Gemma 4's sliding and full
 * layers, gemma4.py:552-559, scale 1.0).
 *
 * Replaces:
 *   F.scaled_dot_product_attention   src/asrback/models/whisper.py:102-104
 *       (encoder self-attention, whisper.py:108-110 via :124; causal prompt
 *       prefix, whisper.py:235-237 with length set)
 *   varlen_attn(..., seqused_k)      src/asrback/models/sensevoice.py:115-125
 *   F.scaled_dot_product_attention   src/asrback/models/sensevoice.py:128-133
 *   varlen_attn(..., window_size, enable_gqa)
 *                                    src/asrback/models/qwen3_asr.py:156-166
 *   F.scaled_dot_product_attention(..., enable_gqa=True)
 *                                    src/asrback/models/qwen3_asr.py:176-180
 */
typedef struct asrattn_fwd_params {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  int64_t q_batch_stride, q_token_stride, q_head_stride;
  int64_t k_batch_stride, k_token_stride, k_head_stride;
  int64_t v_batch_stride, v_token_stride, v_head_stride;
  int64_t o_batch_stride, o_token_stride, o_head_stride;
  const int32_t* cu_seqlens_q; /* int32[batch + 1] or NULL */
  const int32_t* cu_seqlens_k; /* int32[batch + 1] or NULL */
  const int32_t* seqused_k;    /* int32[batch] or NULL */
  int32_t batch;
  int32_t heads_q;
  int32_t heads_kv; /* divides heads_q */
  int32_t head_dim;
  int32_t max_len_q;
  int32_t max_len_k;
  int32_t causal; /* enum asrattn_causal */
  int32_t dtype;  /* enum asrattn_dtype */
  float scale;    /* softmax scale; torch's default is 1 / sqrt(head_dim) */
  int32_t flags;  /* 0 or a combination of ASRATTN_FWD_* flags */
  int32_t window; /* > 0 (causal only): query i also sees no key more than
                     window - 1 before its last visible one (sliding-window
                     attention, gemma4.py:1231-1234); 0: none */
} asrattn_fwd_params;

int asrattn_fwd(const asrattn_fwd_params* params, void* stream);

/*
 * SAN-M self-attention with its FSMN memory, in one launch where the
 * matrix-core kernel applies (bf16, kernel_size <= 11): asrattn_fwd on the
 * padded, non-causal layout (cu_seqlens NULL, heads_q == heads_kv,
 * max_len_q == max_len_k; seqused_k, the frame counts n_b, or NULL for all
 * frames) and, over the values v of the same call,
 *
 *   memory[b, t, c] = keep(t) * (conv + v'[b, t, c]) + bias[c]     (t < max_len_q)
 *   conv            = sum_{i < K} weight[c, i] * v'[b, t + i - (K - 1) / 2, c]
 *   v'[b, s, c]     = v[b, s, h, d] if 0 <= s < n_b else 0,  keep(t) = t < n_b
 *
 * with channel c = h * head_dim + d.  Rounded in the element type as the
 * reference's ops round: the convolution (fp32 sums), then the sum with v',
 * then the sum with the bias.  bias (or NULL) lets the caller fold the
 * output projection's bias in: linear_out(out) + memory becomes one GEMM
 * that accumulates into memory.  memory must not overlap q, k, v or out.
 *
 * Replaces (the reference's mask multiply, pad, depthwise Conv1d, add, mask
 * multiply and the final add):
 *   sensevoice.py:99-107 (FSMN memory) and :135 (linear_out(...) + memory)
 *                                    src/asrback/models/sensevoice.py
 * together with the attention call of asrattn_fwd (sensevoice.py:110-133).
 */
typedef struct asrattn_fsmn_params {
  const void* weight; /* (heads_q * head_dim, kernel_size): Conv1d weight (C, 1, K), contiguous */
  const void* bias;   /* (heads_q * head_dim) added to every row, or NULL */
  void* memory;       /* (batch, max_len_q, heads_q * head_dim), unit channel stride */
  int64_t m_batch_stride, m_token_stride;
  int32_t kernel_size; /* 1 .. 15 */
} asrattn_fsmn_params;

int asrattn_fwd_fsmn(const asrattn_fwd_params* params, const asrattn_fsmn_params* fsmn, void* stream);

/*
 * One query per sequence over a key/value cache (decoder step).  A
 * workgroup streams the keys of one (sequence, kv head); when the batch has
 * too few of those to fill the GPU, the keys are split over several
 * workgroups (split-K) and a second kernel merges their partials.
 *
 *   out[b, h, :] = softmax_j(scale * q[b, h, :] . k[b, j, h / g, :]) v[b, j, h / g, :]
 *   for n_b - window <= j < n_b (window > 0) or j < n_b (window == 0),
 *                 n_b = min(max_len_k, seqused_k[b])      (seqused_k given)
 *                 n_b = min(max_len_k, positions[b] + 1)  (positions given)
 *                 n_b = max_len_k                         (neither)
 *
 * k/v token t of sequence b, head h is at k + b*k_batch_stride +
 * t*k_token_stride + h*k_head_stride: both cache layouts of the reference
 * are plain strides, (batch, heads, length, head_dim) for Whisper and
 * (batch, 1024, kv_heads, head_dim) for Qwen3-ASR.  Tokens 0 .. max_len_k - 1
 * of every sequence must be readable memory: the first load batch may be
 * issued before n_b is read and may touch tokens at or past n_b, which are
 * then discarded whatever they hold (NaN and infinities included).
 *
 * workspace: device memory of asrattn_decode_workspace_size(params) bytes
 * (0 when a single split is used), 256-byte aligned, owned by the caller;
 * it holds the split partials, needs no initialization, must stay valid
 * until the launch completes and must not be shared by concurrent calls.
 *
 * Replaces:
 *   F.scaled_dot_product_attention with the (batch, 1, 1, length) position
 *       mask                         src/asrback/models/whisper.py:235-237
 *       (mask built at whisper.py:263-264)
 *   F.scaled_dot_product_attention over the cross-attention cache
 *                                    src/asrback/models/whisper.py:239-240
 *   varlen_attn(..., seqused_k=positions + 1, num_splits, enable_gqa)
 *                                    src/asrback/models/qwen3_asr.py:414-425
 *   F.scaled_dot_product_attention with queries grouped per kv head
 *                                    src/asrback/models/qwen3_asr.py:427-431
 */
typedef struct asrattn_decode_params {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  int64_t q_batch_stride, q_head_stride;
  int64_t k_batch_stride, k_token_stride, k_head_stride;
  int64_t v_batch_stride, v_token_stride, v_head_stride;
  int64_t o_batch_stride, o_head_stride;
  const int32_t* seqused_k; /* int32[batch] or NULL */
  const int64_t* positions; /* int64[batch] or NULL (ignored if seqused_k) */
  int32_t batch;
  int32_t heads_q;
  int32_t heads_kv;
  int32_t head_dim;
  int32_t max_len_k;
  int32_t num_splits; /* 0: chosen from batch, heads and max_len_k */
  int32_t dtype;
  float scale;
  int32_t window; /* > 0: each query sees only its last `window` keys (sliding-window
                     attention, gemma4.py:720-725); 0: all n_b */
} asrattn_decode_params;

/* Bytes of workspace asrattn_decode needs for these parameters (pointers are
 * not read).  Returns 0 for a single split, or (size_t)-1 on invalid params. */
size_t asrattn_decode_workspace_size(const asrattn_decode_params* params);

/* The split count asrattn_decode uses for these parameters. */
int asrattn_decode_num_splits(const asrattn_decode_params* params);

int asrattn_decode(const asrattn_decode_params* params, void* workspace,
                   size_t workspace_bytes, void* stream);

/*
 * asrattn_decode without a workspace argument and without any allocation,
 * for callers that cannot allocate device memory: code under HIP graph
 * capture, tight serving loops, and harnesses that forbid hipMalloc.  It has
 * no counterpart in the reference.
 *
 * The split partials go to a static device array of
 * ASRATTN_DECODE_NOALLOC_MAX_BYTES bytes that the library holds on each GPU
 * it runs on until the process ends.  That size covers every split count
 * the library chooses itself (num_splits = 0; at most 6 MiB, head_dim 512
 * with 8 query heads per kv head); parameters whose partials need more
 * (asrattn_decode_workspace_size) are rejected with ASRATTN_ERR_WORKSPACE.
 * The array needs no clearing: every launch writes all of the partials it
 * reads.  All calls on one GPU share its array, so calls that may overlap on
 * one GPU (different streams, or different host threads) race; serialize
 * them, or use asrattn_decode with a workspace each.  The stream must belong
 * to the current device.  Results are identical to asrattn_decode's.
 */
#define ASRATTN_DECODE_NOALLOC_MAX_BYTES ((size_t)8 << 20)
int asrattn_decode_noalloc(const asrattn_decode_params* params, void* stream);

/*
 * The decoder step with its prologue fused in: the step's own key and value
 * (one token per sequence) are appended to the cache, and q and the new key
 * get the per-head RMSNorm and rotary embedding the reference applies
 * before attention.  With positions[b] = p (required; seqused_k must be
 * NULL):
 *
 *   q'  = rot(norm(q[b, h, :], q_norm), cos[b], sin[b])
 *   k'  = rot(norm(k_new[b, h', :], k_norm), cos[b], sin[b])
 *   v'  = norm(v_new[b, h', :], 1)                 (v_norm != 0; else v_new)
 *   k[b, p, h', :] = k',  v[b, p, h', :] = v'      (if p < max_len_k)
 *   out[b, h, :] = attention of q' over cache keys j < min(p, max_len_k)
 *                  and the new key/value
 *
 *   norm(x, w)[i] = x[i] / sqrt(mean(x^2) + eps) * w[i]       (w NULL: none)
 *   rot(x, c, s)[i] = x[i] c[i] + r[i] s[i],  r = (-x[d/2:], x[:d/2])
 *                                                        (cos NULL: none)
 *
 * in the cache's dtype, rounded as the reference's float32-accumulated
 * norm and element-wise rotation round.  p_params->q is the raw q
 * (batch, heads_q, head_dim); k/v are the cache.  Workspace as for
 * asrattn_decode (the same size function applies).
 *
 * Replaces (the step path of):
 *   q_norm/k_norm + rotate in TextAttention._project
 *                                    src/asrback/models/qwen3_asr.py:366-372
 *   keys[rows, positions] = k; values[rows, positions] = v, then the
 *       attention                    src/asrback/models/qwen3_asr.py:409-432
 *   keys.scatter_/values.scatter_ of the Whisper step (no norm, no
 *       rotation)                    src/asrback/models/whisper.py:224-228
 *   q_norm/k_norm/v_norm + rotate and the cache writes of Gemma 4's step
 *                                    src/asrback/models/gemma4.py:522-532,
 *                                    :563-587
 */
typedef struct asrattn_append_params {
  const void* k_new; /* (batch, heads_kv, head_dim), before norm and rotation */
  const void* v_new; /* (batch, heads_kv, head_dim) */
  int64_t kn_batch_stride, kn_head_stride;
  int64_t vn_batch_stride, vn_head_stride;
  const void* q_norm; /* (head_dim,) RMSNorm weights, or NULL: no norm */
  const void* k_norm; /* (head_dim,), NULL exactly when q_norm is */
  float eps;
  const void* cos; /* (batch, head_dim) tables at each row's position, or NULL */
  const void* sin; /* NULL exactly when cos is */
  int64_t rope_batch_stride;
  int32_t v_norm; /* nonzero: RMS-normalize the new value, without weights
                     (Gemma 4's v_norm, gemma4.py:515) */
} asrattn_append_params;

int asrattn_decode_append(const asrattn_decode_params* params, const asrattn_append_params* append,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * The decoder step over a paged key/value cache: keys live in pages of
 * page_size tokens taken from one pool, so each sequence holds only the
 * pages its keys need instead of a fixed max_len_k-slot slab.  Logical page
 * i of sequence b (its keys i * page_size .. (i + 1) * page_size - 1) is pool
 * page block_table[b * bt_stride + i]:
 *
 *   key j of sequence b, kv head h at
 *     k + page * k_page_stride + (j % page_size) * k_token_stride + h * k_head_stride,
 *     page = block_table[b * bt_stride + j / page_size]
 *
 * (likewise v); p_params->k/v point at the pool and k/v_batch_stride are
 * ignored.  Everything else is asrattn_decode (append == NULL) or
 * asrattn_decode_append (the new key and value are written to the page of
 * positions[b]); the workspace size is asrattn_decode_workspace_size's.
 * max_len_k bounds the keys a sequence may use (<= bt_stride * page_size).
 * Only entry 0 and the entries of pages holding a sequence's keys are read;
 * an entry outside [0, num_pages) is not dereferenced and its keys are
 * skipped.  The first page's tokens may be read past n_b (the first load
 * batch can be issued before n_b is read) and are then discarded.
 *
 * Replaces (generalizes): the flattened (B * 1024, kv_heads, head_dim) slab
 * with cu_seqlens_k = row * 1024 of the reference's varlen decode
 *                                    src/asrback/models/qwen3_asr.py:511-512
 * whose fixed 1024 slots per row (CACHE_LENGTH, qwen3_asr.py:57-59,
 * allocated at :817-827) bound the batch size.
 */
typedef struct asrattn_paged_kv {
  const int32_t* block_table; /* int32, sequence b's entries at block_table + b * bt_stride */
  int64_t bt_stride;          /* entries per sequence */
  int32_t page_size;          /* tokens per page: a power of two >= 16 (>= 32 for bf16 at head_dim 64) */
  int32_t num_pages;          /* pages in the pool */
  int64_t k_page_stride, v_page_stride; /* elements between consecutive pool pages */
} asrattn_paged_kv;

int asrattn_decode_paged(const asrattn_decode_params* params, const asrattn_append_params* append,
                         const asrattn_paged_kv* paged, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Greedy next token per row of float32 logits:
 *
 *   token[r]   = argmax_j x[r, j]       (first index among equal maxima)
 *   logprob[r] = log_softmax(x[r])[token[r]] = -log(sum_j exp(x[r, j] - max))
 *
 * with x[r, j] = -inf where suppress[j] != 0 (suppress: uint8[vocab], or
 * NULL).  NaN counts as the largest value and makes the row's logprob NaN;
 * a row of -inf gives token 0 and a NaN logprob (torch.argmax and
 * log_softmax behave the same).  logits row r starts at logits +
 * r*row_stride (row_stride >= vocab); token is int64[rows], logprob
 * float32[rows].  1 <= vocab < 2^29.
 *
 * With a workspace of asrattn_choose_workspace_size(rows, vocab) bytes
 * (caller-owned device memory, a fixed address for graphs; 0 means none is
 * needed) each row is read by several workgroups and a second launch folds
 * their partial maxima and sums; without one (NULL, 0) one workgroup per
 * row reads it in a single launch.  A workspace smaller than the size
 * returns ASRATTN_ERR_WORKSPACE.  Results are the same either way.
 *
 * Replaces the greedy path of:
 *   logits.masked_fill_(suppress, -inf); argmax; log_softmax; gather
 *                                    src/asrback/models/whisper.py:962-974
 *   argmax; log_softmax; gather      src/asrback/models/qwen3_asr.py:1200-1210
 */
int asrattn_choose(const float* logits, int64_t rows, int64_t vocab, int64_t row_stride, const uint8_t* suppress,
                   int64_t* token, float* logprob, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes asrattn_choose uses to split rows (0: it does not). */
size_t asrattn_choose_workspace_size(int64_t rows, int64_t vocab);

/*
 * Blocked local attention with relative position scores, in float32 (Gemma 4's
 * audio encoder).  Queries form blocks of `chunk` tokens; block u's context
 * slots t = 0 .. chunk + past + future - 1 hold keys u * chunk - past + t.
 * For query i = u * chunk + c of sequence b, head h:
 *
 *   s[t]   = q_i . k_key + (0 <= t - c < rel_positions ? q_i . rel[t - c] : 0)
 *   s[t]   = tanh(s[t] / softcap) * softcap
 *   s[t]   = invalid  unless  (0 <= i - key < past  or  0 < key - i < future)
 *                     and 0 <= key < lengths[b]
 *   out[b, i, h, :] = sum_t softmax(s)[t] v_key        (keys outside 0 ..
 *                     tokens - 1 are zeros)
 *
 * q, k, v, out: (batch, tokens, heads, head_dim) with element strides;
 * rel: (rel_positions, heads, head_dim), relative keys of distances
 * past .. 0 (row r: distance past - r; the reference's sinusoids through
 * relative_k_proj); lengths: int32[batch], device.  The module scales q and
 * k before the call, as the reference does.  Requires rel_positions <= past
 * + future + 2 (the reference's relative shift then never wraps into the
 * previous row) and a block's staged data within 64 KB of LDS.
 *
 * Replaces (the attention of AudioAttention.forward):
 *   context gathering, content and relative scores, the relative shift,
 *   the soft cap, the mask and the softmax
 *                                    src/asrback/models/gemma4.py:240-282
 */
typedef struct asrattn_local_params {
  const float* q;
  const float* k;
  const float* v;
  const float* rel;
  float* out;
  int64_t q_batch_stride, q_token_stride, q_head_stride;
  int64_t k_batch_stride, k_token_stride, k_head_stride;
  int64_t v_batch_stride, v_token_stride, v_head_stride;
  int64_t o_batch_stride, o_token_stride, o_head_stride;
  int64_t rel_position_stride, rel_head_stride;
  const int32_t* lengths;
  int32_t batch, tokens, heads, head_dim;
  int32_t chunk, past, future, rel_positions;
  float softcap;
  float invalid; /* the score of slots a query may not see (the reference's
                    attention_invalid_logits_value) */
} asrattn_local_params;

int asrattn_local(const asrattn_local_params* params, void* stream);

/* Message of the last failed call on this thread ("" if none). */
const char* asrattn_last_error(void);

/* ASRATTN_ABI_VERSION of the built library. */
int asrattn_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* ASRATTN_H */
