// C ABI of the attention library: argument checks, kernel choice, launch and
// error reporting.  Nothing here allocates device memory or synchronizes, so
// every entry point can run inside HIP graph capture.
#include <stdarg.h>
#include <stdio.h>

#include <cmath>
#include <mutex>
#include <string>

#include "asrattn.h"
#include "kernels.hpp"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return ASRATTN_OK;
}

int elem_bytes(int dtype) { return dtype == ASRATTN_BF16 ? 2 : 4; }

// 16-byte vector access needs 16-byte aligned rows: pointer aligned and every
// stride a multiple of one vector.
bool vec_aligned(const void* ptr, int dtype, std::initializer_list<int64_t> strides) {
  if ((reinterpret_cast<uintptr_t>(ptr) & 15u) != 0) return false;
  const int64_t per_vec = 16 / elem_bytes(dtype);
  for (int64_t s : strides)
    if (s % per_vec != 0) return false;
  return true;
}

int check_common(int dtype, int heads_q, int heads_kv, int head_dim, float scale) {
  if (dtype != ASRATTN_F32 && dtype != ASRATTN_BF16)
    return fail(ASRATTN_ERR_INVALID, "dtype %d is neither ASRATTN_F32 nor ASRATTN_BF16", dtype);
  if (heads_q <= 0 || heads_kv <= 0 || heads_q % heads_kv != 0)
    return fail(ASRATTN_ERR_INVALID, "heads_q (%d) must be a positive multiple of heads_kv (%d)", heads_q,
                heads_kv);
  if (head_dim <= 0) return fail(ASRATTN_ERR_INVALID, "head_dim must be positive, got %d", head_dim);
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(ASRATTN_ERR_INVALID, "scale must be positive and finite, got %g", (double)scale);
  return ASRATTN_OK;
}

int from_hip(hipError_t err, const char* what) {
  if (err == hipSuccess) return ok();
  return fail(ASRATTN_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
}

int decode_splits(const asrattn_decode_params& p) {
  if (p.num_splits > 0) return p.num_splits;
  // One workgroup per (sequence, kv head) once there are enough of them to
  // spread over the 256 CUs (192 and more: Whisper-small's 16 x 12, Qwen3's
  // 64 x 8); fewer get their keys split, at least 256 keys per split (128
  // pairs, Gemma 4's 32 rows x 4 kv heads: two splits measured 7% faster
  // than one).
  const long long pairs = (long long)p.batch * p.heads_kv;
  if (pairs >= 192) return 1;
  long long s = (256 + pairs - 1) / pairs;
  const long long by_len = (p.max_len_k + 255) / 256;
  if (s > by_len) s = by_len;
  if (s > 64) s = 64;
  if (s < 1) s = 1;
  return (int)s;
}

int check_decode(const asrattn_decode_params* p) {
  if (p == nullptr) return fail(ASRATTN_ERR_INVALID, "params is NULL");
  int rc = check_common(p->dtype, p->heads_q, p->heads_kv, p->head_dim, p->scale);
  if (rc != ASRATTN_OK) return rc;
  if (p->batch < 0) return fail(ASRATTN_ERR_INVALID, "batch must be >= 0, got %d", p->batch);
  if (p->max_len_k < 0) return fail(ASRATTN_ERR_INVALID, "max_len_k must be >= 0, got %d", p->max_len_k);
  if (p->window < 0) return fail(ASRATTN_ERR_INVALID, "window must be >= 0, got %d", p->window);
  if (p->num_splits < 0 || p->num_splits > 1024)
    return fail(ASRATTN_ERR_INVALID, "num_splits must be in [0, 1024], got %d", p->num_splits);
  const int group = p->heads_q / p->heads_kv;
  if (!asrattn::decode_supported(p->dtype, p->head_dim, group))
    return fail(ASRATTN_ERR_UNSUPPORTED,
                "no decode kernel for head_dim %d with %d query heads per kv head (supported: head_dim "
                "64/128/256, and 512 in bf16; 1/2/4/8 heads per kv head)",
                p->head_dim, group);
  return ASRATTN_OK;
}

// Workspace layout: partial outputs, then (max, sum) pairs, each section
// 256-byte aligned.
struct DecodeWorkspace {
  size_t partials, stats, total;
};

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

DecodeWorkspace decode_workspace(const asrattn_decode_params& p, int splits) {
  DecodeWorkspace w{0, 0, 0};
  if (splits == 1) return w;
  const size_t rows = (size_t)p.batch * p.heads_q * splits;
  w.partials = 0;
  w.stats = align256(rows * (size_t)p.head_dim * sizeof(float));
  w.total = w.stats + align256(rows * 2 * sizeof(float));
  return w;
}

}  // namespace

extern "C" {

size_t asrattn_decode_workspace_size(const asrattn_decode_params* params) {
  if (check_decode(params) != ASRATTN_OK) return (size_t)-1;
  return decode_workspace(*params, decode_splits(*params)).total;
}

const char* asrattn_last_error(void) { return g_last_error.c_str(); }

int asrattn_abi_version(void) { return ASRATTN_ABI_VERSION; }

}  // extern "C"

namespace {

// Argument checks of asrattn_fwd; *empty is set when there is nothing to do.
int check_fwd(const asrattn_fwd_params* params, bool* empty) {
  if (params == nullptr) return fail(ASRATTN_ERR_INVALID, "params is NULL");
  const asrattn_fwd_params& p = *params;
  int rc = check_common(p.dtype, p.heads_q, p.heads_kv, p.head_dim, p.scale);
  if (rc != ASRATTN_OK) return rc;
  if (p.batch < 0 || p.max_len_q < 0 || p.max_len_k < 0)
    return fail(ASRATTN_ERR_INVALID, "batch (%d), max_len_q (%d) and max_len_k (%d) must be >= 0", p.batch,
                p.max_len_q, p.max_len_k);
  if (p.causal < ASRATTN_CAUSAL_NONE || p.causal > ASRATTN_CAUSAL_BOTTOM_RIGHT)
    return fail(ASRATTN_ERR_INVALID, "causal must be 0, 1 or 2, got %d", p.causal);
  if ((p.cu_seqlens_q == nullptr) != (p.cu_seqlens_k == nullptr))
    return fail(ASRATTN_ERR_INVALID, "cu_seqlens_q and cu_seqlens_k must both be set or both be NULL");
  if (p.window < 0 || (p.window > 0 && p.causal == ASRATTN_CAUSAL_NONE))
    return fail(ASRATTN_ERR_INVALID, "window must be >= 0, and > 0 only with causal attention (got %d)", p.window);
  if ((p.flags & ASRATTN_FWD_ZERO_PADDED_ROWS) != 0 &&
      (p.cu_seqlens_q != nullptr || p.causal != ASRATTN_CAUSAL_NONE || p.seqused_k == nullptr))
    return fail(ASRATTN_ERR_INVALID,
                "ASRATTN_FWD_ZERO_PADDED_ROWS needs the padded, non-causal layout with seqused_k");
  *empty = p.batch == 0 || p.max_len_q == 0;
  if (*empty) return ASRATTN_OK;
  if (p.q == nullptr || p.k == nullptr || p.v == nullptr || p.out == nullptr)
    return fail(ASRATTN_ERR_INVALID, "q, k, v and out must be non-NULL");
  if (!vec_aligned(p.q, p.dtype, {p.q_batch_stride, p.q_token_stride, p.q_head_stride}) ||
      !vec_aligned(p.k, p.dtype, {p.k_batch_stride, p.k_token_stride, p.k_head_stride}) ||
      !vec_aligned(p.v, p.dtype, {p.v_batch_stride, p.v_token_stride, p.v_head_stride}) ||
      !vec_aligned(p.out, p.dtype, {p.o_batch_stride, p.o_token_stride, p.o_head_stride}))
    return fail(ASRATTN_ERR_INVALID,
                "q, k, v and out need 16-byte aligned pointers and strides that are multiples of 16 bytes");
  const bool generic = (p.flags & ASRATTN_FWD_FORCE_VALU) != 0;
  if ((generic || !asrattn::fwd_ring_supported(p)) && !asrattn::fwd_valu_supported(p.dtype, p.head_dim))
    return fail(ASRATTN_ERR_UNSUPPORTED, "no forward kernel for head_dim %d (supported: 64, 128, 256, 512)",
                p.head_dim);
  return ASRATTN_OK;
}

// The attention launch of asrattn_fwd / asrattn_fwd_fsmn; fsmn (or null) is
// fused into the matrix-core kernel, else launched after the attention.
int run_fwd(const asrattn_fwd_params& p, const asrattn::FsmnArgs* fsmn, void* stream, const char* name) {
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool generic = (p.flags & ASRATTN_FWD_FORCE_VALU) != 0;
  hipError_t err;
  if (!generic && asrattn::fwd_ring_supported(p)) {
    const bool fused = fsmn != nullptr && fsmn->kernel_size <= asrattn::kFsmnFusedKernel;
    err = asrattn::launch_fwd_ring(p, fused ? fsmn : nullptr, s);
    if (fused || fsmn == nullptr || err != hipSuccess) return from_hip(err, name);
  } else if (!generic && asrattn::fwd_f32mm_supported(p)) {
    err = asrattn::launch_fwd_f32mm(p, s);
    if (fsmn == nullptr || err != hipSuccess) return from_hip(err, name);
  } else {
    err = asrattn::launch_fwd_valu(p, s);
    if (fsmn == nullptr || err != hipSuccess) return from_hip(err, name);
  }
  return from_hip(asrattn::launch_fsmn(p, *fsmn, s), name);
}

}  // namespace

extern "C" {

int asrattn_fwd(const asrattn_fwd_params* params, void* stream) {
  bool empty = false;
  const int rc = check_fwd(params, &empty);
  if (rc != ASRATTN_OK) return rc;
  if (empty) return ok();
  return run_fwd(*params, nullptr, stream, "asrattn_fwd");
}

int asrattn_fwd_fsmn(const asrattn_fwd_params* params, const asrattn_fsmn_params* fsmn, void* stream) {
  if (fsmn == nullptr) return fail(ASRATTN_ERR_INVALID, "fsmn parameters must be non-NULL");
  bool empty = false;
  const int rc = check_fwd(params, &empty);
  if (rc != ASRATTN_OK) return rc;
  const asrattn_fwd_params& p = *params;
  const asrattn_fsmn_params& f = *fsmn;
  if (p.causal != ASRATTN_CAUSAL_NONE || p.cu_seqlens_q != nullptr || p.heads_q != p.heads_kv ||
      p.max_len_q != p.max_len_k)
    return fail(ASRATTN_ERR_INVALID,
                "the FSMN memory needs the padded, non-causal layout with max_len_q == max_len_k and heads_q == "
                "heads_kv");
  if (f.kernel_size < 1 || f.kernel_size > asrattn::kFsmnMaxKernel)
    return fail(ASRATTN_ERR_UNSUPPORTED, "FSMN kernel_size must be in [1, %d], got %d", asrattn::kFsmnMaxKernel,
                f.kernel_size);
  if (p.head_dim != 64 && p.head_dim != 128)
    return fail(ASRATTN_ERR_UNSUPPORTED, "FSMN memory for head_dim %d (supported: 64, 128)", p.head_dim);
  if (empty) return ok();
  if (f.weight == nullptr || f.memory == nullptr)
    return fail(ASRATTN_ERR_INVALID, "the FSMN weight and memory must be non-NULL");
  if (!vec_aligned(f.memory, p.dtype, {f.m_batch_stride, f.m_token_stride}))
    return fail(ASRATTN_ERR_INVALID, "memory needs a 16-byte aligned pointer and strides that are multiples of 16 bytes");
  const size_t es = (size_t)elem_bytes(p.dtype);
  if ((reinterpret_cast<uintptr_t>(f.weight) % es) != 0 ||
      (f.bias != nullptr && (reinterpret_cast<uintptr_t>(f.bias) % es) != 0))
    return fail(ASRATTN_ERR_INVALID, "weight and bias must be aligned to their element size");
  // Value and memory rows are addressed with 32-bit byte offsets, up to a
  // block of rows past the end.
  if (((long long)p.max_len_k + 160) * p.v_token_stride * (long long)es >= (1LL << 31) ||
      ((long long)p.max_len_q + 160) * f.m_token_stride * (long long)es >= (1LL << 31))
    return fail(ASRATTN_ERR_UNSUPPORTED, "one sequence's values or memory span 2 GiB or more");
  const asrattn::FsmnArgs a{f.weight, f.bias, f.memory, f.m_batch_stride, f.m_token_stride, f.kernel_size};
  return run_fwd(p, &a, stream, "asrattn_fwd_fsmn");
}

int asrattn_decode_num_splits(const asrattn_decode_params* params) {
  if (check_decode(params) != ASRATTN_OK) return -1;
  return decode_splits(*params);
}



namespace {

int run_decode(const asrattn_decode_params* params, const asrattn_append_params* append,
               const asrattn_paged_kv* paged, void* workspace, size_t workspace_bytes, void* stream,
               const char* name) {
  int rc = check_decode(params);
  if (rc != ASRATTN_OK) return rc;
  const asrattn_decode_params& p = *params;
  if (p.batch == 0) return ok();
  if (p.q == nullptr || p.k == nullptr || p.v == nullptr || p.out == nullptr)
    return fail(ASRATTN_ERR_INVALID, "q, k, v and out must be non-NULL");
  if (!vec_aligned(p.q, p.dtype, {p.q_batch_stride, p.q_head_stride}) ||
      !vec_aligned(p.k, p.dtype, {p.k_batch_stride, p.k_token_stride, p.k_head_stride}) ||
      !vec_aligned(p.v, p.dtype, {p.v_batch_stride, p.v_token_stride, p.v_head_stride}))
    return fail(ASRATTN_ERR_INVALID,
                "q, k and v need 16-byte aligned pointers and strides that are multiples of 16 bytes");
  if (append != nullptr) {
    const asrattn_append_params& ap = *append;
    if (p.positions == nullptr || p.seqused_k != nullptr)
      return fail(ASRATTN_ERR_INVALID, "the appending step takes positions and no seqused_k");
    if (ap.k_new == nullptr || ap.v_new == nullptr)
      return fail(ASRATTN_ERR_INVALID, "k_new and v_new must be non-NULL");
    if ((ap.q_norm == nullptr) != (ap.k_norm == nullptr) || (ap.cos == nullptr) != (ap.sin == nullptr))
      return fail(ASRATTN_ERR_INVALID, "q_norm/k_norm and cos/sin come in pairs");
    if (!(ap.eps >= 0.f && ap.eps < 1e30f)) return fail(ASRATTN_ERR_INVALID, "eps must be finite and >= 0");
    if (!vec_aligned(ap.k_new, p.dtype, {ap.kn_batch_stride, ap.kn_head_stride}) ||
        !vec_aligned(ap.v_new, p.dtype, {ap.vn_batch_stride, ap.vn_head_stride}) ||
        (ap.q_norm != nullptr && (!vec_aligned(ap.q_norm, p.dtype, {}) || !vec_aligned(ap.k_norm, p.dtype, {}))) ||
        (ap.cos != nullptr &&
         (!vec_aligned(ap.cos, p.dtype, {ap.rope_batch_stride}) || !vec_aligned(ap.sin, p.dtype, {ap.rope_batch_stride}))))
      return fail(ASRATTN_ERR_INVALID,
                  "k_new, v_new, the norm weights and cos/sin need 16-byte aligned pointers and strides");
  }
  const long long es = p.dtype == ASRATTN_BF16 ? 2 : 4;
  if (paged != nullptr) {
    const asrattn_paged_kv& pk = *paged;
    const int min_page = 4 * asrattn::decode_keys_per_wave(p.dtype, p.head_dim);
    if (pk.block_table == nullptr) return fail(ASRATTN_ERR_INVALID, "block_table must be non-NULL");
    if (pk.page_size < 16 || (pk.page_size & (pk.page_size - 1)) != 0 || pk.page_size < min_page)
      return fail(ASRATTN_ERR_UNSUPPORTED, "page_size must be a power of two >= %d for this dtype and head_dim, got %d",
                  min_page < 16 ? 16 : min_page, pk.page_size);
    if (pk.num_pages < 0 || pk.bt_stride < 1)
      return fail(ASRATTN_ERR_INVALID, "num_pages must be >= 0 and bt_stride >= 1");
    if ((long long)p.max_len_k > pk.bt_stride * (long long)pk.page_size)
      return fail(ASRATTN_ERR_INVALID, "max_len_k (%d) exceeds the block table's reach (%lld pages of %d)", p.max_len_k,
                  (long long)pk.bt_stride, pk.page_size);
    if (!vec_aligned(p.k, p.dtype, {pk.k_page_stride}) || !vec_aligned(p.v, p.dtype, {pk.v_page_stride}))
      return fail(ASRATTN_ERR_INVALID, "page strides must be multiples of 16 bytes");
    // Keys are addressed with 32-bit byte offsets from their page's start.
    if ((long long)pk.page_size * p.k_token_stride * es >= (1LL << 31) ||
        (long long)pk.page_size * p.v_token_stride * es >= (1LL << 31))
      return fail(ASRATTN_ERR_UNSUPPORTED, "one page spans 2 GiB or more");
  } else if ((long long)p.max_len_k * p.k_token_stride * es >= (1LL << 31) ||
             (long long)p.max_len_k * p.v_token_stride * es >= (1LL << 31)) {
    // Keys are addressed with 32-bit byte offsets from the sequence's start.
    return fail(ASRATTN_ERR_UNSUPPORTED, "one sequence's keys span 2 GiB or more");
  }
  const int s = decode_splits(p);
  const DecodeWorkspace w = decode_workspace(p, s);
  float* ws_o = nullptr;
  float* ws_ml = nullptr;
  if (s > 1) {
    if (workspace == nullptr || workspace_bytes < w.total)
      return fail(ASRATTN_ERR_WORKSPACE, "decode needs %zu workspace bytes, got %zu", w.total,
                  workspace == nullptr ? (size_t)0 : workspace_bytes);
    if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
      return fail(ASRATTN_ERR_WORKSPACE, "workspace must be 256-byte aligned");
    char* base = static_cast<char*>(workspace);
    ws_o = reinterpret_cast<float*>(base + w.partials);
    ws_ml = reinterpret_cast<float*>(base + w.stats);
  }
  return from_hip(asrattn::launch_decode(p, append, paged, s, ws_o, ws_ml, static_cast<hipStream_t>(stream)), name);
}

}  // namespace

int asrattn_decode(const asrattn_decode_params* params, void* workspace, size_t workspace_bytes, void* stream) {
  return run_decode(params, nullptr, nullptr, workspace, workspace_bytes, stream, "asrattn_decode");
}

}  // extern "C"

namespace {

// The split partials of asrattn_decode_noalloc: one array per GPU (each GPU
// holds its own copy at its own address), shared by every call on that GPU
// and kept until the process ends.  In host code `scratch` names a host-side
// stand-in, never the device memory: its device address comes from
// hipGetSymbolAddress, once per device, with that device current.
constexpr size_t kScratchBytes = ASRATTN_DECODE_NOALLOC_MAX_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device (which must be the
// device of `stream`).
int scratch_address(void* stream, void** out) {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return from_hip(err, "asrattn_decode_noalloc: hipGetDevice");
  if (device < 0 || device >= kMaxDevices)
    return fail(ASRATTN_ERR_UNSUPPORTED, "asrattn_decode_noalloc: device %d out of range", device);
  if (stream != nullptr) {
    int stream_device = -1;
    err = hipStreamGetDevice(static_cast<hipStream_t>(stream), &stream_device);
    if (err != hipSuccess) return from_hip(err, "asrattn_decode_noalloc: hipStreamGetDevice");
    if (stream_device != device)
      return fail(ASRATTN_ERR_INVALID, "asrattn_decode_noalloc: the stream is on device %d, the current device is %d",
                  stream_device, device);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device] == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr)
      return from_hip(err != hipSuccess ? err : hipErrorInvalidSymbol, "asrattn_decode_noalloc: hipGetSymbolAddress");
    g_scratch_ptr[device] = ptr;
  }
  *out = g_scratch_ptr[device];
  return ASRATTN_OK;
}

}  // namespace

extern "C" {

int asrattn_decode_noalloc(const asrattn_decode_params* params, void* stream) {
  const int checked = check_decode(params);
  if (checked != ASRATTN_OK) return checked;
  const size_t need = decode_workspace(*params, decode_splits(*params)).total;
  if (need > kScratchBytes)
    return fail(ASRATTN_ERR_WORKSPACE,
                "asrattn_decode_noalloc: %zu bytes of split partials exceed its %zu-byte scratch; use "
                "asrattn_decode with a workspace",
                need, kScratchBytes);
  if (need == 0 || params->batch == 0)
    return run_decode(params, nullptr, nullptr, nullptr, 0, stream, "asrattn_decode_noalloc");
  void* ptr = nullptr;
  const int rc = scratch_address(stream, &ptr);
  if (rc != ASRATTN_OK) return rc;
  return run_decode(params, nullptr, nullptr, ptr, kScratchBytes, stream, "asrattn_decode_noalloc");
}

size_t asrattn_choose_workspace_size(int64_t rows, int64_t vocab) {
  if (rows <= 0 || rows > 0x7fffffffLL || vocab < 1 || vocab >= (1LL << 29)) return 0;
  return asrattn::choose_workspace_bytes(rows, vocab);
}

int asrattn_choose(const float* logits, int64_t rows, int64_t vocab, int64_t row_stride, const uint8_t* suppress,
                   int64_t* token, float* logprob, void* workspace, size_t workspace_bytes, void* stream) {
  if (rows < 0 || rows > 0x7fffffffLL) return fail(ASRATTN_ERR_INVALID, "rows (%lld) out of range", (long long)rows);
  // Rows are addressed with 32-bit byte offsets.
  if (vocab < 1 || vocab >= (1LL << 29)) return fail(ASRATTN_ERR_INVALID, "vocab (%lld) out of range", (long long)vocab);
  if (row_stride < vocab) return fail(ASRATTN_ERR_INVALID, "row_stride must be at least vocab");
  if (rows == 0) return ok();
  if (logits == nullptr || token == nullptr || logprob == nullptr)
    return fail(ASRATTN_ERR_INVALID, "logits, token and logprob must be non-NULL");
  if (workspace != nullptr) {
    const size_t need = asrattn::choose_workspace_bytes(rows, vocab);
    if (workspace_bytes < need)
      return fail(ASRATTN_ERR_WORKSPACE, "choose workspace of %zu bytes, %zu needed", workspace_bytes, need);
    if (need == 0) workspace = nullptr;
  } else if (workspace_bytes != 0) {
    return fail(ASRATTN_ERR_INVALID, "workspace_bytes without a workspace");
  }
  return from_hip(asrattn::launch_choose(logits, rows, vocab, row_stride, suppress, token, logprob, workspace,
                                         static_cast<hipStream_t>(stream)),
                  "asrattn_choose");
}

int asrattn_decode_append(const asrattn_decode_params* params, const asrattn_append_params* append,
                          void* workspace, size_t workspace_bytes, void* stream) {
  if (append == nullptr) return fail(ASRATTN_ERR_INVALID, "append parameters must be non-NULL");
  return run_decode(params, append, nullptr, workspace, workspace_bytes, stream, "asrattn_decode_append");
}

int asrattn_local(const asrattn_local_params* params, void* stream) {
  if (params == nullptr) return fail(ASRATTN_ERR_INVALID, "params is NULL");
  const asrattn_local_params& p = *params;
  if (p.batch < 0 || p.tokens < 0 || p.heads <= 0 || p.head_dim <= 0)
    return fail(ASRATTN_ERR_INVALID, "batch, tokens, heads and head_dim must be >= 0 (heads, head_dim > 0)");
  if (p.chunk <= 0 || p.past < 0 || p.future < 0 || p.rel_positions < 0 || p.rel_positions > p.past + p.future + 2)
    return fail(ASRATTN_ERR_INVALID,
                "chunk must be > 0, past and future >= 0, and 0 <= rel_positions <= past + future + 2");
  if (!(p.softcap > 0.f) || !std::isfinite(p.softcap) || std::isnan(p.invalid))
    return fail(ASRATTN_ERR_INVALID, "softcap must be positive and finite, invalid not NaN");
  if (asrattn::local_lds_bytes(p) > 65536)
    return fail(ASRATTN_ERR_UNSUPPORTED, "a block's keys, values, queries and relative keys exceed 64 KB of LDS");
  if (p.batch == 0 || p.tokens == 0) return ok();
  if (p.q == nullptr || p.k == nullptr || p.v == nullptr || p.out == nullptr || p.lengths == nullptr ||
      (p.rel_positions > 0 && p.rel == nullptr))
    return fail(ASRATTN_ERR_INVALID, "q, k, v, out, lengths (and rel) must be non-NULL");
  return from_hip(asrattn::launch_local(p, static_cast<hipStream_t>(stream)), "asrattn_local");
}

int asrattn_decode_paged(const asrattn_decode_params* params, const asrattn_append_params* append,
                         const asrattn_paged_kv* paged, void* workspace, size_t workspace_bytes, void* stream) {
  if (paged == nullptr) return fail(ASRATTN_ERR_INVALID, "paged parameters must be non-NULL");
  return run_decode(params, append, paged, workspace, workspace_bytes, stream, "asrattn_decode_paged");
}

}  // extern "C"
