// Blocked local attention with relative position scores (Gemma 4's audio
// encoder; the math is asrattn_local's, include/asrattn.h).
//
// One workgroup (one wave) per (block of `chunk` queries, head, sequence).
// The block's context keys and values, its queries and the head's relative
// keys are staged in LDS as fp32; the wave then computes every (query,
// context slot) score -- content plus relative term -- soft-caps and masks
// it, takes each query's softmax and the weighted sum of the values.  The
// work is tiny (a few dozen keys per query) and fp32 like the reference's,
// so it stays on the vector ALUs.
#include "common.hpp"
#include "kernels.hpp"

namespace asrattn {
namespace {

constexpr int kLocalThreads = 64;

__global__ __launch_bounds__(kLocalThreads) void local_kernel(const asrattn_local_params p) {
  extern __shared__ float smem[];
  const int C = p.chunk, ctx = p.chunk + p.past + p.future, R = p.rel_positions, D = p.head_dim;
  const int u = blockIdx.x;  // block of queries
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int n = min(max(p.lengths[b], 0), p.tokens);  // valid keys of the sequence
  float* Ks = smem;            // [ctx][D]
  float* Vs = Ks + ctx * D;    // [ctx][D]
  float* Rs = Vs + ctx * D;    // [R][D]
  float* Qs = Rs + R * D;      // [C][D]
  float* Ss = Qs + C * D;      // [C][ctx]

  // Context slot t holds key u C - past + t (zeros outside the sequence's
  // tokens, as the reference's padding).
  for (int i = tid; i < ctx * D; i += kLocalThreads) {
    const int t = i / D, d = i % D;
    const int key = u * C - p.past + t;
    const bool in = key >= 0 && key < p.tokens;
    const int64_t ko = (int64_t)b * p.k_batch_stride + (int64_t)key * p.k_token_stride + (int64_t)h * p.k_head_stride;
    const int64_t vo = (int64_t)b * p.v_batch_stride + (int64_t)key * p.v_token_stride + (int64_t)h * p.v_head_stride;
    Ks[i] = in ? p.k[ko + d] : 0.f;
    Vs[i] = in ? p.v[vo + d] : 0.f;
  }
  for (int i = tid; i < R * D; i += kLocalThreads) {
    const int r = i / D, d = i % D;
    Rs[i] = p.rel[(int64_t)r * p.rel_position_stride + (int64_t)h * p.rel_head_stride + d];
  }
  for (int i = tid; i < C * D; i += kLocalThreads) {
    const int c = i / D, d = i % D;
    const int query = u * C + c;
    const int64_t qo = (int64_t)b * p.q_batch_stride + (int64_t)query * p.q_token_stride + (int64_t)h * p.q_head_stride;
    Qs[i] = query < p.tokens ? p.q[qo + d] : 0.f;
  }
  __syncthreads();

  // Scores: content q . k plus the relative term q . rel[t - c] (the
  // reference's relative shift: zero unless 0 <= t - c < R); soft-capped;
  // slots the query may not see take the invalid value.
  for (int i = tid; i < C * ctx; i += kLocalThreads) {
    const int c = i / ctx, t = i % ctx;
    const float* q = Qs + c * D;
    const float* k = Ks + t * D;
    float content = 0.f;
    for (int d = 0; d < D; ++d) content = fmaf(q[d], k[d], content);
    float position = 0.f;
    const int r = t - c;
    if (r >= 0 && r < R) {
      const float* rel = Rs + r * D;
      for (int d = 0; d < D; ++d) position = fmaf(q[d], rel[d], position);
    }
    const float capped = tanhf((content + position) / p.softcap) * p.softcap;
    const int query = u * C + c;
    const int key = u * C - p.past + t;
    const int distance = query - key;
    bool allowed = distance >= 0 && distance < p.past;
    if (p.future > 0) allowed = allowed || (distance < 0 && -distance < p.future);
    allowed = allowed && key >= 0 && key < n;
    Ss[i] = allowed ? capped : p.invalid;
  }
  __syncthreads();

  // Softmax over each query's context slots (natural exponent, as
  // F.softmax).
  for (int c = tid; c < C; c += kLocalThreads) {
    float* s = Ss + c * ctx;
    float mx = -__builtin_inff();
    for (int t = 0; t < ctx; ++t) mx = fmaxf(mx, s[t]);
    float sum = 0.f;
    for (int t = 0; t < ctx; ++t) {
      s[t] = expf(s[t] - mx);
      sum += s[t];
    }
    const float inv = 1.f / sum;
    for (int t = 0; t < ctx; ++t) s[t] *= inv;
  }
  __syncthreads();

  for (int i = tid; i < C * D; i += kLocalThreads) {
    const int c = i / D, d = i % D;
    const int query = u * C + c;
    if (query >= p.tokens) continue;
    const float* w = Ss + c * ctx;
    float acc = 0.f;
    for (int t = 0; t < ctx; ++t) acc = fmaf(w[t], Vs[t * D + d], acc);
    p.out[(int64_t)b * p.o_batch_stride + (int64_t)query * p.o_token_stride + (int64_t)h * p.o_head_stride + d] = acc;
  }
}

}  // namespace

size_t local_lds_bytes(const asrattn_local_params& p) {
  const size_t ctx = (size_t)p.chunk + p.past + p.future;
  return sizeof(float) * ((2 * ctx + p.rel_positions + p.chunk) * (size_t)p.head_dim + p.chunk * ctx);
}

hipError_t launch_local(const asrattn_local_params& p, hipStream_t stream) {
  const dim3 grid((unsigned)((p.tokens + p.chunk - 1) / p.chunk), (unsigned)p.heads, (unsigned)p.batch);
  hipLaunchKernelGGL(local_kernel, grid, dim3(kLocalThreads), local_lds_bytes(p), stream, p);
  return hipGetLastError();
}

}  // namespace asrattn
