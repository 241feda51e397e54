// Blocked local attention with relative position scores (Gemma 4's audio
// encoder; the math is asrattn_local's, include/asrattn.h).  The work per
// query is a few dozen keys in fp32, as the reference computes it, so it
// runs on the vector ALUs; a layer is bound by reading q, k, v and writing
// the output once.
//
// local_rows_kernel (head_dim 64..256, contexts up to 32 slots): a
// workgroup takes a run of consecutive blocks of one (sequence, head).  The
// run's context keys and values (each key serves two blocks) and the head's
// relative keys are staged in LDS; each query row belongs to four lanes,
// which hold a quarter of its dimensions in registers, sum their partial
// dot products with DPP and read key/value rows from LDS at the same
// addresses as the row's other queries (broadcast reads).
//
// local_kernel (any other shape): one wave per (block, head, sequence),
// one (query, slot) score per lane.
#include "common.hpp"
#include "kernels.hpp"

namespace asrattn {
namespace {

constexpr int kRowsThreads = 256;
constexpr int kRowsMaxContext = 32;
constexpr size_t kRowsLdsBudget = 64 * 1024;

// Sum over the four lanes of a query row (lanes 4k .. 4k + 3).
__device__ __forceinline__ float quad_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xb1, 0xf, 0xf, false));  // quad_perm 1,0,3,2
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4e, 0xf, 0xf, false));  // quad_perm 2,3,0,1
  return x;
}

// Dot product of this lane's DPL dimensions of q with an LDS row segment.
template <int DPL>
__device__ __forceinline__ float dot_lds(const float* q, const float* row) {
  float acc = 0.f;
#pragma unroll
  for (int d = 0; d < DPL; d += 4) {
    const float4 r = *reinterpret_cast<const float4*>(row + d);
    acc = fmaf(q[d], r.x, acc);
    acc = fmaf(q[d + 1], r.y, acc);
    acc = fmaf(q[d + 2], r.z, acc);
    acc = fmaf(q[d + 3], r.w, acc);
  }
  return acc;
}

template <int DPL>
__global__ __launch_bounds__(kRowsThreads) void local_rows_kernel(const asrattn_local_params p, int nblk) {
  extern __shared__ float smem[];
  constexpr int D = 4 * DPL;
  const int C = p.chunk, ctx = p.chunk + p.past + p.future, R = p.rel_positions;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int u0 = blockIdx.x * nblk;          // the run's first block
  const int key0 = u0 * C - p.past;          // key of staged row 0
  const int rows = nblk * C + p.past + p.future;
  const int n = min(max(p.lengths[b], 0), p.tokens);  // valid keys of the sequence
  const int tid = threadIdx.x;
  float* Ks = smem;          // [rows][D]
  float* Vs = Ks + rows * D;  // [rows][D]
  float* Rs = Vs + rows * D;  // [R][D]

  // Staged row r holds key key0 + r: zeros outside the sequence's tokens
  // (the reference's padding).
  for (int i = tid; i < rows * (D / 4); i += blockDim.x) {
    const int r = i / (D / 4), d = (i % (D / 4)) * 4;
    const int key = key0 + r;
    float4 kk = make_float4(0.f, 0.f, 0.f, 0.f), vv = kk;
    if (key >= 0 && key < p.tokens) {
      kk = *reinterpret_cast<const float4*>(p.k + (int64_t)b * p.k_batch_stride + (int64_t)key * p.k_token_stride +
                                            (int64_t)h * p.k_head_stride + d);
      vv = *reinterpret_cast<const float4*>(p.v + (int64_t)b * p.v_batch_stride + (int64_t)key * p.v_token_stride +
                                            (int64_t)h * p.v_head_stride + d);
    }
    *reinterpret_cast<float4*>(Ks + r * D + d) = kk;
    *reinterpret_cast<float4*>(Vs + r * D + d) = vv;
  }
  for (int i = tid; i < R * (D / 4); i += blockDim.x) {
    const int r = i / (D / 4), d = (i % (D / 4)) * 4;
    *reinterpret_cast<float4*>(Rs + r * D + d) =
        *reinterpret_cast<const float4*>(p.rel + (int64_t)r * p.rel_position_stride + (int64_t)h * p.rel_head_stride + d);
  }

  // This lane: dimensions [quarter DPL, +DPL) of query c of block u0 + ub.
  const int lq = tid >> 2, quarter = tid & 3;
  const int ub = lq / C, c = lq % C;
  const int query = (u0 + ub) * C + c;
  const bool active = ub < nblk && query < p.tokens;
  float q[DPL];
  {
    const float* qp = p.q + (int64_t)b * p.q_batch_stride + (int64_t)(active ? query : 0) * p.q_token_stride +
                      (int64_t)h * p.q_head_stride + quarter * DPL;
#pragma unroll
    for (int d = 0; d < DPL; d += 4) {
      const float4 t = active ? *reinterpret_cast<const float4*>(qp + d) : make_float4(0.f, 0.f, 0.f, 0.f);
      q[d] = t.x;
      q[d + 1] = t.y;
      q[d + 2] = t.z;
      q[d + 3] = t.w;
    }
  }
  __syncthreads();
  if (!active) return;  // no barrier follows; DPP partners share the row

  // Scores of the context slots: content q . k plus the relative term
  // q . rel[t - c] (the reference's relative shift: zero unless 0 <= t - c
  // < R), soft-capped; slots the query may not see take the invalid value.
  const float* krow = Ks + ub * C * D + quarter * DPL;  // slot t: staged row ub C + t
  float s[kRowsMaxContext];
  float mx = -__builtin_inff();
#pragma unroll
  for (int t = 0; t < kRowsMaxContext; ++t) {
    if (t < ctx) {
      float sc = quad_sum(dot_lds<DPL>(q, krow + t * D));
      const int r = t - c;
      if (R > 0) {
        const float pos = quad_sum(dot_lds<DPL>(q, Rs + min(max(r, 0), R - 1) * D + quarter * DPL));
        sc += (r >= 0 && r < R) ? pos : 0.f;
      }
      const float capped = tanhf(sc / p.softcap) * p.softcap;
      const int key = (u0 + ub) * C - p.past + t;
      const int distance = query - key;
      bool allowed = distance >= 0 && distance < p.past;
      if (p.future > 0) allowed = allowed || (distance < 0 && -distance < p.future);
      allowed = allowed && key >= 0 && key < n;
      s[t] = allowed ? capped : p.invalid;
      mx = fmaxf(mx, s[t]);
    }
  }
  // Softmax (natural exponent, as F.softmax) and the values' weighted sum.
  float sum = 0.f;
#pragma unroll
  for (int t = 0; t < kRowsMaxContext; ++t)
    if (t < ctx) {
      s[t] = expf(s[t] - mx);
      sum += s[t];
    }
  const float inv = 1.f / sum;
  float o[DPL];
#pragma unroll
  for (int d = 0; d < DPL; ++d) o[d] = 0.f;
  const float* vrow = Vs + ub * C * D + quarter * DPL;
#pragma unroll
  for (int t = 0; t < kRowsMaxContext; ++t)
    if (t < ctx) {
      const float w = s[t] * inv;
#pragma unroll
      for (int d = 0; d < DPL; d += 4) {
        const float4 v = *reinterpret_cast<const float4*>(vrow + t * D + d);
        o[d] = fmaf(w, v.x, o[d]);
        o[d + 1] = fmaf(w, v.y, o[d + 1]);
        o[d + 2] = fmaf(w, v.z, o[d + 2]);
        o[d + 3] = fmaf(w, v.w, o[d + 3]);
      }
    }
  float* op = p.out + (int64_t)b * p.o_batch_stride + (int64_t)query * p.o_token_stride +
              (int64_t)h * p.o_head_stride + quarter * DPL;
#pragma unroll
  for (int d = 0; d < DPL; d += 4) *reinterpret_cast<float4*>(op + d) = make_float4(o[d], o[d + 1], o[d + 2], o[d + 3]);
}

// Blocks per workgroup of local_rows_kernel (0: the shape does not fit it).
int rows_blocks(const asrattn_local_params& p) {
  const int D = p.head_dim;
  if (D != 64 && D != 128 && D != 192 && D != 256) return 0;
  if (p.chunk + p.past + p.future > kRowsMaxContext || 4 * p.chunk > kRowsThreads) return 0;
  // 16-byte loads and stores of every row.
  const void* ptrs[] = {p.q, p.k, p.v, p.rel, p.out};
  for (const void* ptr : ptrs)
    if (reinterpret_cast<uintptr_t>(ptr) % 16 != 0) return 0;
  const int64_t strides[] = {p.q_batch_stride, p.q_token_stride, p.q_head_stride, p.k_batch_stride,
                             p.k_token_stride, p.k_head_stride, p.v_batch_stride, p.v_token_stride,
                             p.v_head_stride, p.o_batch_stride, p.o_token_stride, p.o_head_stride,
                             p.rel_position_stride, p.rel_head_stride};
  for (int64_t st : strides)
    if (st % 4 != 0) return 0;
  for (int nblk = kRowsThreads / (4 * p.chunk); nblk > 0; --nblk) {
    const size_t rows = (size_t)nblk * p.chunk + p.past + p.future;
    if (sizeof(float) * (2 * rows + p.rel_positions) * D <= kRowsLdsBudget) return nblk;
  }
  return 0;
}

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
  const int blocks = (p.tokens + p.chunk - 1) / p.chunk;
  const int nblk = rows_blocks(p);
  if (nblk > 0) {
    const dim3 grid((unsigned)((blocks + nblk - 1) / nblk), (unsigned)p.heads, (unsigned)p.batch);
    const int threads = (4 * nblk * p.chunk + 63) / 64 * 64;
    const size_t rows = (size_t)nblk * p.chunk + p.past + p.future;
    const size_t lds = sizeof(float) * (2 * rows + p.rel_positions) * p.head_dim;
    switch (p.head_dim) {
      case 64: hipLaunchKernelGGL(local_rows_kernel<16>, grid, dim3(threads), lds, stream, p, nblk); break;
      case 128: hipLaunchKernelGGL(local_rows_kernel<32>, grid, dim3(threads), lds, stream, p, nblk); break;
      case 192: hipLaunchKernelGGL(local_rows_kernel<48>, grid, dim3(threads), lds, stream, p, nblk); break;
      default: hipLaunchKernelGGL(local_rows_kernel<64>, grid, dim3(threads), lds, stream, p, nblk); break;
    }
    return hipGetLastError();
  }
  const dim3 grid((unsigned)blocks, (unsigned)p.heads, (unsigned)p.batch);
  hipLaunchKernelGGL(local_kernel, grid, dim3(kLocalThreads), local_lds_bytes(p), stream, p);
  return hipGetLastError();
}

}  // namespace asrattn
