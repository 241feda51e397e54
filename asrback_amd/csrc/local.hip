// Blocked local attention with relative position scores (Gemma 4's audio
// encoder; the math is asrattn_local's, include/asrattn.h).  The work per
// query is a few dozen keys in fp32, as the reference computes it, so it
// runs on the vector ALUs; a layer is bound by reading q, k, v and writing
// the output once.
//
// local_mfma_kernel (head_dim 64, 128 or 192, blocks of at most 16
// queries over at most 32 context slots): a workgroup walks runs of
// consecutive blocks of one (sequence, head), one wave per block, loading
// the next run's operands while the current one computes.  A run's values
// (each serves two blocks) and the head's relative keys are staged in LDS,
// the queries and keys go straight to registers; each wave computes
// its block's scores, relative terms and weighted values as fp32 matrix
// products on the matrix cores
// (v_mfma_f32_16x16x4_f32, fp32 operands and accumulation), transposed as
// in the bf16 encoder kernel so that a query's scores stay in its lanes:
//   S^T = K . Q^T and R^T = Rel . Q^T (16 context slots or relative rows x
//   16 queries per product), P^T from S^T in registers, O^T = V^T . P^T.
//
// local_kernel (any other shape): one wave per (block, head, sequence),
// one (query, slot) score per lane.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace asrattn {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kMfmaMaxWaves = 4;
constexpr int kMfmaMaxContext = 32;  // two 16-slot tiles
constexpr size_t kMfmaLdsBudget = 64 * 1024;

// 16 x 16 x 4 fp32 product, lane l: A[l % 16][l / 16], B[l / 16][l % 16],
// D[4 (l / 16) + r][l % 16] (layout checked on the GPU).
__device__ __forceinline__ f32x4_t mfma16(float a, float b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// LDS floats of a workgroup of nblk blocks: the values of its rows and 16
// relative rows (padded with zeros), each row padded by 4 floats so that the
// value reads of a product (four rows four apart, 16 columns) hit distinct
// banks; then per wave 16 x 17 relative scores.
size_t mfma_lds_floats(const asrattn_local_params& p, int nblk) {
  const size_t rows = (size_t)nblk * p.chunk + p.past + p.future;
  return (rows + 16) * (p.head_dim + 4) + (size_t)nblk * 16 * 17;
}

// Staging copies in flight per thread (16-byte loads issued before their
// LDS stores).
constexpr int kStageBatch = 8;
// Relative-key copies per thread issued ahead of the first run's loads
// (every chunk at head_dim up to 192 with four waves).
constexpr int kRelBatch = 3;

template <int KS>  // head_dim / 4: k-steps of a product over the head dimensions
__global__ __launch_bounds__(64 * kMfmaMaxWaves, 2) void local_mfma_kernel(const asrattn_local_params p, int nblk,
                                                                            int rpw) {
  extern __shared__ float smem[];
  constexpr int D = 4 * KS, RS = D + 4;
  constexpr bool kPrefetch = KS <= 32;
  const int C = p.chunk, ctx = p.chunk + p.past + p.future, R = p.rel_positions;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int runs = ((p.tokens + C - 1) / C + nblk - 1) / nblk;
  // The workgroup's runs: r0 .. r1 - 1 (one at head_dim 192, which has no
  // registers for the next run's operands).
  const int r0 = blockIdx.x * rpw;
  const int r1 = kPrefetch ? min(runs, r0 + rpw) : r0 + 1;
  const int rows = nblk * C + p.past + p.future;
  const int n = min(max(p.lengths[b], 0), p.tokens);  // valid keys of the sequence
  const int tid = threadIdx.x;
  float* Vs = smem;            // [rows][RS]
  float* Rs = Vs + rows * RS;  // [16][RS]
  float* Xs = Rs + 16 * RS;    // [wave][16][17]

  // Lane (col, m): query column col of the wave's block; k slot m of
  // product step 4 j + e is head dimension 16 j + 4 m + e (any order of the
  // dimensions over the k slots gives the same sums), so a row's operands
  // are 16-byte loads of which four lanes cover 64 contiguous bytes.
  const int lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, m = lane >> 4;
  // Every row goes through a buffer resource that ends at the sequence's
  // last token, so tokens outside [0, tokens) read as zeros (the reference's
  // padding; offsets of negative keys wrap past the end) with no branch.
  const uint32_t qts = (uint32_t)p.q_token_stride * 4, kts = (uint32_t)p.k_token_stride * 4;
  const uint32_t vts = (uint32_t)p.v_token_stride * 4, rps = (uint32_t)p.rel_position_stride * 4;
  const __amdgpu_buffer_rsrc_t qrs =
      buffer_rsrc(p.q + (int64_t)b * p.q_batch_stride + (int64_t)h * p.q_head_stride, (uint32_t)p.tokens * qts);
  const __amdgpu_buffer_rsrc_t krs =
      buffer_rsrc(p.k + (int64_t)b * p.k_batch_stride + (int64_t)h * p.k_head_stride, (uint32_t)p.tokens * kts);
  const __amdgpu_buffer_rsrc_t vrs =
      buffer_rsrc(p.v + (int64_t)b * p.v_batch_stride + (int64_t)h * p.v_head_stride, (uint32_t)p.tokens * vts);
  const __amdgpu_buffer_rsrc_t rrs = buffer_rsrc(p.rel + (int64_t)h * p.rel_head_stride, (uint32_t)R * rps);

  // The query col of the wave's block in run `run` and the keys of context
  // slots col and 16 + col, straight into the product operands.  Query
  // columns past the block and slots past the context read nothing (an
  // offset past every range; their results are never stored or are dropped
  // from the softmax below).
  // Context slot of row 4 mm + r of score tile nt, or -1.  With at most 24
  // slots the second tile's (at most 8) sit in its rows 4 mm + {0, 1}, so
  // the value product skips that tile's steps r = 2, 3.
  const bool packed = ctx <= 24;
  auto slot_of = [&](int nt, int mm, int r) -> int {
    if (nt == 0) return 4 * mm + r;
    if (packed) return r < 2 ? 16 + 2 * mm + r : -1;
    return 16 + 4 * mm + r;
  };
  float qv[KS], kv[2][KS];
  auto load_qk = [&](int run) {
    constexpr uint32_t kNowhere = 0x80000000u;  // past any range (ranges stay below 2^31)
    const int u = run * nblk + wave;
    const uint32_t dim0 = (uint32_t)m * 16;
    const uint32_t qo = col < C ? (uint32_t)(u * C + col) * qts + dim0 : kNowhere;
    const int key = u * C - p.past + col;
    const uint32_t ko0 = col < ctx ? (uint32_t)key * kts + dim0 : kNowhere;
    const int t1 = slot_of(1, col >> 2, col & 3);  // the slot of tile 1's row col
    const uint32_t ko1 = t1 >= 0 && t1 < ctx ? (uint32_t)(key - col + t1) * kts + dim0 : kNowhere;
#pragma unroll
    for (int d = 0; d < KS; d += 4) {
      const float4 t = __builtin_bit_cast(float4, buffer_load16(qrs, qo + d * 16));
      const float4 k0 = __builtin_bit_cast(float4, buffer_load16(krs, ko0 + d * 16));
      const float4 k1 = __builtin_bit_cast(float4, buffer_load16(krs, ko1 + d * 16));
      qv[d] = t.x, qv[d + 1] = t.y, qv[d + 2] = t.z, qv[d + 3] = t.w;
      kv[0][d] = k0.x, kv[0][d + 1] = k0.y, kv[0][d + 2] = k0.z, kv[0][d + 3] = k0.w;
      kv[1][d] = k1.x, kv[1][d + 1] = k1.y, kv[1][d + 2] = k1.z, kv[1][d + 3] = k1.w;
    }
  };

  // Staged value row r of run `run` holds key run nblk C - past + r.  Loads
  // go out in batches ahead of their stores; the last batch's surplus
  // threads repeat the last chunk (same value, same place).
  const int vchunks = rows * KS;
  const int vstride = kStageBatch * (int)blockDim.x;
  float4 x[kStageBatch];
  auto load_v = [&](int run, int base) {
    const int key0 = run * nblk * C - p.past;
#pragma unroll
    for (int j = 0; j < kStageBatch; ++j) {
      const int i = min(base + j * (int)blockDim.x, vchunks - 1);
      x[j] = __builtin_bit_cast(float4, buffer_load16(vrs, (uint32_t)(key0 + i / KS) * vts + (uint32_t)(i % KS) * 16));
    }
  };
  auto store_v = [&](int base) {
#pragma unroll
    for (int j = 0; j < kStageBatch; ++j) {
      const int i = min(base + j * (int)blockDim.x, vchunks - 1);
      *reinterpret_cast<float4*>(Vs + (i / KS) * RS + (i % KS) * 4) = x[j];
    }
  };
  // The first batch comes from loads issued earlier (x); the rest load here.
  auto stage_rest = [&](int run) {
    store_v(tid);
    for (int base = tid + vstride; base < vchunks; base += vstride) {
      load_v(run, base);
      store_v(base);
    }
  };

  // The head's relative keys (16 rows, zeros past R) serve every run.  Their
  // loads go out first, so that storing them waits for nothing else; the
  // first run's queries and keys follow, then its values, which are only
  // needed after its scores.
  const int rchunks = 16 * KS;
  float4 rl[kRelBatch];
#pragma unroll
  for (int j = 0; j < kRelBatch; ++j) {
    const int i = min(tid + j * (int)blockDim.x, rchunks - 1);
    rl[j] = __builtin_bit_cast(float4, buffer_load16(rrs, (uint32_t)(i / KS) * rps + (uint32_t)(i % KS) * 16));
  }
  load_qk(r0);
  load_v(r0, tid);
#pragma unroll
  for (int j = 0; j < kRelBatch; ++j) {
    const int i = min(tid + j * (int)blockDim.x, rchunks - 1);
    *reinterpret_cast<float4*>(Rs + (i / KS) * RS + (i % KS) * 4) = rl[j];
  }
  for (int i = tid + kRelBatch * (int)blockDim.x; i < rchunks; i += blockDim.x)
    *reinterpret_cast<float4*>(Rs + (i / KS) * RS + (i % KS) * 4) =
        __builtin_bit_cast(float4, buffer_load16(rrs, (uint32_t)(i / KS) * rps + (uint32_t)(i % KS) * 16));
  __syncthreads();

  const float inv_cap = 1.f / p.softcap;
  float* xs = Xs + wave * 16 * 17;
  for (int run = r0; run < r1; ++run) {
    const int u = run * nblk + wave;
    const int query = u * C + col;
    const bool qok = col < C && query < p.tokens;

    // S^T: context slot 16 nt + col against query column col.
    f32x4_t st[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      st[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int d = 0; d < KS; ++d) st[nt] = mfma16(kv[nt][d], qv[d], st[nt]);
    }
    // Relative scores R^T[row][query]; lane holds rows 4 m + r of column col.
    f32x4_t rt = f32x4_t{0.f, 0.f, 0.f, 0.f};
    {
      const float* rr = Rs + col * RS + 4 * m;
#pragma unroll
      for (int d = 0; d < KS; d += 4) {
        const float4 rv = *reinterpret_cast<const float4*>(rr + 4 * d);
        rt = mfma16(rv.x, qv[d], rt);
        rt = mfma16(rv.y, qv[d + 1], rt);
        rt = mfma16(rv.z, qv[d + 2], rt);
        rt = mfma16(rv.w, qv[d + 3], rt);
      }
    }
    // The next run's queries and keys go out now, into the registers just
    // freed, and arrive while this run finishes.
    const bool more = run + 1 < r1;
    if (more) {
      __builtin_amdgcn_sched_barrier(0);
      load_qk(run + 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    // The reference's relative shift: slot t of query c adds relative row
    // t - c when 0 <= t - c < R; rows move between lanes through LDS.
#pragma unroll
    for (int r = 0; r < 4; ++r) xs[col * 17 + 4 * m + r] = rt[r];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // Soft cap and mask; slots past the context are not part of the softmax.
    float s[8];
    float mx = -__builtin_inff();
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = slot_of(nt, m, r);
        const int dr = t - col;
        const float rel = xs[col * 17 + min(max(dr, 0), 15)];
        const float sc = st[nt][r] + ((dr >= 0 && dr < R) ? rel : 0.f);
        const float capped = tanhf(sc * inv_cap) * p.softcap;
        const int key = u * C - p.past + t;
        const int distance = query - key;
        bool allowed = distance >= 0 && distance < p.past;
        if (p.future > 0) allowed = allowed || (distance < 0 && -distance < p.future);
        allowed = allowed && key >= 0 && key < n;
        const float v = t < 0 || t >= ctx ? -__builtin_inff() : allowed ? capped : p.invalid;
        s[4 * nt + r] = v;
        mx = fmaxf(mx, v);
      }
    // A query's slots live in lanes col, col + 16, col + 32, col + 48.
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      s[i] = expf(s[i] - mx);  // natural exponent, as F.softmax; 0 past the context
      sum += s[i];
    }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);

    // This run's values into LDS once every wave is done with the last
    // run's; then the next run's first values go out.
    __syncthreads();
    stage_rest(run);
    __syncthreads();
    if (more) load_v(run + 1, tid);

    // O^T = V^T . P^T: step (nt, r) takes slot slot_of(nt, m, r) in k slot
    // m, the same slot this lane's P^T register holds.
    f32x4_t ot[KS / 4];
#pragma unroll
    for (int d = 0; d < KS / 4; ++d) ot[d] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (nt == 1 && packed && r >= 2) continue;  // uniform: rows without a slot
        const int t = slot_of(nt, m, r);
        const bool in = t >= 0 && t < ctx;
        const float* vr = Vs + min(wave * C + max(t, 0), rows - 1) * RS + col;
#pragma unroll
        for (int d = 0; d < KS / 4; ++d) {
          const float x = vr[16 * d];
          ot[d] = mfma16(in ? x : 0.f, s[4 * nt + r], ot[d]);
        }
      }
    if (qok) {
      const float inv = 1.f / sum;
      float* op = p.out + (int64_t)b * p.o_batch_stride + (int64_t)query * p.o_token_stride +
                  (int64_t)h * p.o_head_stride + 4 * m;
#pragma unroll
      for (int d = 0; d < KS / 4; ++d)
        *reinterpret_cast<float4*>(op + 16 * d) =
            make_float4(ot[d][0] * inv, ot[d][1] * inv, ot[d][2] * inv, ot[d][3] * inv);
    }
  }
}

// Blocks (waves) per workgroup of local_mfma_kernel; 0: the shape does not
// fit it.
int mfma_blocks(const asrattn_local_params& p) {
  if (p.head_dim != 64 && p.head_dim != 128 && p.head_dim != 192) return 0;
  if (p.chunk > 16 || p.chunk + p.past + p.future > kMfmaMaxContext || p.rel_positions > 16) return 0;
  // Buffer offsets are 32-bit, with everything at or past 2^31 out of range
  // (negative keys, at least -past, wrap to 2^32 - past * stride).
  const int64_t token_strides[] = {p.q_token_stride, p.k_token_stride, p.v_token_stride};
  for (int64_t st : token_strides)
    if (st < p.head_dim || ((int64_t)p.tokens + p.past + 32) * st * 4 >= (1LL << 31)) return 0;
  if ((int64_t)p.rel_positions * p.rel_position_stride * 4 >= (1LL << 31)) return 0;
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
  for (int nblk = kMfmaMaxWaves; nblk > 0; --nblk)
    if (sizeof(float) * mfma_lds_floats(p, nblk) <= kMfmaLdsBudget) return nblk;
  return 0;
}

// Runs per workgroup of local_mfma_kernel: as few as let the whole grid be
// resident at once (two waves per SIMD, the LDS per CU), so that every
// workgroup's next run loads while its current one computes instead of a
// second round of workgroups loading after the first has finished.
int mfma_runs_per_workgroup(const asrattn_local_params& p, int nblk, int runs, size_t lds) {
  int device = 0, cus = 0;
  if (hipGetDevice(&device) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0)
    cus = 256;
  const int per_cu = std::max(1, std::min(8 / nblk, (int)(160 * 1024 / lds)));
  const long long slots = (long long)cus * per_cu;
  const long long total = (long long)runs * p.heads * p.batch;
  const long long rpw = (total + slots - 1) / slots;
  return (int)std::max(1LL, std::min(rpw, (long long)runs));
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
  const int nblk = mfma_blocks(p);
  if (nblk > 0) {
    const int runs = (blocks + nblk - 1) / nblk;
    const size_t lds = sizeof(float) * mfma_lds_floats(p, nblk);
    const int rpw = p.head_dim == 192 ? 1 : mfma_runs_per_workgroup(p, nblk, runs, lds);
    const dim3 grid((unsigned)((runs + rpw - 1) / rpw), (unsigned)p.heads, (unsigned)p.batch);
    switch (p.head_dim) {
      case 64: hipLaunchKernelGGL(local_mfma_kernel<16>, grid, dim3(64 * nblk), lds, stream, p, nblk, rpw); break;
      case 128: hipLaunchKernelGGL(local_mfma_kernel<32>, grid, dim3(64 * nblk), lds, stream, p, nblk, rpw); break;
      default: hipLaunchKernelGGL(local_mfma_kernel<48>, grid, dim3(64 * nblk), lds, stream, p, nblk, rpw); break;
    }
    return hipGetLastError();
  }
  const dim3 grid((unsigned)blocks, (unsigned)p.heads, (unsigned)p.batch);
  hipLaunchKernelGGL(local_kernel, grid, dim3(kLocalThreads), local_lds_bytes(p), stream, p);
  return hipGetLastError();
}

}  // namespace asrattn
