// Decoder-step attention: one query per sequence over a key/value cache.
//
// The step is bound by HBM: every key and value of a sequence is read once
// and used for one (or, with grouped-query attention, g) dot products.  The
// kernel therefore streams K and V with 16-byte loads, many in flight per
// lane, and keeps all arithmetic in registers:
//
//   * A key row (head_dim elements) is covered by LPK lanes, 16 bytes each;
//     a wave loads 64 / LPK key rows per instruction, so every load touches
//     whole rows.  Each group of LPK lanes runs its own online softmax over
//     the keys it reads (a "stream"); the g query heads sharing the kv head
//     ride along on the same loads.
//   * The keys of a sequence are split over gridDim.x workgroups (split-K);
//     the streams of a workgroup merge in LDS and each split writes an
//     unnormalized partial (o, max, sum) to the workspace, which the combine
//     pass folds into the output.  A single split writes the output directly.
//   * Sequence lengths are read from device memory (seqused_k or
//     positions + 1), and splits past a sequence's end write an empty
//     partial, so the grid depends only on shapes and the launch can be
//     replayed from a graph while lengths change.
//
// Softmax runs in base 2: q is pre-multiplied by scale * log2(e), so
// p = 2^(s - max) on v_exp_f32.
#include "common.hpp"
#include "kernels.hpp"

namespace asrattn {
namespace {

struct DecodeArgs {
  asrattn_decode_params p;
  float* ws_o;
  float* ws_ml;
  int splits;
  float c;  // scale * log2(e)
};

constexpr int kDecodeThreads = 256;  // four waves per workgroup

template <typename T, int HD>
struct DecodeShape {
  static constexpr int kEPL = Elem<T>::kPerVec;   // elements per lane per load
  static constexpr int kLPK = HD / kEPL;          // lanes per key row
  static constexpr int kKPW = 64 / kLPK;          // key rows per wave load
  static constexpr int kThreads = kDecodeThreads;
  static constexpr int kWaves = kThreads / 64;
  static constexpr int kStreams = kWaves * kKPW;  // softmax streams per workgroup
  static constexpr int kUnroll = 8;               // keys per stream per iteration
  static_assert(kLPK >= 1 && kLPK <= 64 && (64 % kLPK) == 0, "head_dim/lane mapping");
};

template <typename T>
__device__ __forceinline__ uint4 load_vec(const T* p) {
  return *reinterpret_cast<const uint4*>(p);
}

template <typename T>
__device__ __forceinline__ void unpack(const uint4& r, float* out);

template <>
__device__ __forceinline__ void unpack<float>(const uint4& r, float* out) {
  out[0] = __uint_as_float(r.x); out[1] = __uint_as_float(r.y);
  out[2] = __uint_as_float(r.z); out[3] = __uint_as_float(r.w);
}

template <>
__device__ __forceinline__ void unpack<bf16_raw>(const uint4& r, float* out) {
  out[0] = bf16_lo(r.x); out[1] = bf16_hi(r.x);
  out[2] = bf16_lo(r.y); out[3] = bf16_hi(r.y);
  out[4] = bf16_lo(r.z); out[5] = bf16_hi(r.z);
  out[6] = bf16_lo(r.w); out[7] = bf16_hi(r.w);
}

template <typename T, int HD, int G>
__global__ __launch_bounds__(kDecodeThreads) void decode_split_kernel(const DecodeArgs a) {
  using S = DecodeShape<T, HD>;
  constexpr int EPL = S::kEPL, LPK = S::kLPK, NS = S::kStreams, U = S::kUnroll;
  const asrattn_decode_params& p = a.p;

  const int split = blockIdx.x;
  const int hkv = blockIdx.y;
  const int b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = lane % LPK;
  const int stream = wave * S::kKPW + lane / LPK;

  const int n = decode_key_count(p.seqused_k, p.positions, b, p.max_len_k);
  const int chunk = (n + a.splits - 1) / a.splits;
  const int k0 = min(n, split * chunk);
  const int k1 = min(n, k0 + chunk);

  // Queries of the G heads sharing kv head hkv, pre-scaled into base 2.
  float q[G][EPL];
  {
    const T* qp = static_cast<const T*>(p.q) + (int64_t)b * p.q_batch_stride +
                  (int64_t)hkv * G * p.q_head_stride + sub * EPL;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      unpack<T>(load_vec(qp + (int64_t)g * p.q_head_stride), q[g]);
#pragma unroll
      for (int e = 0; e < EPL; ++e) q[g][e] *= a.c;
    }
  }

  float m[G], l[G], o[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kNegInf;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) o[g][e] = 0.f;
  }

  const T* kp = static_cast<const T*>(p.k) + (int64_t)b * p.k_batch_stride +
                (int64_t)hkv * p.k_head_stride + sub * EPL;
  const T* vp = static_cast<const T*>(p.v) + (int64_t)b * p.v_batch_stride +
                (int64_t)hkv * p.v_head_stride + sub * EPL;

  for (int base = k0; base < k1; base += NS * U) {
    uint4 kr[U], vr[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = base + u * NS + stream;
      if (j < k1) {
        kr[u] = load_vec(kp + (int64_t)j * p.k_token_stride);
        vr[u] = load_vec(vp + (int64_t)j * p.v_token_stride);
      } else {
        kr[u] = make_uint4(0, 0, 0, 0);
        vr[u] = make_uint4(0, 0, 0, 0);
      }
    }

    float s[U][G];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float kf[EPL];
      unpack<T>(kr[u], kf);
      const bool valid = base + u * NS + stream < k1;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc = fmaf(q[g][e], kf[e], acc);
        acc = group_sum<LPK>(acc);
        s[u][g] = valid ? acc : kNegInf;
      }
    }

    float mu[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mt = s[0][g];
#pragma unroll
      for (int u = 1; u < U; ++u) mt = fmaxf(mt, s[u][g]);
      const float mn = fmaxf(m[g], mt);
      mu[g] = mn == kNegInf ? 0.f : mn;
      const float alpha = fast_exp2(m[g] - mu[g]);
      l[g] *= alpha;
#pragma unroll
      for (int e = 0; e < EPL; ++e) o[g][e] *= alpha;
      m[g] = mn;
    }

#pragma unroll
    for (int u = 0; u < U; ++u) {
      float vf[EPL];
      unpack<T>(vr[u], vf);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pu = fast_exp2(s[u][g] - mu[g]);
        l[g] += pu;
#pragma unroll
        for (int e = 0; e < EPL; ++e) o[g][e] = fmaf(pu, vf[e], o[g][e]);
      }
    }
  }

  // Merge the workgroup's streams.
  __shared__ float sm_m[NS][G];
  __shared__ float sm_l[NS][G];
  __shared__ float sm_o[NS][G][HD];
  if (sub == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      sm_m[stream][g] = m[g];
      sm_l[stream][g] = l[g];
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < EPL; ++e) sm_o[stream][g][sub * EPL + e] = o[g][e];
  __syncthreads();

  for (int t = threadIdx.x; t < G * HD; t += S::kThreads) {
    const int g = t / HD;
    const int d = t % HD;
    float mx = kNegInf;
    for (int s2 = 0; s2 < NS; ++s2) mx = fmaxf(mx, sm_m[s2][g]);
    const float mxu = mx == kNegInf ? 0.f : mx;
    float lsum = 0.f, osum = 0.f;
    for (int s2 = 0; s2 < NS; ++s2) {
      const float w = fast_exp2(sm_m[s2][g] - mxu);
      lsum = fmaf(sm_l[s2][g], w, lsum);
      osum = fmaf(sm_o[s2][g][d], w, osum);
    }
    const int hq = hkv * G + g;
    if (a.splits == 1) {
      T* op = static_cast<T*>(p.out) + (int64_t)b * p.o_batch_stride + (int64_t)hq * p.o_head_stride + d;
      Elem<T>::store1(op, lsum > 0.f ? osum / lsum : 0.f);
    } else {
      const int64_t idx = ((int64_t)b * p.heads_q + hq) * a.splits + split;
      a.ws_o[idx * HD + d] = osum;
      if (d == 0) {
        a.ws_ml[idx * 2] = mx;
        a.ws_ml[idx * 2 + 1] = lsum;
      }
    }
  }
}

// Folds the splits' partials of one (sequence, query head) into the output.
template <typename T, int HD>
__global__ __launch_bounds__(HD) void decode_combine_kernel(const DecodeArgs a) {
  const asrattn_decode_params& p = a.p;
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int d = threadIdx.x;
  const int64_t idx0 = ((int64_t)b * p.heads_q + hq) * a.splits;
  float mx = kNegInf;
  for (int s = 0; s < a.splits; ++s) mx = fmaxf(mx, a.ws_ml[(idx0 + s) * 2]);
  const float mxu = mx == kNegInf ? 0.f : mx;
  float lsum = 0.f, osum = 0.f;
  for (int s = 0; s < a.splits; ++s) {
    const float w = fast_exp2(a.ws_ml[(idx0 + s) * 2] - mxu);
    lsum = fmaf(a.ws_ml[(idx0 + s) * 2 + 1], w, lsum);
    osum = fmaf(a.ws_o[(idx0 + s) * HD + d], w, osum);
  }
  T* op = static_cast<T*>(p.out) + (int64_t)b * p.o_batch_stride + (int64_t)hq * p.o_head_stride + d;
  Elem<T>::store1(op, lsum > 0.f ? osum / lsum : 0.f);
}

template <typename T, int HD, int G>
hipError_t launch_typed(const DecodeArgs& a, hipStream_t stream) {
  using S = DecodeShape<T, HD>;
  const asrattn_decode_params& p = a.p;
  dim3 grid(a.splits, p.heads_kv, p.batch);
  hipLaunchKernelGGL((decode_split_kernel<T, HD, G>), grid, dim3(S::kThreads), 0, stream, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || a.splits == 1) return err;
  hipLaunchKernelGGL((decode_combine_kernel<T, HD>), dim3(p.heads_q, p.batch), dim3(HD), 0, stream, a);
  return hipGetLastError();
}

template <typename T, int HD>
hipError_t launch_hd(const DecodeArgs& a, int group, hipStream_t stream) {
  switch (group) {
    case 1: return launch_typed<T, HD, 1>(a, stream);
    case 2: return launch_typed<T, HD, 2>(a, stream);
    case 4: return launch_typed<T, HD, 4>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool decode_supported(int dtype, int head_dim, int group) {
  const bool dt = dtype == ASRATTN_F32 || dtype == ASRATTN_BF16;
  const bool hd = head_dim == 64 || head_dim == 128;
  const bool g = group == 1 || group == 2 || group == 4;
  return dt && hd && g;
}

hipError_t launch_decode(const asrattn_decode_params& p, int splits, float* ws_o, float* ws_ml,
                         hipStream_t stream) {
  DecodeArgs a;
  a.p = p;
  a.ws_o = ws_o;
  a.ws_ml = ws_ml;
  a.splits = splits;
  a.c = p.scale * kLog2e;
  const int group = p.heads_q / p.heads_kv;
  if (p.dtype == ASRATTN_BF16) {
    return p.head_dim == 64 ? launch_hd<bf16_raw, 64>(a, group, stream)
                            : launch_hd<bf16_raw, 128>(a, group, stream);
  }
  return p.head_dim == 64 ? launch_hd<float, 64>(a, group, stream)
                          : launch_hd<float, 128>(a, group, stream);
}

}  // namespace asrattn
