// Multi-row attention on the vector ALUs, fp32 arithmetic throughout.
//
// One wave per workgroup; each lane owns one query row (its scaled query and
// output accumulator stay in registers).  Key/value tiles of kBN rows are
// staged in LDS as fp32 and read by all lanes at the same address
// (broadcast, no bank conflicts).  This is the fp32 path (Whisper in
// float32, the reference's CPU/fp32 dtype) and the exact-arithmetic twin of
// the bf16 matrix-core kernel.
#include "common.hpp"
#include "fwd_common.hpp"
#include "kernels.hpp"

namespace asrattn {
namespace {

constexpr int kRows = 64;  // query rows per workgroup (one per lane)
constexpr int kBN = 32;    // keys per LDS tile

template <typename T, int HD>
__global__ __launch_bounds__(kRows) void fwd_valu_kernel(const FwdArgs a) {
  constexpr int EPV = Elem<T>::kPerVec;
  const asrattn_fwd_params& p = a.p;
  const int hq = blockIdx.y;
  const int b = blockIdx.z;
  const int hkv = hq / (p.heads_q / p.heads_kv);
  const SeqView sv = seq_view(p, b, hq, hkv);
  const int row0 = blockIdx.x * kRows;
  if (row0 >= sv.len_q) return;  // uniform over the workgroup

  const int lane = threadIdx.x;
  const int row = row0 + lane;
  const bool row_ok = row < sv.len_q;
  const int row_lim = visible_keys(p, sv, row);
  const int kend = visible_keys(p, sv, min(row0 + kRows, sv.len_q) - 1);

  float q[HD], o[HD];
  {
    const T* qp = static_cast<const T*>(p.q) + sv.q_off + (int64_t)(row_ok ? row : 0) * p.q_token_stride;
#pragma unroll
    for (int d = 0; d < HD; d += EPV) {
      float t[EPV];
      Elem<T>::load16(qp + d, t);
#pragma unroll
      for (int e = 0; e < EPV; ++e) q[d + e] = row_ok ? t[e] * a.c : 0.f;
    }
#pragma unroll
    for (int d = 0; d < HD; ++d) o[d] = 0.f;
  }
  float m = kNegInf, l = 0.f;

  __shared__ float Ks[kBN][HD];
  __shared__ float Vs[kBN][HD];
  const T* kbase = static_cast<const T*>(p.k) + sv.k_off;
  const T* vbase = static_cast<const T*>(p.v) + sv.v_off;

  for (int kt = 0; kt < kend; kt += kBN) {
    __syncthreads();
    constexpr int kVecs = kBN * HD / EPV;
    for (int c = lane; c < kVecs; c += kRows) {
      const int j = c / (HD / EPV);
      const int d = (c % (HD / EPV)) * EPV;
      float tk[EPV], tv[EPV];
      if (kt + j < kend) {
        Elem<T>::load16(kbase + (int64_t)(kt + j) * p.k_token_stride + d, tk);
        Elem<T>::load16(vbase + (int64_t)(kt + j) * p.v_token_stride + d, tv);
      } else {
#pragma unroll
        for (int e = 0; e < EPV; ++e) tk[e] = tv[e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        Ks[j][d + e] = tk[e];
        Vs[j][d + e] = tv[e];
      }
    }
    __syncthreads();

    float s[kBN];
    float mt = kNegInf;
#pragma unroll
    for (int j = 0; j < kBN; ++j) {
      float acc = 0.f;
#pragma unroll
      for (int d = 0; d < HD; ++d) acc = fmaf(q[d], Ks[j][d], acc);
      s[j] = kt + j < row_lim ? acc : kNegInf;
      mt = fmaxf(mt, s[j]);
    }
    const float mn = fmaxf(m, mt);
    const float mu = mn == kNegInf ? 0.f : mn;
    const float alpha = fast_exp2(m - mu);
    l *= alpha;
#pragma unroll
    for (int d = 0; d < HD; ++d) o[d] *= alpha;
#pragma unroll
    for (int j = 0; j < kBN; ++j) {
      const float pj = fast_exp2(s[j] - mu);
      l += pj;
#pragma unroll
      for (int d = 0; d < HD; ++d) o[d] = fmaf(pj, Vs[j][d], o[d]);
    }
    m = mn;
  }

  if (row_ok) {
    T* op = static_cast<T*>(p.out) + sv.o_off + (int64_t)row * p.o_token_stride;
#pragma unroll
    for (int d = 0; d < HD; ++d) Elem<T>::store1(op + d, l > 0.f ? o[d] / l : 0.f);
  }
}

template <typename T, int HD>
hipError_t launch_typed(const FwdArgs& a, hipStream_t stream) {
  const asrattn_fwd_params& p = a.p;
  dim3 grid((p.max_len_q + kRows - 1) / kRows, p.heads_q, p.batch);
  hipLaunchKernelGGL((fwd_valu_kernel<T, HD>), grid, dim3(kRows), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

bool fwd_valu_supported(int dtype, int head_dim) {
  return (dtype == ASRATTN_F32 || dtype == ASRATTN_BF16) && (head_dim == 64 || head_dim == 128);
}

hipError_t launch_fwd_valu(const asrattn_fwd_params& p, hipStream_t stream) {
  FwdArgs a;
  a.p = p;
  a.c = p.scale * kLog2e;
  if (p.dtype == ASRATTN_BF16) {
    return p.head_dim == 64 ? launch_typed<bf16_raw, 64>(a, stream) : launch_typed<bf16_raw, 128>(a, stream);
  }
  return p.head_dim == 64 ? launch_typed<float, 64>(a, stream) : launch_typed<float, 128>(a, stream);
}

}  // namespace asrattn
