// Multi-row attention on the vector ALUs, fp32 arithmetic throughout.
//
// One wave per workgroup.  A query row belongs to LPR lanes (one lane up to
// head_dim 128; head_dim / 128 lanes beyond, each holding 128 dimensions),
// which keep its scaled query and output accumulator in registers; the
// partial dot products of a row's lanes are summed with DPP.  Key/value
// tiles of BN rows are staged in LDS as fp32 and read by all lanes at the
// same address (broadcast, no bank conflicts).  This is the fp32 path
// (Whisper in float32, the reference's CPU/fp32 dtype; Gemma 4 in float32 at
// head_dim 256 and 512) and the exact-arithmetic twin of the bf16
// matrix-core kernel.
#include "common.hpp"
#include "fwd_common.hpp"
#include "kernels.hpp"

namespace asrattn {
namespace {

constexpr int kLanes = 64;  // one wave per workgroup

template <int HD>
struct ValuShape {
  static constexpr int kLPR = HD <= 128 ? 1 : HD / 128;  // lanes per query row
  static constexpr int kDPL = HD / kLPR;                  // dimensions per lane
  static constexpr int kRows = kLanes / kLPR;             // query rows per workgroup
  static constexpr int kBN = 32 * 128 / (HD > 128 ? HD : 128);  // keys per LDS tile (32 KB of K and V)
};

template <typename T, int HD>
__global__ __launch_bounds__(kLanes) void fwd_valu_kernel(const FwdArgs a) {
  using S = ValuShape<HD>;
  constexpr int EPV = Elem<T>::kPerVec, LPR = S::kLPR, DPL = S::kDPL, ROWS = S::kRows, BN = S::kBN;
  const asrattn_fwd_params& p = a.p;
  const int hq = blockIdx.y;
  const int b = blockIdx.z;
  const int hkv = hq / (p.heads_q / p.heads_kv);
  const SeqView sv = seq_view(p, b, hq, hkv);
  const int row0 = blockIdx.x * ROWS;
  if (row0 >= sv.len_q) return;  // uniform over the workgroup

  const int lane = threadIdx.x;
  const int sub = lane % LPR;  // this lane's dimensions: [sub * DPL, +DPL)
  const int row = row0 + lane / LPR;
  const bool row_ok = row < sv.len_q;
  const int row_lim = visible_keys(p, sv, row);
  const int row_lo = first_key(p, sv, row);
  const int last = min(row0 + ROWS, sv.len_q) - 1;
  const int kend = visible_keys(p, sv, last);
  const int kbeg = first_key(p, sv, row0) / BN * BN;

  float q[DPL], o[DPL];
  {
    const T* qp = static_cast<const T*>(p.q) + sv.q_off + (int64_t)(row_ok ? row : 0) * p.q_token_stride + sub * DPL;
#pragma unroll
    for (int d = 0; d < DPL; d += EPV) {
      float t[EPV];
      Elem<T>::load16(qp + d, t);
#pragma unroll
      for (int e = 0; e < EPV; ++e) q[d + e] = row_ok ? t[e] * a.c : 0.f;
    }
#pragma unroll
    for (int d = 0; d < DPL; ++d) o[d] = 0.f;
  }
  float m = kNegInf, l = 0.f;

  __shared__ float Ks[BN][HD];
  __shared__ float Vs[BN][HD];
  const T* kbase = static_cast<const T*>(p.k) + sv.k_off;
  const T* vbase = static_cast<const T*>(p.v) + sv.v_off;

  for (int kt = kbeg; kt < kend; kt += BN) {
    __syncthreads();
    constexpr int kVecs = BN * HD / EPV;
    for (int c = lane; c < kVecs; c += kLanes) {
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

    float s[BN];
    float mt = kNegInf;
#pragma unroll
    for (int j = 0; j < BN; ++j) {
      float acc = 0.f;
#pragma unroll
      for (int d = 0; d < DPL; ++d) acc = fmaf(q[d], Ks[j][sub * DPL + d], acc);
      acc = group_sum<LPR>(acc);
      s[j] = kt + j < row_lim && kt + j >= row_lo ? acc : kNegInf;
      mt = fmaxf(mt, s[j]);
    }
    const float mn = fmaxf(m, mt);
    const float mu = mn == kNegInf ? 0.f : mn;
    const float alpha = fast_exp2(m - mu);
    l *= alpha;
#pragma unroll
    for (int d = 0; d < DPL; ++d) o[d] *= alpha;
#pragma unroll
    for (int j = 0; j < BN; ++j) {
      const float pj = fast_exp2(s[j] - mu);
      l += pj;
#pragma unroll
      for (int d = 0; d < DPL; ++d) o[d] = fmaf(pj, Vs[j][sub * DPL + d], o[d]);
    }
    m = mn;
  }

  if (row_ok) {
    T* op = static_cast<T*>(p.out) + sv.o_off + (int64_t)row * p.o_token_stride + sub * DPL;
    // Zero-padded rows: a padded sequence's rows at or past its key count.
    const bool zero = (p.flags & ASRATTN_FWD_ZERO_PADDED_ROWS) != 0 && row >= sv.n_k;
#pragma unroll
    for (int d = 0; d < DPL; ++d) Elem<T>::store1(op + d, l > 0.f && !zero ? o[d] / l : 0.f);
  }
}

template <typename T, int HD>
hipError_t launch_typed(const FwdArgs& a, hipStream_t stream) {
  const asrattn_fwd_params& p = a.p;
  constexpr int ROWS = ValuShape<HD>::kRows;
  dim3 grid((p.max_len_q + ROWS - 1) / ROWS, p.heads_q, p.batch);
  hipLaunchKernelGGL((fwd_valu_kernel<T, HD>), grid, dim3(kLanes), 0, stream, a);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_dtype(const FwdArgs& a, hipStream_t stream) {
  switch (a.p.head_dim) {
    case 64: return launch_typed<T, 64>(a, stream);
    case 128: return launch_typed<T, 128>(a, stream);
    case 256: return launch_typed<T, 256>(a, stream);
    case 512: return launch_typed<T, 512>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool fwd_valu_supported(int dtype, int head_dim) {
  return (dtype == ASRATTN_F32 || dtype == ASRATTN_BF16) &&
         (head_dim == 64 || head_dim == 128 || head_dim == 256 || head_dim == 512);
}

hipError_t launch_fwd_valu(const asrattn_fwd_params& p, hipStream_t stream) {
  FwdArgs a;
  a.p = p;
  a.c = p.scale * kLog2e;
  return p.dtype == ASRATTN_BF16 ? launch_dtype<bf16_raw>(a, stream) : launch_dtype<float>(a, stream);
}

}  // namespace asrattn
