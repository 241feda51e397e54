// SAN-M's FSMN memory as a kernel of its own: the fp32 path and the
// layouts the fused attention epilogue does not take.  One workgroup of 256
// threads per 128 rows of one (sequence, head).
#include "fsmn.hpp"
#include "kernels.hpp"

namespace asrattn {
namespace {

constexpr int kFsmnThreads = 256;
constexpr int kFsmnRows = 128;

template <typename T, int HD, int KW>
__global__ __launch_bounds__(kFsmnThreads) void fsmn_kernel(const asrattn_fwd_params p, const FsmnArgs f) {
  constexpr int RS = kFsmnRows * (HD / 4) / kFsmnThreads;
  const int row0 = blockIdx.x * kFsmnRows;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  int n = p.max_len_k;
  if (p.seqused_k != nullptr) n = min(n, max(p.seqused_k[b], 0));
  const T* v_seq = static_cast<const T*>(p.v) + (int64_t)b * p.v_batch_stride + (int64_t)h * p.v_head_stride;
  __shared__ __attribute__((aligned(16))) unsigned char lds[fsmn_lds_bytes<T, HD, KW>()];
  fsmn_rows<T, HD, KW, RS, kFsmnThreads>(f, v_seq, p.v_token_stride, b, h, row0, n, p.max_len_q, threadIdx.x, lds);
}

template <typename T, int HD>
hipError_t launch_hd(const asrattn_fwd_params& p, const FsmnArgs& f, hipStream_t stream) {
  const dim3 grid((unsigned)((p.max_len_q + kFsmnRows - 1) / kFsmnRows), (unsigned)p.heads_q, (unsigned)p.batch);
  if (f.kernel_size <= 11)
    hipLaunchKernelGGL((fsmn_kernel<T, HD, 11>), grid, dim3(kFsmnThreads), 0, stream, p, f);
  else
    hipLaunchKernelGGL((fsmn_kernel<T, HD, kFsmnMaxKernel>), grid, dim3(kFsmnThreads), 0, stream, p, f);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_typed(const asrattn_fwd_params& p, const FsmnArgs& f, hipStream_t stream) {
  return p.head_dim == 64 ? launch_hd<T, 64>(p, f, stream) : launch_hd<T, 128>(p, f, stream);
}

}  // namespace

hipError_t launch_fsmn(const asrattn_fwd_params& p, const FsmnArgs& f, hipStream_t stream) {
  if (p.batch == 0 || p.max_len_q == 0) return hipSuccess;
  return p.dtype == ASRATTN_BF16 ? launch_typed<bf16_raw>(p, f, stream) : launch_typed<float>(p, f, stream);
}

}  // namespace asrattn
