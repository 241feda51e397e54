// Multi-row attention in fp32 on the gfx950 matrix cores
// (v_mfma_f32_32x32x2_f32: fp32 operands, fp32 accumulation).
//
// Workgroup: KS waves over one block of 32 query rows of one (sequence,
// head); wave ks takes the key sub-tiles ks, ks + KS, ... (32 keys each) and
// the waves merge their (O, max, sum) through LDS at the end.  The products
// are the transposed ones of the bf16 kernel, so a query row's scores and
// output stay in its lanes:
//
//   S^T = K . Q^T    A = 32 keys x 2 head dims per step, B = Q^T (registers).
//   O^T = V^T . P^T  A = 32 head dims x 2 keys per step, B = P^T straight from
//                    the S^T accumulators.
//
// The k slots of a step are summed in any order, so the head dimensions (for
// S^T) and keys (for O^T) are assigned to (step t, half h = lane / 32) as
// 8 (t / 4) + 4 h + t % 4: then the accumulator register r of S^T holds key
// 8 (r / 4) + 4 h + r % 4 of the sub-tile, which is exactly what step r of
// O^T needs from that lane, and a lane's K operands for four consecutive
// steps are one 16-byte load.
//
// At fp32 a product step moves 256 bytes of operands per 64 matrix cycles,
// so the operands come straight from memory (L2: a head's K/V are shared by
// all its row blocks) into registers, one sub-tile ahead of the products --
// no LDS in the main loop and no barriers.  K rows are 16-byte loads; V^T
// operands are 4-byte loads (lanes 0..31 read 128 contiguous bytes of one
// key row, lanes 32..63 of another).  Buffer resources end at the block's
// last visible key, so loads past it return zeros without a branch.
//
// Softmax in base 2 with scale * log2(e) folded into one FMA per score; the
// running max is lazy as in the bf16 kernel (rescale only when a row's max
// grows by more than 2^8).
#include "common.hpp"
#include "fwd_common.hpp"
#include "kernels.hpp"
#include "ring_common.hpp"

namespace asrattn {
namespace {

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x16_t mfma_f32(float a, float b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4_t load4(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset) {
  return __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rsrc, voffset, 0, 0));
}

__device__ __forceinline__ float load1(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, voffset, 0, 0));
}

template <int HD>
struct F32Shape {
  static constexpr int kSteps = HD / 2;    // product steps of S^T over the head dimensions
  static constexpr int kQ4 = HD / 8;       // 16-byte K (and Q) loads per lane per sub-tile
  static constexpr int kDB = HD / 32;      // 32-row blocks of O^T
  static constexpr int kV = 16 * kDB;      // 4-byte V loads per lane per sub-tile
};

// One sub-tile's operands in registers.
template <int HD>
struct Operands {
  f32x4_t k[F32Shape<HD>::kQ4];
  float v[F32Shape<HD>::kV];
};

template <int HD, int KS, int OCC>
__global__ __launch_bounds__(64 * KS, OCC) void fwd_f32mm_kernel(const FwdArgs a, int q_tiles, int total) {
  using S = F32Shape<HD>;
  constexpr int NQ = S::kQ4, DB = S::kDB;
  const asrattn_fwd_params& p = a.p;
  // Each XCD takes a contiguous range of (sequence, head, row block) items,
  // so a head's keys and values stay in that XCD's L2 for all its row blocks.
  const int item = ring::xcd_remap((int)blockIdx.x, total);
  const int qt = item % q_tiles;
  const int hq = (item / q_tiles) % p.heads_q;
  const int b = item / q_tiles / p.heads_q;
  const int hkv = hq / (p.heads_q / p.heads_kv);
  const SeqView sv = seq_view(p, b, hq, hkv);
  const int row0 = qt * 32;
  if (row0 >= sv.len_q) return;  // uniform over the workgroup
  const int len_c = (p.flags & ASRATTN_FWD_ZERO_PADDED_ROWS) != 0 ? min(sv.len_q, sv.n_k) : sv.len_q;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int ks = tid >> 6;
  const int r32 = lane & 31;
  const int half = lane >> 5;
  if (row0 >= len_c) {
    // Rows at or past the key count of a zero-padded batch: zeros.
    for (int i = tid; i < (min(row0 + 32, sv.len_q) - row0) * (HD / 4); i += 64 * KS) {
      float* op = static_cast<float*>(p.out) + sv.o_off + (int64_t)(row0 + i / (HD / 4)) * p.o_token_stride +
                  (i % (HD / 4)) * 4;
      *reinterpret_cast<float4*>(op) = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    return;
  }
  const int row = row0 + r32;
  const bool row_ok = row < len_c;
  const int row_lim = row_ok ? visible_keys(p, sv, row) : 0;  // keys [0, row_lim) of this row
  const int kend = visible_keys(p, sv, min(row0 + 32, len_c) - 1);
  const int n_sub = (kend + 31) / 32;

  // Q^T operand: step t takes head dimension 8 (t / 4) + 4 half + t % 4 of the row.
  float qreg[S::kSteps];
  {
    const float* qp = static_cast<const float*>(p.q) + sv.q_off + (int64_t)(row_ok ? row : 0) * p.q_token_stride +
                      4 * half;
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      const float4 v = row_ok ? *reinterpret_cast<const float4*>(qp + 8 * j) : make_float4(0.f, 0.f, 0.f, 0.f);
      qreg[4 * j] = v.x;
      qreg[4 * j + 1] = v.y;
      qreg[4 * j + 2] = v.z;
      qreg[4 * j + 3] = v.w;
    }
  }

  const uint32_t kts = (uint32_t)p.k_token_stride * 4;
  const uint32_t vts = (uint32_t)p.v_token_stride * 4;
  const __amdgpu_buffer_rsrc_t krs =
      buffer_rsrc(static_cast<const float*>(p.k) + sv.k_off, (uint32_t)kend * kts);
  const __amdgpu_buffer_rsrc_t vrs =
      buffer_rsrc(static_cast<const float*>(p.v) + sv.v_off, (uint32_t)kend * vts);
  // Lane offsets inside a sub-tile: K row r32 at head dimensions 8 j + 4 half;
  // V^T row (head dimension) 32 db + r32 of key 8 (t / 4) + 4 half + t % 4.
  const uint32_t koff = (uint32_t)r32 * kts + (uint32_t)half * 16;
  const uint32_t voff = (uint32_t)(4 * half) * vts + (uint32_t)r32 * 4;

  auto load = [&](Operands<HD>& o, int sub) {
    const uint32_t kb = (uint32_t)(sub * 32) * kts + koff;
    const uint32_t vb = (uint32_t)(sub * 32) * vts + voff;
#pragma unroll
    for (int j = 0; j < NQ; ++j) o.k[j] = load4(krs, kb + (uint32_t)j * 32);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int t = 0; t < 16; ++t)
        o.v[16 * db + t] = load1(vrs, vb + (uint32_t)(8 * (t / 4) + t % 4) * vts + (uint32_t)db * 128);
  };

  f32x16_t oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db] = f32x16_t{};
  const float c = a.c;
  constexpr float kLazy = 8.f;
  float m_run = kNegInf;
  float l_run = 0.f;

  auto tile = [&](const Operands<HD>& o, int sub) {
    f32x16_t s = f32x16_t{};
#pragma unroll
    for (int t = 0; t < S::kSteps; ++t) s = mfma_f32(o.k[t / 4][t % 4], qreg[t], s);
    // Keys past the row's limit -> -inf (register r: key 32 sub + 8 (r / 4) + 4 half + r % 4).
    const int kt = sub * 32;
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (kt + 8 * (r / 4) + 4 * half + r % 4 >= row_lim) s[r] = kNegInf;
    float mt = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mt = fmaxf(mt, s[r]);
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
    mt = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * c;
    if (__any(mt > m_run + kLazy)) {
      const float mn = fmaxf(m_run, mt);
      const float alpha = mn == kNegInf ? 1.f : fast_exp2(m_run - mn);
#pragma unroll
      for (int db = 0; db < DB; ++db) oacc[db] *= alpha;
      l_run *= alpha;
      m_run = mn;
    }
    const float mu = m_run == kNegInf ? 0.f : m_run;
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = fast_exp2(fmaf(s[r], c, -mu));
      ps += s[r];
    }
    l_run += ps;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int t = 0; t < 16; ++t) oacc[db] = mfma_f32(o.v[16 * db + t], s[t], oacc[db]);
  };

  // This wave's sub-tiles ks, ks + KS, ... in register ping-pong: the next
  // sub-tile's operands load while the current one computes.
  // The loads are unconditional (past the block's last key they read zeros
  // and are never used): a load under a branch makes the compiler drain
  // every load at the join, the prefetch included.
  Operands<HD> opa, opb;
  load(opa, ks);
  for (int sub = ks; sub < n_sub; sub += 2 * KS) {
    load(opb, sub + KS);
    tile(opa, sub);
    if (sub + KS >= n_sub) break;
    load(opa, sub + 2 * KS);
    tile(opb, sub + KS);
  }

  // Merge the key splits through LDS: waves 1..KS-1 store (O^T, max, sum),
  // wave 0 folds them in and writes the rows.
  if constexpr (KS > 1) {
    constexpr int kPer = (16 * DB + 2) * 64;
    __shared__ float mf[(KS - 1) * kPer];
    if (ks > 0) {
      float* dst = mf + (ks - 1) * kPer + lane;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) dst[(16 * db + r) * 64] = oacc[db][r];
      dst[(16 * DB) * 64] = m_run;
      dst[(16 * DB + 1) * 64] = l_run;
    }
    __syncthreads();
    if (ks > 0) return;
#pragma unroll
    for (int s2 = 1; s2 < KS; ++s2) {
      const float* src = mf + (s2 - 1) * kPer + lane;
      const float m2 = src[(16 * DB) * 64];
      const float l2 = src[(16 * DB + 1) * 64];
      const float mn = fmaxf(m_run, m2);
      const float mu = mn == kNegInf ? 0.f : mn;
      const float w1 = fast_exp2(m_run - mu);
      const float w2 = fast_exp2(m2 - mu);
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[db][r] = oacc[db][r] * w1 + src[(16 * db + r) * 64] * w2;
      l_run = l_run * w1 + l2 * w2;
      m_run = mn;
    }
  }
  if (row >= sv.len_q) return;
  // The half waves hold disjoint keys of the same rows.
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = l_tot > 0.f && row_ok ? 1.f / l_tot : 0.f;  // rows past len_c get zeros
  float* op = static_cast<float*>(p.out) + sv.o_off + (int64_t)row * p.o_token_stride + 4 * half;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<float4*>(op + 32 * db + 8 * j) =
          make_float4(oacc[db][4 * j] * inv, oacc[db][4 * j + 1] * inv, oacc[db][4 * j + 2] * inv,
                      oacc[db][4 * j + 3] * inv);
}

template <int HD, int KS>
hipError_t launch_ks(const FwdArgs& a, hipStream_t stream) {
  const asrattn_fwd_params& p = a.p;
  const int q_tiles = (p.max_len_q + 31) / 32;
  const long long total = (long long)q_tiles * p.heads_q * p.batch;
  if (total > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  // Two waves per SIMD at head_dim 64 (about 240 VGPRs), one at 128.
  constexpr int OCC = HD == 64 ? 2 : 1;
  hipLaunchKernelGGL((fwd_f32mm_kernel<HD, KS, OCC>), dim3((unsigned)total), dim3(64 * KS), 0, stream, a, q_tiles,
                     (int)total);
  return hipGetLastError();
}

template <int HD>
hipError_t launch_hd(const FwdArgs& a, hipStream_t stream) {
  const asrattn_fwd_params& p = a.p;
  const long long blocks = (long long)((p.max_len_q + 31) / 32) * p.heads_q * p.batch;
  const int subs = (p.max_len_k + 31) / 32;
  // Key splits: as many waves per row block as the CUs hold at once for
  // all blocks (two per SIMD at head_dim 64; one at 128, where a wave needs
  // more than 256 registers), and at least two sub-tiles per split.  A
  // second round of workgroups would run on few CUs: Whisper-tiny's 282 row
  // blocks take four splits (1128 waves, one round) in 66 us and took 73.8
  // with eight (2256 waves, two rounds).
  constexpr int kMaxKs = HD == 64 ? 8 : 4;
  constexpr long long kResidentWaves = HD == 64 ? 2048 : 1024;
  int ks = 1;
  while (ks < kMaxKs && blocks * 2 * ks <= kResidentWaves && subs >= 4 * ks) ks *= 2;
  switch (ks) {
    case 1: return launch_ks<HD, 1>(a, stream);
    case 2: return launch_ks<HD, 2>(a, stream);
    case 4: return launch_ks<HD, 4>(a, stream);
    default:
      if constexpr (HD == 64) return launch_ks<HD, 8>(a, stream);
      return launch_ks<HD, 4>(a, stream);
  }
}

}  // namespace

bool fwd_f32mm_supported(const asrattn_fwd_params& p) {
  if (p.dtype != ASRATTN_F32 || p.window > 0) return false;
  if (p.head_dim != 64 && p.head_dim != 128) return false;
  // K/V addressed with 32-bit byte offsets from the sequence's first key, up
  // to the prefetch of two rounds of eight 32-key sub-tiles past the last.
  const long long span_k = ((long long)p.max_len_k + 16 * 32 + 32) * p.k_token_stride * 4;
  const long long span_v = ((long long)p.max_len_k + 16 * 32 + 32) * p.v_token_stride * 4;
  return span_k < (1LL << 31) && span_v < (1LL << 31) && p.k_token_stride >= p.head_dim &&
         p.v_token_stride >= p.head_dim;
}

hipError_t launch_fwd_f32mm(const asrattn_fwd_params& p, hipStream_t stream) {
  if (p.max_len_q > 0x7fffffff - 31) return hipErrorInvalidConfiguration;
  FwdArgs a;
  a.p = p;
  a.c = p.scale * kLog2e;
  a.f = FsmnArgs{};
  return p.head_dim == 64 ? launch_hd<64>(a, stream) : launch_hd<128>(a, stream);
}

}  // namespace asrattn
