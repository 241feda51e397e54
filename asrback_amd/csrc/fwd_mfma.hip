// Multi-row attention on the gfx950 matrix cores, bf16 operands with fp32
// accumulation (v_mfma_f32_32x32x16_bf16).
//
// Workgroup: NW waves, BM = 32 * NW query rows of one (sequence, head); each
// wave owns 32 rows.  Keys are processed in tiles of BN = 64.
//
// The kernel computes the transposed products, so that everything a query
// row needs sits in one lane:
//
//   S^T = K . Q^T   A = K tile (LDS, row-major), B = Q^T (registers, loaded
//                   once).  The 32x32 result puts query row (lane % 32) in
//                   the lane and 16 keys in its accumulators; the two half
//                   waves hold disjoint key subsets of the same rows.
//   O^T = V^T . P^T A = V^T (LDS, stored transposed), B = P^T taken straight
//                   from the S^T accumulators: the MFMA sums over its 16 k
//                   slots in any order, so the key order of the accumulator
//                   layout is used for both operands and P never moves.
//
// Row max and row sum are lane-local apart from one exchange between the
// half waves per tile (max) and one at the end (sum); the output rescale is
// lane-local too.  Softmax runs in base 2 with scale * log2(e) folded into
// one FMA per score.
//
// Pipeline: the next K/V tile is loaded from global memory into registers
// while the current tile is computed, then written to LDS (V transposed on
// the way: each thread packs VK keys of one head_dim column).
//
// Work mapping: a flat grid of (sequence, head, query tile) items; item ids
// are remapped so that the items dispatched to one XCD (ids i, i+8, ...) are
// consecutive, which keeps the query tiles of one (sequence, kv head) on one
// XCD and its K/V in that XCD's L2.
#include "common.hpp"
#include "fwd_common.hpp"
#include "kernels.hpp"

namespace asrattn {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBN = 64;

__device__ __forceinline__ f32x16_t mfma32(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Id -> work item such that the ids one XCD receives (round-robin dispatch
// over 8 XCDs) map to a contiguous range of items.
__device__ __forceinline__ int xcd_remap(int id, int total) {
  const int per = total / 8;
  const int rem = total % 8;
  const int x = id % 8;
  const int k = id / 8;
  return x * per + min(x, rem) + k;
}

template <int HD, int NW>
struct MfmaShape {
  static constexpr int kBM = 32 * NW;
  static constexpr int kThreads = 64 * NW;
  static constexpr int kKS = HD / 16;                 // k-steps of S^T
  static constexpr int kDB = HD / 32;                 // 32-row blocks of O^T
  static constexpr int kKRow = HD + 8;                // LDS row stride of K (elements)
  static constexpr int kVRow = kBN + 8;               // LDS row stride of V^T (elements)
  static constexpr int kChunks = kBN * HD / 8 / kThreads;  // 16-byte K loads per thread
  static constexpr int kVK = kChunks;                 // keys per thread in the V transpose
  static_assert(kChunks >= 1, "tile too small for the workgroup");
  static_assert(kBN % kVK == 0, "V transpose mapping");
};

template <int HD, int NW>
__global__ __launch_bounds__(64 * NW, 2) void fwd_mfma_kernel(const FwdArgs a, int q_tiles, int total) {
  using S = MfmaShape<HD, NW>;
  constexpr int BM = S::kBM, NT = S::kThreads, KS = S::kKS, DB = S::kDB;
  constexpr int KROW = S::kKRow, VROW = S::kVRow, CH = S::kChunks, VK = S::kVK;
  const asrattn_fwd_params& p = a.p;

  const int item = xcd_remap(blockIdx.x, total);
  const int qt = item % q_tiles;
  const int bh = item / q_tiles;
  const int hq = bh % p.heads_q;
  const int b = bh / p.heads_q;
  const int hkv = hq / (p.heads_q / p.heads_kv);
  const SeqView sv = seq_view(p, b, hq, hkv);
  const int row0 = qt * BM;
  if (row0 >= sv.len_q) return;  // uniform over the workgroup

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r32 = lane & 31;
  const int half = lane >> 5;
  const int row = row0 + wave * 32 + r32;
  const bool row_ok = row < sv.len_q;
  const int row_lim = visible_keys(p, sv, row);
  const int kend = visible_keys(p, sv, min(row0 + BM, sv.len_q) - 1);

  __shared__ __attribute__((aligned(16))) bf16_raw Ks[kBN * KROW];
  __shared__ __attribute__((aligned(16))) bf16_raw Vt[HD * VROW];

  // Q^T operand: lane (row, half) holds head_dim [16 ks + 8 half, +8).
  bf16x8_t qreg[KS];
  {
    const bf16_raw* qp = static_cast<const bf16_raw*>(p.q) + sv.q_off +
                         (int64_t)(row_ok ? row : 0) * p.q_token_stride + half * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      uint4 v = row_ok ? *reinterpret_cast<const uint4*>(qp + ks * 16) : make_uint4(0, 0, 0, 0);
      qreg[ks] = __builtin_bit_cast(bf16x8_t, v);
    }
  }

  f32x16_t oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db] = f32x16_t{};
  float m_run = kNegInf;
  float l_run = 0.f;

  const bf16_raw* kbase = static_cast<const bf16_raw*>(p.k) + sv.k_off;
  const bf16_raw* vbase = static_cast<const bf16_raw*>(p.v) + sv.v_off;

  // Global -> register staging.  K: chunk c = tid + i * NT is key c / (HD/8),
  // columns (c % (HD/8)) * 8.  V: thread covers keys [vkg * VK, +VK) of
  // columns [vcol, +8).
  const int vcol = (tid % (HD / 8)) * 8;
  const int vkg = tid / (HD / 8);
  uint4 kreg[CH];
  uint4 vreg[VK];
  auto load_tile = [&](int kt) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + i * NT;
      const int j = c / (HD / 8);
      const int col = (c % (HD / 8)) * 8;
      kreg[i] = kt + j < kend ? *reinterpret_cast<const uint4*>(kbase + (int64_t)(kt + j) * p.k_token_stride + col)
                              : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < VK; ++i) {
      const int j = vkg * VK + i;
      vreg[i] = kt + j < kend ? *reinterpret_cast<const uint4*>(vbase + (int64_t)(kt + j) * p.v_token_stride + vcol)
                              : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + i * NT;
      const int j = c / (HD / 8);
      const int col = (c % (HD / 8)) * 8;
      *reinterpret_cast<uint4*>(&Ks[j * KROW + col]) = kreg[i];
    }
    // Transpose: column (vcol + e) gets keys [vkg * VK, +VK) as VK packed bf16.
    const uint32_t* w = reinterpret_cast<const uint32_t*>(vreg);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      uint32_t packed[VK / 2 > 0 ? VK / 2 : 1];
#pragma unroll
      for (int i = 0; i < VK; i += 2) {
        const uint32_t x0 = w[i * 4 + e / 2];
        const uint32_t x1 = w[(i + 1) * 4 + e / 2];
        const uint32_t lo = (e & 1) ? (x0 >> 16) : (x0 & 0xffffu);
        const uint32_t hi = (e & 1) ? (x1 & 0xffff0000u) : (x1 << 16);
        packed[i / 2] = lo | hi;
      }
      bf16_raw* dst = &Vt[(vcol + e) * VROW + vkg * VK];
      if constexpr (VK == 2) {
        *reinterpret_cast<uint32_t*>(dst) = packed[0];
      } else if constexpr (VK == 4) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(packed[0], packed[1]);
      } else {
        static_assert(VK == 8, "VK");
        *reinterpret_cast<uint4*>(dst) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
      }
    }
  };

  const float c = a.c;
  if (kend > 0) load_tile(0);
  for (int kt = 0; kt < kend; kt += kBN) {
    __syncthreads();
    store_tile();
    __syncthreads();
    if (kt + kBN < kend) load_tile(kt + kBN);

    // S^T for two 32-key blocks.
    f32x16_t sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sacc[kb] = f32x16_t{};
      const bf16_raw* kr = &Ks[(kb * 32 + r32) * KROW + half * 8];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8_t av = *reinterpret_cast<const bf16x8_t*>(kr + ks * 16);
        sacc[kb] = mfma32(av, qreg[ks], sacc[kb]);
      }
    }

    // Accumulator r of block kb is key kt + 32 kb + 8 (r / 4) + 4 half + r % 4.
    const bool need_mask = kt + kBN > row_lim || kt + kBN > kend;
    if (need_mask) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kt + kb * 32 + (r / 4) * 8 + half * 4 + (r % 4);
          if (key >= row_lim) sacc[kb][r] = kNegInf;
        }
    }

    float mt = kNegInf;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sacc[kb][r]);
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float mn = fmaxf(m_run, mt * c);
    const float mu = mn == kNegInf ? 0.f : mn;
    const float alpha = fast_exp2(m_run - mu);
    m_run = mn;

    float psum = 0.f;
    bf16x8_t pb[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p0 = fast_exp2(fmaf(sacc[t / 2][(t % 2) * 8 + 2 * i], c, -mu));
        const float p1 = fast_exp2(fmaf(sacc[t / 2][(t % 2) * 8 + 2 * i + 1], c, -mu));
        psum += p0 + p1;
        w[i] = pack_bf16x2(p0, p1);
      }
      pb[t] = __builtin_bit_cast(bf16x8_t, make_uint4(w[0], w[1], w[2], w[3]));
    }
    l_run = fmaf(l_run, alpha, psum);
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[db] *= alpha;

    // O^T += V^T . P^T.  MFMA t covers keys 16 t + 8 (idx / 4) + 4 half + idx % 4.
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const bf16_raw* vr = &Vt[(db * 32 + r32) * VROW + 16 * t + 4 * half];
        const uint2 lo = *reinterpret_cast<const uint2*>(vr);
        const uint2 hi = *reinterpret_cast<const uint2*>(vr + 8);
        const bf16x8_t av = __builtin_bit_cast(bf16x8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
        oacc[db] = mfma32(av, pb[t], oacc[db]);
      }
    }
  }

  // The half waves hold disjoint keys of the same rows.
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (row_ok) {
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    bf16_raw* op = static_cast<bf16_raw*>(p.out) + sv.o_off + (int64_t)row * p.o_token_stride;
    // Accumulator r of block db is column 32 db + 8 (r / 4) + 4 half + r % 4.
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t w0 = pack_bf16x2(oacc[db][4 * i] * inv, oacc[db][4 * i + 1] * inv);
        const uint32_t w1 = pack_bf16x2(oacc[db][4 * i + 2] * inv, oacc[db][4 * i + 3] * inv);
        *reinterpret_cast<uint2*>(op + db * 32 + i * 8 + half * 4) = make_uint2(w0, w1);
      }
  }
}

template <int HD, int NW>
hipError_t launch_typed(const FwdArgs& a, hipStream_t stream) {
  const asrattn_fwd_params& p = a.p;
  constexpr int BM = MfmaShape<HD, NW>::kBM;
  const int q_tiles = (p.max_len_q + BM - 1) / BM;
  const long long total = (long long)q_tiles * p.heads_q * p.batch;
  if (total <= 0) return hipSuccess;
  if (total > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((fwd_mfma_kernel<HD, NW>), dim3((unsigned)total), dim3(64 * NW), 0, stream, a,
                     q_tiles, (int)total);
  return hipGetLastError();
}

}  // namespace

bool fwd_mfma_supported(int dtype, int head_dim) {
  return dtype == ASRATTN_BF16 && (head_dim == 64 || head_dim == 128);
}

hipError_t launch_fwd_mfma(const asrattn_fwd_params& p, hipStream_t stream) {
  FwdArgs a;
  a.p = p;
  a.c = p.scale * kLog2e;
  // Four waves (128 query rows) per workgroup when that still gives every
  // CU two workgroups; two waves (64 rows) otherwise.
  const long long tiles128 = (long long)((p.max_len_q + 127) / 128) * p.heads_q * p.batch;
  const bool wide = tiles128 >= 512;
  if (p.head_dim == 64) return wide ? launch_typed<64, 4>(a, stream) : launch_typed<64, 2>(a, stream);
  return wide ? launch_typed<128, 4>(a, stream) : launch_typed<128, 2>(a, stream);
}

}  // namespace asrattn
