// Multi-row attention on the gfx950 matrix cores, bf16 operands with fp32
// accumulation (v_mfma_f32_32x32x16_bf16).
//
// Workgroup: RB x KS waves.  Each wave owns 32 query rows (row block rb) and
// one key split ks: the workgroup covers BM = 32 * RB rows of one (sequence,
// head), and its KS key splits walk interleaved BN-key tiles of the same
// keys.  Splitting keys across waves multiplies the waves per SIMD on short
// sequences (SenseVoice rows are 104-504 long) without shrinking the MFMA
// tiles; the splits merge through LDS at the end.
//
// The kernel computes the transposed products, so that everything a query
// row needs sits in one lane:
//
//   S^T = K . Q^T   A = K tile (LDS, row-major), B = Q^T (registers, loaded
//                   once).  The 32x32 result puts query row (lane % 32) in
//                   the lane and 16 keys in its accumulators; the two half
//                   waves hold disjoint key subsets of the same rows.
//   O^T = V^T . P^T A = V^T read from the row-major V tile with the gfx950
//                   transpose load (ds_read_b64_tr_b16), B = P^T taken
//                   straight from the S^T accumulators: the MFMA sums over
//                   its 16 k slots in any order, so the key order of the
//                   accumulator layout is used for both operands and P never
//                   moves between lanes.
//
// Row max and row sum are lane-local apart from one exchange between the
// half waves per tile (max) and one at the end (sum); the output rescale is
// lane-local too.  Softmax runs in base 2 with scale * log2(e) folded into
// one FMA per score.
//
// LDS rows are padded so that the MFMA operand reads spread over the banks:
// K rows by 16 bytes (consecutive rows of a b128 read land 16 bytes apart),
// V rows by 64 bytes (the 4-row groups of a transpose read land 64 bytes
// apart).
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
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) short4_t* lds_short4_ptr;

__device__ __forceinline__ f32x16_t mfma32(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Transpose load of 4 bf16: within each 16-lane group, lane j receives
// element (j % 4) of the 8-byte chunks addressed by lanes 4k + j / 4,
// k = 0..3.
__device__ __forceinline__ short4_t ds_read_tr(const bf16_raw* lds) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_ptr)(lds));
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

template <int HD, int RB, int KS, int BN>
struct MfmaShape {
  static constexpr int kBN = BN;                     // keys per tile (per key split)
  static constexpr int kKB = BN / 32;                // 32-key blocks per tile
  static constexpr int kWaves = RB * KS;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kBM = 32 * RB;
  static constexpr int kKSteps = HD / 16;            // k-steps of S^T
  static constexpr int kDB = HD / 32;                // 32-row blocks of O^T
  static constexpr int kKRow = HD + 8;               // LDS row stride of K (elements)
  static constexpr int kVRow = HD + 32;              // LDS row stride of V (elements)
  static constexpr int kKTile = BN * kKRow;          // elements per K tile
  static constexpr int kVTile = BN * kVRow;
  static constexpr int kCPR = HD / 8;                // 16-byte chunks per row
  static constexpr int kChunks = KS * BN * kCPR / kThreads;  // per thread, per K or V
  static constexpr int kMerge = RB * (KS - 1) * ((HD / 32) * 16 + 2) * 64 * 4;  // bytes
  static constexpr int kTiles = KS * (kKTile + kVTile) * 2;  // bytes
  static constexpr int kLds = kTiles > kMerge ? kTiles : kMerge;
  static_assert(KS * BN * kCPR % kThreads == 0, "tile / workgroup mapping");
  static_assert(BN == 32 || BN == 64, "tile");
};

template <int HD, int RB, int KS, int BN>
__global__ __launch_bounds__(64 * RB * KS, 2) void fwd_mfma_kernel(const FwdArgs a, int q_tiles, int total) {
  using S = MfmaShape<HD, RB, KS, BN>;
  constexpr int BM = S::kBM, NT = S::kThreads, KST = S::kKSteps, DB = S::kDB, KB = S::kKB;
  constexpr int KROW = S::kKRow, VROW = S::kVRow, CPR = S::kCPR, CH = S::kChunks;
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
  const int rb = wave % RB;
  const int ks = wave / RB;
  const int r32 = lane & 31;
  const int half = lane >> 5;
  const int row = row0 + rb * 32 + r32;
  const bool row_ok = row < sv.len_q;
  const int row_lim = visible_keys(p, sv, row);
  const int kend = visible_keys(p, sv, min(row0 + BM, sv.len_q) - 1);

  __shared__ __attribute__((aligned(16))) bf16_raw lds[S::kLds / 2];
  bf16_raw* const Ks = lds;                       // [KS][BN][KROW]
  bf16_raw* const Vs = lds + KS * S::kKTile;      // [KS][BN][VROW]

  // Q^T operand: lane (row, half) holds head_dim [16 kk + 8 half, +8).
  bf16x8_t qreg[KST];
  {
    const bf16_raw* qp = static_cast<const bf16_raw*>(p.q) + sv.q_off +
                         (int64_t)(row_ok ? row : 0) * p.q_token_stride + half * 8;
#pragma unroll
    for (int kk = 0; kk < KST; ++kk) {
      uint4 v = row_ok ? *reinterpret_cast<const uint4*>(qp + kk * 16) : make_uint4(0, 0, 0, 0);
      qreg[kk] = __builtin_bit_cast(bf16x8_t, v);
    }
  }

  f32x16_t oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db] = f32x16_t{};
  float m_run = kNegInf;
  float l_run = 0.f;

  const bf16_raw* kbase = static_cast<const bf16_raw*>(p.k) + sv.k_off;
  const bf16_raw* vbase = static_cast<const bf16_raw*>(p.v) + sv.v_off;

  // Transpose-load addressing of V^T (see ds_read_tr): lane (group g, i)
  // points at key row 4 (g / 2) + i / 4 and column 16 (g % 2) + 4 (i % 4) of
  // each 8-key x 32-column block.
  const int tr_row = 4 * ((lane >> 4) >> 1) + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const bf16_raw* const Kw = Ks + ks * S::kKTile;
  const bf16_raw* const Vw = Vs + ks * S::kVTile + tr_row * VROW + tr_col;

  const float c = a.c;
  // Global -> register staging: chunk ch = tid + i * NT is row ch / CPR of
  // the KS tiles (split row / BN), columns (ch % CPR) * 8.  Rows past kend
  // read the last visible row (in bounds) and are zeroed.
  uint4 kreg[CH], vreg[CH];
  auto load_tiles = [&](int kt0) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int ch = tid + i * NT;
      const int key = kt0 + ch / CPR;
      const int col = (ch % CPR) * 8;
      const bool in = key < kend;
      const int64_t safe = in ? key : kend - 1;
      const uint4 kv = *reinterpret_cast<const uint4*>(kbase + safe * p.k_token_stride + col);
      const uint4 vv = *reinterpret_cast<const uint4*>(vbase + safe * p.v_token_stride + col);
      kreg[i] = in ? kv : make_uint4(0, 0, 0, 0);
      vreg[i] = in ? vv : make_uint4(0, 0, 0, 0);
    }
  };
  if (kend > 0) load_tiles(0);
  for (int kt0 = 0; kt0 < kend; kt0 += KS * BN) {
    __syncthreads();  // the previous tiles are no longer read
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int ch = tid + i * NT;
      const int r = ch / CPR;  // 0 .. KS * BN - 1
      const int col = (ch % CPR) * 8;
      const int split = r / BN;
      const int lr = r % BN;
      *reinterpret_cast<uint4*>(&Ks[split * S::kKTile + lr * KROW + col]) = kreg[i];
      *reinterpret_cast<uint4*>(&Vs[split * S::kVTile + lr * VROW + col]) = vreg[i];
    }
    __syncthreads();
    // The next tiles load while this one is computed.
    if (kt0 + KS * BN < kend) load_tiles(kt0 + KS * BN);

    const int kt = kt0 + ks * BN;  // this wave's tile
    if (kt >= kend) continue;      // uniform per wave; barriers are above

    // S^T for the tile's 32-key blocks: the K operands of a block are read
    // ahead of its MFMA chain, and the blocks' chains interleave.
    f32x16_t sacc[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) sacc[kb] = f32x16_t{};
#pragma unroll
    for (int kk = 0; kk < KST; ++kk) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const bf16x8_t av = *reinterpret_cast<const bf16x8_t*>(Kw + (kb * 32 + r32) * KROW + half * 8 + kk * 16);
        sacc[kb] = mfma32(av, qreg[kk], sacc[kb]);
      }
    }

    // Accumulator r of block kb is key kt + 32 kb + 8 (r / 4) + 4 half + r % 4.
    if (kt + BN > row_lim) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kt + kb * 32 + (r / 4) * 8 + half * 4 + (r % 4);
          if (key >= row_lim) sacc[kb][r] = kNegInf;
        }
    }

    float mt = kNegInf;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sacc[kb][r]);
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float mn = fmaxf(m_run, mt * c);
    const float mu = mn == kNegInf ? 0.f : mn;
    // Rescale only when some row's running max moved (rare after the first
    // tiles); the test is uniform over the wave.
    const bool moved = mn != m_run;
    const float alpha = fast_exp2(m_run - mu);
    m_run = mn;

    float psum = 0.f;
    bf16x8_t pb[2 * KB];
#pragma unroll
    for (int t = 0; t < 2 * KB; ++t) {
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
    if (__any(moved)) {
#pragma unroll
      for (int db = 0; db < DB; ++db) oacc[db] *= alpha;
    }

    // O^T += V^T . P^T.  MFMA t covers keys 16 t + 8 (idx / 4) + 4 half + idx % 4.
#pragma unroll
    for (int t = 0; t < 2 * KB; ++t) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const bf16_raw* vr = Vw + (16 * t) * VROW + 32 * db;
        const short4_t lo = ds_read_tr(vr);
        const short4_t hi = ds_read_tr(vr + 8 * VROW);
        const bf16x8_t av = __builtin_bit_cast(
            bf16x8_t, (short __attribute__((ext_vector_type(8)))){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
        oacc[db] = mfma32(av, pb[t], oacc[db]);
      }
    }
  }

  // Merge the key splits of each row block through LDS (the tiles are done).
  // Afterwards wave (rb, 0) stages its output rows in LDS: in the first merge
  // slot of its row block (which only it reads) when the keys were split,
  // else in a region of the tile buffer once every wave is past its tiles.
  bf16_raw* stage;
  constexpr int ORS = HD + 8;  // staged output row stride (elements)
  if constexpr (KS > 1) {
    float* const mf = reinterpret_cast<float*>(lds);
    // Split ks > 0 of row block rb: [rb][ks-1][DB*16 + 2][64 lanes] floats.
    constexpr int kPer = (DB * 16 + 2) * 64;
    static_assert(32 * ORS * 2 <= kPer * 4, "output staging fits a merge slot");
    __syncthreads();
    if (ks > 0) {
      float* dst = mf + (rb * (KS - 1) + (ks - 1)) * kPer + lane;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) dst[(db * 16 + r) * 64] = oacc[db][r];
      dst[(DB * 16) * 64] = m_run;
      dst[(DB * 16 + 1) * 64] = l_run;
    }
    __syncthreads();
    if (ks > 0) return;
#pragma unroll
    for (int s2 = 1; s2 < KS; ++s2) {
      const float* src = mf + (rb * (KS - 1) + (s2 - 1)) * kPer + lane;
      const float m2 = src[(DB * 16) * 64];
      const float l2 = src[(DB * 16 + 1) * 64];
      const float mn = fmaxf(m_run, m2);
      const float mu = mn == kNegInf ? 0.f : mn;
      const float w1 = fast_exp2(m_run - mu);
      const float w2 = fast_exp2(m2 - mu);
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[db][r] = oacc[db][r] * w1 + src[(db * 16 + r) * 64] * w2;
      l_run = l_run * w1 + l2 * w2;
      m_run = mn;
    }
    stage = reinterpret_cast<bf16_raw*>(mf + rb * (KS - 1) * kPer);
  } else {
    static_assert(KS > 1 || RB * 32 * ORS * 2 <= S::kLds, "output staging fits the tiles");
    __syncthreads();
    stage = lds + rb * 32 * ORS;
  }

  // The half waves hold disjoint keys of the same rows.
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  // Accumulator r of block db is column 32 db + 8 (r / 4) + 4 half + r % 4
  // of row r32: write the normalized rows to LDS ...
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t w0 = pack_bf16x2(oacc[db][4 * i] * inv, oacc[db][4 * i + 1] * inv);
      const uint32_t w1 = pack_bf16x2(oacc[db][4 * i + 2] * inv, oacc[db][4 * i + 3] * inv);
      *reinterpret_cast<uint2*>(stage + r32 * ORS + db * 32 + i * 8 + half * 4) = make_uint2(w0, w1);
    }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // ... and store them to global memory 16 bytes per lane, whole rows per
  // instruction.
  constexpr int kRowChunks = HD / 8;
#pragma unroll
  for (int i = 0; i < 32 * kRowChunks / 64; ++i) {
    const int ch = i * 64 + lane;
    const int r = ch / kRowChunks;
    const int col = (ch % kRowChunks) * 8;
    const int orow = row0 + rb * 32 + r;
    const uint4 val = *reinterpret_cast<const uint4*>(stage + r * ORS + col);
    if (orow < sv.len_q) {
      bf16_raw* op = static_cast<bf16_raw*>(p.out) + sv.o_off + (int64_t)orow * p.o_token_stride + col;
      *reinterpret_cast<uint4*>(op) = val;
    }
  }
}

template <int HD, int RB, int KS, int BN>
hipError_t launch_typed(const FwdArgs& a, hipStream_t stream) {
  using S = MfmaShape<HD, RB, KS, BN>;
  static_assert(S::kLds <= 160 * 1024, "LDS");
  const asrattn_fwd_params& p = a.p;
  const int q_tiles = (p.max_len_q + S::kBM - 1) / S::kBM;
  const long long total = (long long)q_tiles * p.heads_q * p.batch;
  if (total <= 0) return hipSuccess;
  if (total > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((fwd_mfma_kernel<HD, RB, KS, BN>), dim3((unsigned)total), dim3(S::kThreads), 0, stream, a,
                     q_tiles, (int)total);
  return hipGetLastError();
}

template <int HD>
hipError_t launch_hd(const FwdArgs& a, hipStream_t stream) {
  const asrattn_fwd_params& p = a.p;
  // Waves a launch would have with 128-row workgroups; below ~4 per SIMD the
  // keys are split across waves instead, trading query rows per workgroup
  // for more waves.
  const long long tiles128 = (long long)((p.max_len_q + 127) / 128) * p.heads_q * p.batch;
  // Head dim 128 uses 32-key tiles when the keys are split, so that the
  // prefetched tiles fit in registers beside two waves per SIMD.
  constexpr int kSplitBN = HD == 128 ? 32 : 64;
  if (tiles128 >= 1024) return launch_typed<HD, 4, 1, 64>(a, stream);
  const long long tiles64 = (long long)((p.max_len_q + 63) / 64) * p.heads_q * p.batch;
  if (tiles64 >= 256) return launch_typed<HD, 2, 2, kSplitBN>(a, stream);
  return launch_typed<HD, 1, 4, kSplitBN>(a, stream);
}

}  // namespace

bool fwd_mfma_supported(int dtype, int head_dim) {
  return dtype == ASRATTN_BF16 && (head_dim == 64 || head_dim == 128);
}

hipError_t launch_fwd_mfma(const asrattn_fwd_params& p, hipStream_t stream) {
  FwdArgs a;
  a.p = p;
  a.c = p.scale * kLog2e;
  return p.head_dim == 64 ? launch_hd<64>(a, stream) : launch_hd<128>(a, stream);
}

}  // namespace asrattn
