// Multi-row attention on the gfx950 matrix cores (bf16 operands, fp32
// accumulation, v_mfma_f32_32x32x16_bf16) with K/V tiles streamed into an LDS
// ring by DMA.
//
// Workgroup: W waves, each owning 32 query rows of one (sequence, head); the
// waves share BN-key K and V tiles.  Tiles move from HBM straight into LDS
// with buffer_load_dwordx4 ... lds (no register staging): ST ring stages keep
// ST - 1 tiles in flight, and one barrier per tile separates "stage landed
// for everyone" from "stage free for the next DMA".  The buffer resources end
// at the workgroup's last visible key, so DMA lanes past it write zeros and
// the last tile needs no guard.
//
// Per wave and tile the arithmetic is the transposed product, which keeps
// everything a query row needs in one lane:
//
//   S^T = K . Q^T   A = K rows (LDS), B = Q^T (registers, loaded once).  The
//                   32x32 result puts query row (lane % 32) in the lane and
//                   16 keys in its accumulators; the half waves hold disjoint
//                   keys of the same rows.
//   O^T = V^T . P^T A = V^T read from the row-major V tile with the gfx950
//                   transpose load (ds_read_b64_tr_b16), B = P^T taken
//                   straight from the S^T accumulators: the MFMA sums its 16
//                   k slots in any order, so one key order serves both
//                   operands and P never moves between lanes.
//
// Softmax runs in base 2 with scale * log2(e) folded into one FMA per score;
// the output is rescaled only when some row's running max moved by more
// than a slack (at head_dim 64 the row max itself is taken only when the
// tile's probabilities, summed, show that it may have).
//
// LDS layout: the DMA writes 64 consecutive 16-byte chunks per instruction,
// so rows cannot be padded; instead the chunk order inside each row is
// permuted (each lane fetches the global chunk that belongs in its slot):
//   K: chunk c of row r sits at (c + r) mod 16 (head_dim 128) or
//      (c + r / 2) mod 8 (head_dim 64), so the 16 rows one b128 operand read
//      touches per cycle hit 16 different bank groups;
//   V: chunk c of row r sits at c ^ 4 (r mod 4) (128) or c ^ 4 ((r / 2) mod 2)
//      (64), so the four rows of a transpose read land in four different
//      64-byte bank ranges.
//
// Workgroups may also split the keys across waves (KS splits, merged through
// LDS at the end), which shortens the longest workgroups of ragged batches.
//
// Work mapping: a flat grid of (sequence, head, query tile) items, taken
// longest-first in ragged batches, with the query tiles of one (sequence,
// head) -- and its K/V -- on one XCD's L2 (work_item).
//
// SAN-M's FSMN memory (fsmn.hpp) can ride along: the grid then holds a
// second copy of the items, each computing the memory of its row block.
// Dispatched after every attention item, they take the CUs that short
// sequences free while the longest ones finish; computed instead at the end
// of each attention item, the memory lengthened the longest items (and, with
// the tap-pair code, spilled).
#include "common.hpp"
#include "fwd_common.hpp"
#include "kernels.hpp"
#include "ring_common.hpp"

namespace asrattn {
namespace {

using namespace ring;

// Waits until at most `ahead` tiles' DMAs (PER instructions each) of this
// wave are outstanding.
template <int PER, int MAXAHEAD>
__device__ __forceinline__ void wait_dma(int ahead) {
  static_assert(MAXAHEAD <= 2, "ring depth");
  if (MAXAHEAD >= 2 && ahead >= 2) {
    wait_vmcnt<2 * PER>();
  } else if (MAXAHEAD >= 1 && ahead >= 1) {
    wait_vmcnt<PER>();
  } else {
    wait_vmcnt<0>();
  }
}

// Ranking costs every workgroup a round trip for all sequences' key
// counts before its own loads; it pays only when items differ by more than
// a couple of tiles (SenseVoice, up to 504 keys: 22.8 against 24.4 us
// unranked; Qwen3's audio windows of at most 104 keys: 11.9 against 10.5).
constexpr int kRankMinKeys = 128;

// Launch id -> (sequence, query head, query tile).  Dispatch hands ids out
// in order as workgroup slots free up, round-robin over the 8 XCDs.  With
// per-sequence key counts (ragged batches of at most 64 sequences, some
// longer than kRankMinKeys, none of 2^25 keys or more) the
// (sequence, kv head) units are taken in decreasing key count -- the
// longest work starts first and short units fill in behind it -- and unit U
// goes to XCD U % 8 with all its items consecutive there (every query head
// sharing the kv head, every query tile), so its K/V stay in one L2.  The
// second half of each XCD's items runs in increasing key count: when the
// grid fills two slots per CU, the longest items then share a CU with the
// shortest (3% on the SenseVoice batch).  Otherwise ids are remapped so that
// each XCD gets a contiguous range of items (the same L2 grouping).
__device__ __forceinline__ void work_item(const asrattn_fwd_params& p, int q_tiles, int total, int id, int& b,
                                          int& hq, int& qt) {
  const bool ragged = p.seqused_k != nullptr || p.cu_seqlens_k != nullptr;
  if (ragged && p.max_len_k > kRankMinKeys && p.max_len_k < (1 << 25) && p.batch <= 64 &&
      (p.batch * p.heads_kv) % 8 == 0) {
    const int group = p.heads_q / p.heads_kv;
    const int per_unit = group * q_tiles;
    const int per = total / 8, half = per / 2;
    int k = id >> 3;
    if (k >= half) k = per - 1 - (k - half);
    const int unit = (k / per_unit) * 8 + (id & 7);
    const int w = k % per_unit;
    qt = w % q_tiles;
    hq = (unit % p.heads_kv) * group + w / q_tiles;
    b = ranked_sequence(p, unit / p.heads_kv);
    return;
  }
  const int item = xcd_remap(id, total);
  qt = item % q_tiles;
  const int bh = item / q_tiles;
  hq = bh % p.heads_q;
  b = bh / p.heads_q;
}

// DS > 1 splits the head dimensions over DS waves per row block (head_dim
// 512, whose 32 rows of queries and outputs do not fit one wave's registers
// without spilling): each takes HD / DS dimensions of the queries, keys and
// outputs, the partial scores of a row block's waves are summed through LDS,
// and every one of them runs the same softmax.
template <int HD, int RB, int KS, int BN, int ST, int DS = 1>
struct RingShape {
  static constexpr int kW = RB * KS * DS;             // waves
  static constexpr int kBM = 32 * RB;                 // query rows per workgroup
  static constexpr int kThreads = 64 * kW;
  static constexpr int kSpan = KS * BN;               // keys per ring stage
  static constexpr int kKB = BN / 32;                 // 32-key blocks per sub-tile
  static constexpr int kDH = HD / DS;                 // head dimensions per wave
  static constexpr int kKSteps = kDH / 16;            // k-steps of S^T
  static constexpr int kDB = kDH / 32;                // 32-row blocks of O^T
  static constexpr int kRowBytes = HD * 2;
  static constexpr int kCPR = HD / 8;                 // 16-byte chunks per row
  static constexpr int kTileBytes = kSpan * kRowBytes;  // the K (or V) rows of a stage
  static constexpr int kStageBytes = 2 * kTileBytes;  // K rows, then V rows
  static constexpr int kDmaPerTile = kSpan * kCPR / 64;  // DMA instructions per K (or V) rows of a stage
  static constexpr int kDmaPerWave = kDmaPerTile / kW;
  static constexpr int kOutRow = HD + 8;              // staged output row stride (elements)
  static constexpr int kOutBytes = RB * 32 * kOutRow * 2;
  // Key-split merge: per (row block, split > 0) the wave's O^T accumulators
  // and (max, sum), lane-major floats.
  static constexpr int kMergeFloats = (kDB * 16 + 2) * 64;
  static constexpr int kMergeBytes = RB * (KS - 1) * kMergeFloats * 4;
  static constexpr int kRingBytes = ST * kStageBytes;
  // Partial scores of the dimension splits (lane-major, per wave), after
  // the ring.
  static constexpr int kPartialBytes = DS > 1 ? kW * kKB * 16 * 64 * 4 : 0;
  static constexpr int kEpilogue = KS > 1 ? kMergeBytes : kOutBytes;
  static constexpr int kMain = kRingBytes + kPartialBytes;
  static constexpr int kLds = kMain > kEpilogue ? kMain : kEpilogue;
  static_assert(HD == 64 || HD == 128 || HD == 256 || HD == 512, "head_dim");
  static_assert(BN % 32 == 0 && kDmaPerTile % kW == 0 && kDmaPerWave >= 1, "tile / workgroup mapping");
  static_assert(ST >= 2 && ST <= 4, "ring depth");
  static_assert(KS == 1 || 32 * kOutRow * 2 <= kMergeFloats * 4, "output staging fits a merge slot");
  static_assert(DS == 1 || (KS == 1 && kKSteps % 8 == 0), "dimension splits: one key split, whole 256-byte groups");
};

template <int HD, int RB, int KS, int BN, int ST, int OCC, int FS, bool WIN, int DS>
__global__ __launch_bounds__(64 * RB * KS * DS, OCC) void fwd_ring_kernel(const FwdArgs a, int q_tiles, int total) {
  using S = RingShape<HD, RB, KS, BN, ST, DS>;
  constexpr int DH = S::kDH;
  constexpr int BM = S::kBM, KST = S::kKSteps, DB = S::kDB, KB = S::kKB, RBYTES = S::kRowBytes;
  constexpr int CPR = S::kCPR, NPW = S::kDmaPerWave, SB = S::kStageBytes, TB = S::kTileBytes;
  constexpr int SPAN = S::kSpan;
  const asrattn_fwd_params& p = a.p;

  const int tid = threadIdx.x;
  __shared__ __attribute__((aligned(16))) unsigned char lds[S::kLds];

  // FSMN items (ids total .. 2 total - 1, same (sequence, head, row block)
  // and XCD as attention item id - total): the memory of the block's rows.
  // They are dispatched after every attention item and fill the CUs that
  // short sequences leave idle while the longest ones finish.
  if constexpr (FS > 0) {
    if ((int)blockIdx.x >= total) {
      int b, h, qt;
      work_item(p, q_tiles, total, (int)blockIdx.x - total, b, h, qt);
      const SeqView sv = seq_view(p, b, h, h);
      constexpr int NT = S::kThreads;
      static_assert(fsmn_lds_bytes<bf16_raw, HD, FS>() <= S::kLds, "FSMN filter fits the LDS");
      fsmn_rows<bf16_raw, HD, FS, BM * (HD / 4) / NT, NT>(a.f, static_cast<const bf16_raw*>(p.v) + sv.v_off,
                                                         p.v_token_stride, b, h, qt * BM, sv.n_k, sv.len_q, tid,
                                                         lds);
      return;
    }
  }

  int b, hq, qt;
  work_item(p, q_tiles, total, (int)blockIdx.x, b, hq, qt);
  const int hkv = hq / (p.heads_q / p.heads_kv);
  const SeqView sv = seq_view(p, b, hq, hkv);
  const int row0 = qt * BM;
  if (row0 >= sv.len_q) return;  // uniform over the workgroup
  // Rows computed: [0, len_c).  With zero-padded rows a padded sequence's
  // rows at or past its key count are not computed; they get zeros.
  const int len_c = (p.flags & ASRATTN_FWD_ZERO_PADDED_ROWS) != 0 ? min(sv.len_q, sv.n_k) : sv.len_q;
  if (row0 >= len_c) {
    constexpr int kCPRz = HD / 8;
    for (int ch = (int)threadIdx.x; ch < (min(row0 + BM, sv.len_q) - row0) * kCPRz; ch += S::kThreads) {
      bf16_raw* op = static_cast<bf16_raw*>(p.out) + sv.o_off + (int64_t)(row0 + ch / kCPRz) * p.o_token_stride +
                     (ch % kCPRz) * 8;
      __builtin_nontemporal_store((u32x4_t){0u, 0u, 0u, 0u}, reinterpret_cast<u32x4_t*>(op));
    }
    return;  // uniform over the workgroup
  }

  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: DMA destinations live in SGPRs
  const int rb = wave % RB;         // row block
  const int ks = (wave / RB) % KS;  // key split
  const int dh = wave / (RB * KS);  // dimension split: head dims [dh DH, dh DH + DH)
  const int r32 = lane & 31;
  const int half = lane >> 5;
  const int wrow0 = row0 + 32 * rb;
  const int row = wrow0 + r32;
  const bool row_ok = row < len_c;
  // Keys the workgroup (its last row) and this wave (its last row) see; with
  // a sliding window they start at the workgroup's first row's first key,
  // kofs, and the tiles count keys from there.
  const int last = min(row0 + BM, len_c) - 1;
  const int wlast = min(wrow0 + 32, len_c) - 1;
  const int kend = visible_keys(p, sv, last);
  const int kofs = WIN ? min(first_key(p, sv, row0), kend) : 0;
  const int n_tiles = (kend - kofs + SPAN - 1) / SPAN;
  const int row_lim = visible_keys(p, sv, row) - kofs;  // this row: keys [row_lo, row_lim) after kofs
  const int row_lo = WIN ? first_key(p, sv, row) - kofs : 0;
  const int wkend = wrow0 < len_c ? visible_keys(p, sv, wlast) - kofs : 0;
  const int wkbeg = WIN && wrow0 < len_c ? first_key(p, sv, wrow0) - kofs : 0;

  // Low 32 bits of the flat address of an LDS variable are its LDS offset.
  const uint32_t lds_base = (uint32_t)(uintptr_t)lds;

  // Q^T operand: lane (row, half) holds head_dim [16 kk + 8 half, +8).
  bf16x8_t qreg[KST];
  {
    const bf16_raw* qp = static_cast<const bf16_raw*>(p.q) + sv.q_off +
                         (int64_t)(row_ok ? row : 0) * p.q_token_stride + dh * DH + half * 8;
#pragma unroll
    for (int kk = 0; kk < KST; ++kk) {
      const uint4 v = row_ok ? *reinterpret_cast<const uint4*>(qp + kk * 16) : make_uint4(0, 0, 0, 0);
      qreg[kk] = __builtin_bit_cast(bf16x8_t, v);
    }
  }

  // K/V of the (sequence, kv head) up to the workgroup's last visible key.
  const uint32_t kts = (uint32_t)(p.k_token_stride * 2);
  const uint32_t vts = (uint32_t)(p.v_token_stride * 2);
  const __amdgpu_buffer_rsrc_t krs = buffer_rsrc(
      static_cast<const bf16_raw*>(p.k) + sv.k_off + (int64_t)kofs * p.k_token_stride, (uint32_t)(kend - kofs) * kts);
  const __amdgpu_buffer_rsrc_t vrs = buffer_rsrc(
      static_cast<const bf16_raw*>(p.v) + sv.v_off + (int64_t)kofs * p.v_token_stride, (uint32_t)(kend - kofs) * vts);

  // DMA instruction wave * NPW + i of a tile fills LDS slots 64 j + lane:
  // physical row s / CPR, physical chunk s % CPR, holding the logical chunk
  // the permutation puts there.
  uint32_t koff[NPW], voff[NPW];
#pragma unroll
  for (int i = 0; i < NPW; ++i) {
    const int s = 64 * (wave * NPW + i) + lane;
    const int pr = s / CPR;
    const int pc = s % CPR;
    koff[i] = (uint32_t)pr * kts + (uint32_t)k_logical<HD>(pr, pc) * 16;
    voff[i] = (uint32_t)pr * vts + (uint32_t)v_phys<HD>(pr, pc) * 16;
  }
  // Tile t goes to ring stage t % ST (passed as `stage`, a constant after
  // unrolling).
  auto issue = [&](int t, int stage_idx) {
    const uint32_t stage = lds_base + (uint32_t)stage_idx * SB;
    const uint32_t kk0 = (uint32_t)(t * SPAN) * kts;
    const uint32_t vv0 = (uint32_t)(t * SPAN) * vts;
#pragma unroll
    for (int i = 0; i < NPW; ++i)
      dma16(krs, stage + (uint32_t)(wave * NPW + i) * 1024, koff[i] + kk0);
#pragma unroll
    for (int i = 0; i < NPW; ++i)
      dma16(vrs, stage + TB + (uint32_t)(wave * NPW + i) * 1024, voff[i] + vv0);
  };

  // Operand addresses in stage 0, in this wave's sub-tile (rows ks BN ..).
  // K: row 32 kb + r32, logical chunk 2 kk + half.  V (transpose read): key
  // row 16 t + 8 hi + tr_row and columns 32 db + tr_col of each 8-key x
  // 32-column block.  BN is a multiple of 32, so the chunk permutations
  // depend on the same low row bits in every sub-tile.  The addresses
  // are masked to 18 bits (LDS addresses), which proves their sign bit
  // clear: only then do the constant parts added below (stage, key block,
  // k-step) fold into the ds_read offset field.
  // Past 16 chunks the rotation repeats in every 256-byte group, so k-step
  // kk reads at kaddr[kk % 8] + 256 (kk / 8) (and V column block db at
  // vaddr[db % 4] + 256 (db / 4)).
  constexpr int KA = KST < 8 ? KST : 8;
  constexpr int VA = DB < 4 ? DB : 4;
  uint32_t kaddr[KA];
#pragma unroll
  for (int kk = 0; kk < KA; ++kk)
    kaddr[kk] = (lds_base + (uint32_t)(ks * BN + r32) * RBYTES +
                 (uint32_t)k_phys<HD>(r32, 2 * (dh * KST + kk) + half) * 16) &
                0x3ffffu;
  const int tr_row = 4 * ((lane >> 4) >> 1) + ((lane & 15) >> 2);
  const int tr_cc = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);  // chunk within the 32-column block
  uint32_t vaddr[VA];
#pragma unroll
  for (int db = 0; db < VA; ++db)
    vaddr[db] = (lds_base + TB + (uint32_t)(ks * BN + tr_row) * RBYTES +
                 (uint32_t)v_phys<HD>(tr_row, 4 * (dh * DB + db) + tr_cc) * 16 + (lane & 1) * 8) &
                0x3ffffu;

  f32x16_t oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db] = f32x16_t{};
  const float c = a.c;
  // Running row max in scaled (base-2) units, possibly stale by up to
  // kLazy: scores are exponentiated against it, so p <= 2^kLazy, which fp32
  // sums and bf16 operands hold with unchanged relative precision.  O and l
  // are rescaled only when some row's max grows by more than that.
  constexpr float kLazy = 8.f;
  // Head_dim 64 (kSumFirst): a tile is first exponentiated against m_run
  // without its row max; the result stands when each lane's sum over its
  // keys is at most kSumCap, which bounds every p by 2^13 (bf16 and fp32
  // keep their relative precision at any magnitude; the cap keeps l and O
  // far from overflow).  Otherwise the tile takes the row max and the lazy
  // rescale above.  Whisper large-v3-turbo's encoder: 217 -> 211.5 us per
  // launch; at head_dim 128 (SenseVoice) the row max first was 2% faster.
  constexpr bool kSumFirst = HD == 64;
  constexpr float kSumCap = 8192.f;
  float m_run = kNegInf;
  float l_run = 0.f;

  // Whether the sub-tile starting at key kt needs the per-key mask (some row
  // of the wave sees fewer than all of its keys -- the wave's first row sees
  // the fewest -- or, with a window, some row's window starts inside it --
  // the wave's last row's starts latest).
  const int wmin = wrow0 < len_c ? visible_keys(p, sv, wrow0) - kofs : 0;
  const int wlo = WIN && wrow0 < len_c ? first_key(p, sv, wlast) - kofs : 0;
  auto masked = [&](int kt) { return kt + BN > wmin || (WIN && kt < wlo); };

  // S^T of tile j (stage stage_idx) into s.  The K operands' LDS reads run
  // two k-steps ahead of their matrix instructions; the scheduling groups
  // pin that order (left alone, the compiler keeps one k-step's reads in
  // flight, and the encoder lines measured 0.4-2% longer; three or four
  // k-steps ahead cost Whisper large-v3-turbo 3-4%).
  auto qk = [&](int stage_idx, f32x16_t* s) {
    const uint32_t so = (uint32_t)stage_idx * SB;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) s[kb] = f32x16_t{};
    bf16x8_t kf[KST][KB];
#pragma unroll
    for (int kk = 0; kk < KST; ++kk)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) kf[kk][kb] = lds_read16(kaddr[kk % KA] + (kk / KA) * 256 + so + kb * 32 * RBYTES);
#pragma unroll
    for (int kk = 0; kk < KST; ++kk)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) s[kb] = mfma32(kf[kk][kb], qreg[kk], s[kb]);
    constexpr int kAhead = KST < 2 ? KST : 2;
    constexpr int kDsRead = 0x100, kMfma = 0x008;  // sched_group_barrier instruction classes
    __builtin_amdgcn_sched_group_barrier(kDsRead, kAhead * KB, 0);
#pragma unroll
    for (int i = 0; i < KST - kAhead; ++i) {
      __builtin_amdgcn_sched_group_barrier(kMfma, KB, 0);
      __builtin_amdgcn_sched_group_barrier(kDsRead, KB, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kMfma, kAhead * KB, 0);
  };
  // Keys outside the row's [row_lo, row_lim) -> -inf.  Accumulator r of
  // block kb is key kt + 32 kb + 8 (r / 4) + 4 half + r % 4.
  auto mask = [&](int kt, f32x16_t* s) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kt + kb * 32 + (r / 4) * 8 + half * 4 + (r % 4);
        if (key >= row_lim || (WIN && key < row_lo)) s[kb][r] = kNegInf;
      }
  };
  // Row max over the tile, combined across the half waves, scaled.
  auto rowmax = [&](const f32x16_t* s) {
    float mt = s[0][0];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int r = (kb == 0 ? 1 : 0); r < 16; ++r) mt = fmaxf(mt, s[kb][r]);
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
    return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * c;
  };
  // P^T = 2^(s c - mu) as bf16 MFMA operands; returns the lane's fp32 sum:
  // at head_dim 64 the sum of the bf16 P^T operands themselves, two per
  // v_dot2_f32_bf16 in four chains (Whisper large-v3-turbo's encoder 213.6
  // -> 208 us per launch; head_dim 128 1-5% slower than fp32 adds), else a
  // pairwise tree of fp32 adds (five dependent adds at 32 values).
  auto softmax = [&](const f32x16_t* s, float mu, bf16x8_t* pb) {
    typedef short short2_t __attribute__((ext_vector_type(2)));
    const short2_t ones = {0x3f80, 0x3f80};  // bf16 1.0
    float pacc[4] = {0.f, 0.f, 0.f, 0.f};
    float pr[16 * KB];
#pragma unroll
    for (int t = 0; t < 2 * KB; ++t) {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p0 = fast_exp2(fmaf(s[t / 2][(t % 2) * 8 + 2 * i], c, -mu));
        const float p1 = fast_exp2(fmaf(s[t / 2][(t % 2) * 8 + 2 * i + 1], c, -mu));
        pr[8 * t + 2 * i] = p0;
        pr[8 * t + 2 * i + 1] = p1;
        w[i] = pack_bf16x2(p0, p1);
        if constexpr (HD == 64)
          pacc[i] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(short2_t, w[i]), ones, pacc[i], false);
      }
      pb[t] = __builtin_bit_cast(bf16x8_t, make_uint4(w[0], w[1], w[2], w[3]));
    }
    if constexpr (HD == 64) {
      return (pacc[0] + pacc[1]) + (pacc[2] + pacc[3]);
    } else {
#pragma unroll
      for (int w = 8 * KB; w >= 1; w /= 2)
#pragma unroll
        for (int i = 0; i < w; ++i) pr[i] += pr[i + w];
      return pr[0];
    }
  };
  // O^T += V^T . P^T over tile stage stage_idx.  MFMA t covers keys
  // 16 t + 8 (idx / 4) + 4 half + idx % 4.
  auto pv = [&](int stage_idx, const bf16x8_t* pb) {
    const uint32_t so = (uint32_t)stage_idx * SB;
#pragma unroll
    for (int t = 0; t < 2 * KB; ++t) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const uint32_t va = vaddr[db % VA] + (db / VA) * 256 + so;
        const short4_t lo = ds_read_tr(va + 16 * t * RBYTES);
        const short4_t hi = ds_read_tr(va + (16 * t + 8) * RBYTES);
        const bf16x8_t av = __builtin_bit_cast(bf16x8_t, (short8_t){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
        oacc[db] = mfma32(av, pb[t], oacc[db]);
      }
    }
  };
#pragma unroll
  for (int t = 0; t < ST - 1; ++t)
    if (t < n_tiles) issue(t, t);
  // The compiler tracks the Q loads but not the DMAs; consuming Q here makes
  // its wait for them happen once, before the loop, instead of before the
  // first MFMA of every tile (where it would drain the ring).
#pragma unroll
  for (int kk = 0; kk < KST; ++kk) asm volatile("" ::"v"(qreg[kk]));

  // Tile j (ring stage stage_idx = j % ST): S^T, mask, row max, lazy
  // rescale, P^T and O^T += V^T P^T.
  auto tile = [&](int j, int stage_idx) {
    // This wave's part of tile j has landed once at most the tiles after it
    // are outstanding; after the barrier every wave's part has, and every
    // wave is done with tile j - 1, whose stage the next DMA reuses.
    wait_dma<2 * NPW, ST - 2>(min(ST - 2, n_tiles - 1 - j));
    __syncthreads();
    if (j + ST - 1 < n_tiles) issue(j + ST - 1, (stage_idx + ST - 1) % ST);
    const int kt = j * SPAN + ks * BN;  // this wave's first key (after kofs)
    const bool idle = kt >= wkend || (WIN && kt + BN <= wkbeg);  // uniform per wave
    f32x16_t s[KB];
    if constexpr (DS > 1) {
      // Every wave reaches the partial-score barrier, idle or not.
      float* const part = reinterpret_cast<float*>(lds + S::kRingBytes);
      if (!idle) {
        qk(stage_idx, s);
        float* mine = part + (size_t)wave * KB * 16 * 64 + lane;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) mine[(kb * 16 + r) * 64] = s[kb][r];
      }
      __syncthreads();
      if (idle) return;
      // Every wave of the row block sums the partials in the same order, so
      // all of them run the same softmax.
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) s[kb] = f32x16_t{};
#pragma unroll
      for (int d = 0; d < DS; ++d) {
        const float* src = part + (size_t)(rb + RB * d) * KB * 16 * 64 + lane;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) s[kb][r] += src[(kb * 16 + r) * 64];
      }
    } else {
      if (idle) return;  // the barrier is above
      qk(stage_idx, s);
    }
    if (masked(kt)) mask(kt, s);
    // kSumFirst: first against the running max as it stands, with no row
    // max taken; kept unless some row has no max yet or some lane's sum
    // shows a probability above kSumCap (or is not finite).
    bf16x8_t pb[2 * KB];
    float ps = 0.f;
    bool full = !kSumFirst || __any(m_run == kNegInf);
    if (!full) {
      ps = softmax(s, m_run, pb);
      full = __any(!(ps <= kSumCap));
    }
    if (full) {
      const float mt = rowmax(s);
      // Rescale only when some row's max grew past the slack (always on
      // the first tile, where m_run is -inf).
      if (__any(mt > m_run + kLazy)) {
        const float mn = fmaxf(m_run, mt);
        const float alpha = mn == kNegInf ? 1.f : fast_exp2(m_run - mn);
#pragma unroll
        for (int db = 0; db < DB; ++db) oacc[db] *= alpha;
        l_run *= alpha;
        m_run = mn;
      }
      const float mu = m_run == kNegInf ? 0.f : m_run;
      ps = softmax(s, mu, pb);
    }
    l_run += ps;
    pv(stage_idx, pb);
  };
  // Unrolled over the ring so that every stage offset is a constant.
  for (int j0 = 0; j0 < n_tiles; j0 += ST) {
#pragma unroll
    for (int st = 0; st < ST; ++st)
      if (j0 + st < n_tiles) tile(j0 + st, st);
  }
  __syncthreads();  // the ring is free for the merge and the output staging


  // Merge the key splits of each row block through LDS; afterwards wave
  // (rb, 0) stages its rows in the first merge slot of its row block (which
  // only it reads) or, without splits, in its own region.
  constexpr int ORS = S::kOutRow;
  bf16_raw* stage;
  if constexpr (KS > 1) {
    constexpr int kPer = S::kMergeFloats;
    float* const mf = reinterpret_cast<float*>(lds);
    if (ks > 0) {
      float* dst = mf + (rb * (KS - 1) + ks - 1) * kPer + lane;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) dst[(db * 16 + r) * 64] = oacc[db][r];
      dst[(DB * 16) * 64] = m_run;
      dst[(DB * 16 + 1) * 64] = l_run;
    }
    __syncthreads();
    if (ks > 0) return;  // no barrier follows
#pragma unroll
    for (int s2 = 1; s2 < KS; ++s2) {
      const float* src = mf + (rb * (KS - 1) + s2 - 1) * kPer + lane;
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
    stage = reinterpret_cast<bf16_raw*>(lds) + rb * 32 * ORS;
  }
  if (wrow0 >= sv.len_q) return;  // uniform per wave; no barrier follows

  // The half waves hold disjoint keys of the same rows.
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = l_tot > 0.f && row_ok ? 1.f / l_tot : 0.f;  // rows past len_c get zeros
  // Accumulator r of block db is column 32 db + 8 (r / 4) + 4 half + r % 4
  // of row r32: write the normalized rows to LDS ...
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t w0 = pack_bf16x2(oacc[db][4 * i] * inv, oacc[db][4 * i + 1] * inv);
      const uint32_t w1 = pack_bf16x2(oacc[db][4 * i + 2] * inv, oacc[db][4 * i + 3] * inv);
      *reinterpret_cast<uint2*>(stage + r32 * ORS + dh * DH + db * 32 + i * 8 + half * 4) = make_uint2(w0, w1);
    }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // ... and store them to global memory 16 bytes per lane, whole rows per
  // instruction.
  constexpr int kRowChunks = DH / 8;  // this wave's columns
#pragma unroll
  for (int i = 0; i < 32 * kRowChunks / 64; ++i) {
    const int ch = i * 64 + lane;
    const int r = ch / kRowChunks;
    const int col = dh * DH + (ch % kRowChunks) * 8;
    const int orow = wrow0 + r;
    const uint4 val = *reinterpret_cast<const uint4*>(stage + r * ORS + col);
    if (orow < sv.len_q) {
      bf16_raw* op = static_cast<bf16_raw*>(p.out) + sv.o_off + (int64_t)orow * p.o_token_stride + col;
      // Nontemporal: the output is not read again in this launch (Qwen3's
      // prompt pass 20.2 -> 19.3 us, SenseVoice -1%).
      __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, val), reinterpret_cast<u32x4_t*>(op));
    }
  }
}

template <int HD, int RB, int KS, int BN, int ST, int OCC, int FS, bool WIN = false, int DS = 1>
hipError_t launch_typed(const FwdArgs& a, hipStream_t stream) {
  using S = RingShape<HD, RB, KS, BN, ST, DS>;
  const asrattn_fwd_params& p = a.p;
  const int q_tiles = (p.max_len_q + S::kBM - 1) / S::kBM;
  const long long total = (long long)q_tiles * p.heads_q * p.batch;
  if (total <= 0) return hipSuccess;
  // With FSMN items the grid holds every item twice (attention, then FSMN).
  const int copies = FS > 0 ? 2 : 1;
  if (copies * total > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  const unsigned grid = (unsigned)(copies * total);
  hipLaunchKernelGGL((fwd_ring_kernel<HD, RB, KS, BN, ST, OCC, FS, WIN, DS>), dim3(grid), dim3(S::kThreads), 0, stream, a,
                     q_tiles, (int)total);
  return hipGetLastError();
}

template <int HD>
hipError_t launch_hd(const FwdArgs& a, hipStream_t stream) {
  // Four waves (128 query rows) share each 64-key tile through two stages:
  // two workgroups per CU, whose waves pair up on the SIMDs without sharing
  // a barrier.  Key splits (KS > 1) halve the rows a CU holds at two waves
  // per SIMD, which costs more than they save once the batch fills the GPU.
  // Head dims 256 and 512 (Gemma 4) split each row block's dimensions over
  // waves (32 rows' queries and outputs of all 256 dimensions fit one wave
  // only at one wave per SIMD, of 512 not without spilling); 32-key tiles.
  // Sliding windows (causal, Gemma 4) take a variant that starts each
  // workgroup's keys at its first row's window.
  const bool win = a.p.window > 0;
  if constexpr (HD == 512) {
    // 64 query rows, each row block's dimensions over four waves (eight
    // waves, the whole 160 KB of LDS; 7% faster than two waves per row block).
    if (win) return launch_typed<HD, 2, 1, 32, 2, 1, 0, true, 4>(a, stream);
    return launch_typed<HD, 2, 1, 32, 2, 1, 0, false, 4>(a, stream);
  } else if constexpr (HD == 256) {
    // 128 query rows, each row block's dimensions over two waves (eight
    // waves, two per SIMD: 9% faster on Gemma 4's prompt pass than four
    // waves holding all 256 dimensions at one per SIMD).
    if (win) return launch_typed<HD, 4, 1, 32, 2, 1, 0, true, 2>(a, stream);
    return launch_typed<HD, 4, 1, 32, 2, 1, 0, false, 2>(a, stream);
  } else {
    if (win) return launch_typed<HD, 4, 1, 64, 2, 2, 0, true>(a, stream);
    if (a.f.memory != nullptr) return launch_typed<HD, 4, 1, 64, 2, 2, kFsmnFusedKernel>(a, stream);
    return launch_typed<HD, 4, 1, 64, 2, 2, 0>(a, stream);
  }
}

}  // namespace

bool fwd_ring_supported(const asrattn_fwd_params& p) {
  if (p.dtype != ASRATTN_BF16) return false;
  if (p.head_dim != 64 && p.head_dim != 128 && p.head_dim != 256 && p.head_dim != 512) return false;
  // A key row must end before the next one starts for the resource bound
  // (last visible key's row end) to cover every visible key.
  if (p.k_token_stride < p.head_dim || p.v_token_stride < p.head_dim) return false;
  // K/V are addressed with 32-bit byte offsets from the sequence's first key,
  // up to one tile past its last.
  const long long span_k = ((long long)p.max_len_k + 256) * p.k_token_stride * 2;
  const long long span_v = ((long long)p.max_len_k + 256) * p.v_token_stride * 2;
  return span_k < (1LL << 31) && span_v < (1LL << 31);
}

hipError_t launch_fwd_ring(const asrattn_fwd_params& p, const FsmnArgs* fsmn, hipStream_t stream) {
  FwdArgs a;
  a.p = p;
  a.c = p.scale * kLog2e;
  a.f = fsmn != nullptr ? *fsmn : FsmnArgs{};
  switch (p.head_dim) {
    case 64: return launch_hd<64>(a, stream);
    case 128: return launch_hd<128>(a, stream);
    case 256: return launch_hd<256>(a, stream);
    default: return launch_hd<512>(a, stream);
  }
}

}  // namespace asrattn
