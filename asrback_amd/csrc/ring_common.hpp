// Building blocks of the matrix-core forward kernel (fwd_ring.hip): bf16
// MFMA operands, LDS reads by byte address, the gfx950 transpose read, K/V
// DMA straight from HBM into LDS, and the launch-id -> work-item orders (XCD
// grouping, longest sequences first).
#pragma once

#include "common.hpp"
#include "fwd_common.hpp"

namespace asrattn {
namespace ring {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef short short8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t* lds_short4_ptr;
typedef __attribute__((address_space(3))) const bf16x8_t* lds_bf16x8_ptr;

__device__ __forceinline__ f32x16_t mfma32(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// LDS reads by byte address, so that constant parts of an address fold
// into the instruction's offset field.
__device__ __forceinline__ bf16x8_t lds_read16(uint32_t addr) { return *(lds_bf16x8_ptr)(size_t)addr; }

// Transpose load of 4 bf16: within each 16-lane group, lane j receives
// element (j % 4) of the 8-byte chunks addressed by lanes 4k + j / 4,
// k = 0..3.
__device__ __forceinline__ short4_t ds_read_tr(uint32_t addr) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_ptr)(size_t)addr);
}

// One DMA instruction: lane i copies the 16 bytes at buffer offset `voff`
// into LDS bytes [lds_base + 16 i, +16).  Issued as inline assembly so that
// the compiler's wait-count pass, which cannot tell ring stages apart, does
// not drain every DMA before each LDS read; the kernels wait for them
// themselves (wait_vmcnt).  M0 is saved and restored around the instruction.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds_base, uint32_t voff) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds_base), "v"(voff), "s"(rsrc)
      : "memory");
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt in bits 3:0 and 15:14; expcnt
// and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
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

// Visible keys of sequence b before any causal limit.
__device__ __forceinline__ int sequence_keys(const asrattn_fwd_params& p, int b) {
  int n = p.cu_seqlens_k != nullptr ? p.cu_seqlens_k[b + 1] - p.cu_seqlens_k[b] : p.max_len_k;
  n = min(max(n, 0), p.max_len_k);
  if (p.seqused_k != nullptr) n = min(n, max(p.seqused_k[b], 0));
  return n;
}

// Rank of lane's key count n among lanes 0 .. N - 1 (decreasing count, ties
// in lane order); lanes past the batch hold -1, below every count.  Each
// lane's (count, lane) pair is one unique 32-bit key, (n << 6) | (63 - lane)
// (n < 2^25, which the caller checks), so a step is a lane read and one
// compare.  Unrolled with a constant bound, so the compiler overlaps each
// lane read with the compare of the one before (a loop to the batch size
// waited on every read: SenseVoice's 32 sequences 20.1 -> 19.8 us per
// launch, with the FSMN memory 27.6 -> 26.5; the single-compare key a
// further 0-3%).
template <int N>
__device__ __forceinline__ int count_rank(int n, int lane) {
  const uint32_t key = n < 0 ? 0u : ((uint32_t)n << 6) | (uint32_t)(63 - lane);
  int rank = 0;
#pragma unroll
  for (int j = 0; j < N; ++j) rank += (uint32_t)__builtin_amdgcn_readlane((int)key, j) > key ? 1 : 0;
  return rank;
}

// The sequence of rank r in decreasing key count (ties in index order), for
// batches of at most 64: lane b ranks sequence b against all others.
__device__ __forceinline__ int ranked_sequence(const asrattn_fwd_params& p, int r) {
  const int lane = threadIdx.x & 63;
  const int n = lane < p.batch ? sequence_keys(p, lane) : -1;
  const int rank = p.batch <= 8    ? count_rank<8>(n, lane)
                   : p.batch <= 16 ? count_rank<16>(n, lane)
                   : p.batch <= 32 ? count_rank<32>(n, lane)
                                   : count_rank<64>(n, lane);
  const unsigned long long hit = __ballot(lane < p.batch && rank == r);
  return __ffsll(hit) - 1;  // ranks are a permutation: exactly one lane
}

// Physical chunk of logical chunk c in row r of a K tile, and its inverse;
// rows of more than 16 chunks (head_dim 256, 512) rotate within each group
// of 16 chunks.  The rotation puts the 16 rows one b128 operand read touches
// per cycle in 16 different bank groups.
template <int HD>
__device__ __forceinline__ int k_phys(int r, int c) {
  if constexpr (HD == 64) return (c + (r >> 1)) & 7;
  return (c & ~15) | ((c + r) & 15);
}
template <int HD>
__device__ __forceinline__ int k_logical(int r, int pc) {
  if constexpr (HD == 64) return (pc - (r >> 1)) & 7;
  return (pc & ~15) | ((pc - r) & 15);
}
// V tiles: an XOR (its own inverse) that puts the four rows of a transpose
// read in four different 64-byte bank ranges.
template <int HD>
__device__ __forceinline__ int v_phys(int r, int c) {
  return HD == 64 ? (c ^ (4 * ((r >> 1) & 1))) : (c ^ (4 * (r & 3)));
}

}  // namespace ring
}  // namespace asrattn
