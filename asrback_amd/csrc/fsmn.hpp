// SAN-M's FSMN memory (a depthwise convolution over time of the masked
// values, plus those values, masked again), computed for a block of rows of
// one (sequence, head):
//
//   memory[b, t, c] = keep(t) * (conv_t + v'[t, c]) + bias[c]
//   conv_t          = sum_i weight[c, i] * v'[t + i - left, c]
//   v'[s, c]        = v[b, s, c] if 0 <= s < n else 0,   keep(t) = t < n
//
// with c = h * HD + d, left = (K - 1) / 2 and n the sequence's frame count.
// Rounding follows the reference's sequence of ops in the element type: the
// convolution (fp32 accumulation) is rounded, then the sum with v', then the
// sum with the bias.
//
// Thread layout: each thread owns 4 channels (one 8- or 16-byte vector) and
// RS consecutive rows; it loads the RS + KW - 1 value rows its outputs
// touch once (range-checked buffer loads: rows outside [0, n) read zeros)
// and slides the KW-tap window over them in registers.  KW is the window
// the code is unrolled for (odd); any K <= KW runs in it, the window taps
// outside the filter having weight zero (so for K < KW an infinite value in
// a row next to the filter's reach turns the output NaN, where the
// convolution alone would not see it).
#pragma once

#include "common.hpp"

namespace asrattn {

// Largest filter the kernels take (any K <= 15), and the window of the
// attention kernel's fused epilogue (K <= 11; SenseVoiceSmall's K is 11).
constexpr int kFsmnMaxKernel = 15;
constexpr int kFsmnFusedKernel = 11;

struct FsmnArgs {
  const void* weight;  // (HD * heads, K), row c = channel c
  const void* bias;    // (HD * heads) or null
  void* memory;        // (batch, rows, HD * heads), unit channel stride
  int64_t m_batch_stride, m_token_stride;
  int kernel_size;
};

template <typename T>
struct FsmnElem;

template <>
struct FsmnElem<float> {
  typedef uint4 Raw;  // 4 channels
  static __device__ __forceinline__ Raw load(__amdgpu_buffer_rsrc_t r, uint32_t off) { return buffer_load16(r, off); }
  static __device__ __forceinline__ float get(const Raw& x, int j) {
    return __uint_as_float(j == 0 ? x.x : j == 1 ? x.y : j == 2 ? x.z : x.w);
  }
  static __device__ __forceinline__ float round(float x) { return x; }
  static __device__ __forceinline__ void store(__amdgpu_buffer_rsrc_t r, uint32_t off, const float* v) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int,
                                                              (f32x4){v[0], v[1], v[2], v[3]}),
                                           r, off, 0, 0);
  }
  static __device__ __forceinline__ float scalar(const float* p) { return *p; }
  static __device__ __forceinline__ float from_bits(uint32_t x) { return __uint_as_float(x); }
};

template <>
struct FsmnElem<bf16_raw> {
  typedef uint2 Raw;
  static __device__ __forceinline__ Raw load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    return make_uint2(v[0], v[1]);
  }
  static __device__ __forceinline__ float get(const Raw& x, int j) {
    return j == 0 ? bf16_lo(x.x) : j == 1 ? bf16_hi(x.x) : j == 2 ? bf16_lo(x.y) : bf16_hi(x.y);
  }
  static __device__ __forceinline__ float round(float x) { return bf16_to_f32(f32_to_bf16(x)); }
  static __device__ __forceinline__ void store(__amdgpu_buffer_rsrc_t r, uint32_t off, const float* v) {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    __builtin_amdgcn_raw_buffer_store_b64((u32x2){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])}, r, off, 0, 0);
  }
  static __device__ __forceinline__ float scalar(const bf16_raw* p) { return bf16_to_f32(*p); }
};

// LDS bytes fsmn_rows needs for the head's filter: fp32 taps, or bf16 taps
// in pairs (the last, odd one paired with zero).
template <typename T, int HD, int KW>
constexpr int fsmn_lds_bytes() {
  return sizeof(T) == 2 ? (KW + 1) / 2 * HD * 4 : KW * HD * 4;
}

// Rows [row0, min(row0 + NT * 4 * RS / HD, len)) of head h of sequence b,
// by the NT threads of the workgroup (thread index tid; all of them must
// call, it has a barrier).  v_seq points at the sequence's value row 0 of
// head h; n is its frame count (<= len); vts the value token stride
// (elements).  lds: fsmn_lds_bytes<T, HD, KW>() bytes of LDS, 16-byte
// aligned, for the head's filter laid out tap-major (window tap wi of
// channel d at wi * HD + d, zero where the window has no filter tap), so
// that a thread's four channels of one tap (or tap pair) are one vector
// read.
//
// bf16 sums the taps in pairs with v_dot2_f32_bf16 (products of bf16 values
// are exact in fp32, the pair's sum rounds once), on value pairs (row s,
// row s + 1) of one channel formed with v_perm_b32; the last tap is an FMA.
template <typename T, int HD, int KW, int RS, int NT>
__device__ __forceinline__ void fsmn_rows(const FsmnArgs& f, const T* v_seq, int64_t vts, int b, int h, int row0,
                                          int n, int len, int tid, unsigned char* lds) {
  using E = FsmnElem<T>;
  constexpr bool kPairs = sizeof(T) == 2;
  constexpr int G = HD / 4;  // channel groups of a head
  constexpr int CW = (KW - 1) / 2;
  constexpr int NR = RS + KW - 1;  // value rows a thread reads
  constexpr int NP = (KW + 1) / 2;  // tap pairs (bf16)
  static_assert(NT % G == 0, "threads cover whole rows");
  static_assert(KW % 2 == 1, "odd window");
  const int g = tid % G;
  const int t0 = row0 + (tid / G) * RS;
  const int K = f.kernel_size;
  const int left = (K - 1) / 2;
  const int c0 = h * HD + g * 4;

  // Value rows t0 - CW .. t0 + RS + CW - 1, issued first; rows outside
  // [0, n) read zeros (negative rows wrap to offsets far past the end).
  const uint32_t row_bytes = (uint32_t)(vts * (int64_t)sizeof(T));
  const __amdgpu_buffer_rsrc_t vr = buffer_rsrc(v_seq, (uint32_t)n * row_bytes);
  typename E::Raw x[NR];
#pragma unroll
  for (int s = 0; s < NR; ++s)
    x[s] = E::load(vr, (uint32_t)(t0 - CW + s) * row_bytes + (uint32_t)(g * 4 * sizeof(T)));

  // The head's filter into LDS, tap-major.  Window tap wi is filter tap
  // wi - CW + left.
  const T* wp = static_cast<const T*>(f.weight) + (int64_t)h * HD * K;
  auto tap = [&](int wi, int d) -> uint32_t {  // raw bits (bf16 in the low half)
    const int i = wi - CW + left;
    if (wi >= KW || i < 0 || i >= K) return 0u;
    if constexpr (kPairs) return (uint32_t)wp[d * K + i];
    else return __float_as_uint(wp[d * K + i]);
  };
  uint32_t* wl = reinterpret_cast<uint32_t*>(lds);
  constexpr int kRows = kPairs ? NP : KW;
  for (int idx = tid; idx < kRows * HD; idx += NT) {
    const int r = idx / HD;
    const int d = idx % HD;
    wl[idx] = kPairs ? (tap(2 * r, d) | (tap(2 * r + 1, d) << 16)) : tap(r, d);
  }
  float bias[4] = {0.f, 0.f, 0.f, 0.f};
  if (f.bias != nullptr) {
#pragma unroll
    for (int j = 0; j < 4; ++j) bias[j] = E::scalar(static_cast<const T*>(f.bias) + c0 + j);
  }
  __syncthreads();
  uint32_t w[kRows][4];
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const uint4 q = *reinterpret_cast<const uint4*>(wl + r * HD + g * 4);
    w[r][0] = q.x, w[r][1] = q.y, w[r][2] = q.z, w[r][3] = q.w;
  }

  // The row sums of the convolution.
  float conv[RS][4];
  if constexpr (kPairs) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    auto pair = [](uint32_t u) { return __builtin_bit_cast(bf16x2_t, u); };
    // (row s, row s + 1) of channel j, for the pairs the taps 0..KW-2 use.
    uint32_t vp[RS + KW - 2][4];
#pragma unroll
    for (int s = 0; s < RS + KW - 2; ++s) {
      vp[s][0] = __builtin_amdgcn_perm(x[s + 1].x, x[s].x, 0x05040100u);
      vp[s][1] = __builtin_amdgcn_perm(x[s + 1].x, x[s].x, 0x07060302u);
      vp[s][2] = __builtin_amdgcn_perm(x[s + 1].y, x[s].y, 0x05040100u);
      vp[s][3] = __builtin_amdgcn_perm(x[s + 1].y, x[s].y, 0x07060302u);
    }
#pragma unroll
    for (int r = 0; r < RS; ++r)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float acc = fmaf(bf16_lo(w[NP - 1][j]), E::get(x[r + KW - 1], j), 0.f);
#pragma unroll
        for (int p = 0; p < NP - 1; ++p) acc = __builtin_amdgcn_fdot2_f32_bf16(pair(vp[r + 2 * p][j]), pair(w[p][j]), acc, false);
        conv[r][j] = acc;
      }
  } else {
#pragma unroll
    for (int r = 0; r < RS; ++r)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float acc = 0.f;
#pragma unroll
        for (int wi = 0; wi < KW; ++wi) acc = fmaf(__uint_as_float(w[wi][j]), E::get(x[r + wi], j), acc);
        conv[r][j] = acc;
      }
  }

  // Stores past row len fall outside the resource and are dropped.
  const uint32_t m_row = (uint32_t)(f.m_token_stride * (int64_t)sizeof(T));
  const __amdgpu_buffer_rsrc_t mr =
      buffer_rsrc(static_cast<T*>(f.memory) + (int64_t)b * f.m_batch_stride, (uint32_t)len * m_row);
#pragma unroll
  for (int r = 0; r < RS; ++r) {
    const int t = t0 + r;
    float m[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float mem = E::round(E::round(conv[r][j]) + E::get(x[r + CW], j));
      // The store rounds the sum with the bias (zero without one).
      m[j] = (t < n ? mem : 0.f) + bias[j];
    }
    E::store(mr, (uint32_t)t * m_row + (uint32_t)(c0 * sizeof(T)), m);
  }
}

}  // namespace asrattn
