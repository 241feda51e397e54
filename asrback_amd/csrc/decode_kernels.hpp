// Decoder-step attention: one query per sequence over a key/value cache.
//
// The step is bound by HBM: every key and value of a sequence is read once
// and used for one (or, with grouped-query attention, g) dot products.  The
// kernel therefore streams K and V with 16-byte loads, keeps a second batch
// of loads in flight while it consumes the first, and does all arithmetic in
// registers:
//
//   * K and V are read once, with nontemporal loads (no L2 allocation).
//   * A key row (head_dim elements) is covered by LPK lanes, 16 bytes each;
//     a wave loads 64 / LPK key rows per instruction, so every load touches
//     whole rows.  Each group of LPK lanes runs its own online softmax over
//     the keys it reads (a "stream"); the g query heads sharing the kv head
//     ride along on the same loads.
//   * A workgroup of W waves covers one (sequence, kv head) -- or, for small
//     batches, one of `splits` key ranges of it.  Its streams merge first
//     inside each wave (a butterfly of lane swaps) and then across waves in
//     LDS.
//     With enough (sequence, kv head) pairs to fill the GPU there is one
//     split and the workgroup writes the output; otherwise each split writes
//     an unnormalized partial (o, max, sum) and a small combine kernel folds
//     them.  No workgroup waits on another.
//   * Sequence lengths are read from device memory (seqused_k or
//     positions + 1), and splits past a sequence's end write an empty
//     partial, so the grid depends only on shapes and the launch can be
//     replayed from a graph while lengths change.
//
// Softmax runs in base 2: each reduced score q . k is multiplied by
// scale * log2(e), so p = 2^(s - max) on v_exp_f32.
//
// Paged caches (asrattn_decode_paged): a load batch is U slices of NS
// consecutive keys (one key per stream), NS-aligned; with page sizes that
// are multiples of NS each slice lies in one page, whose pool index is one
// uniform (scalar) load from the block table.  The slice's buffer resource
// starts at that page and ends at the sequence's last key in it, so unused
// page slots and pages past the sequence are never read.
#pragma once

#include "common.hpp"
#include "decode_args.hpp"
#include "kernels.hpp"

namespace asrattn {
namespace {


template <typename T, int HD, int G, int W>
struct DecodeShape {
  static constexpr int kEPL = Elem<T>::kPerVec;   // elements per lane per load
  static constexpr int kLPK = HD / kEPL;          // lanes per key row
  static constexpr int kKPW = 64 / kLPK;          // key rows per wave load (streams per wave)
  static constexpr int kThreads = 64 * W;
  static constexpr int kStreams = W * kKPW;       // softmax streams per workgroup
  // Keys per stream per load batch; with four query heads per kv head the
  // batches are halved so that two of them fit beside the heads' state in
  // 128 VGPRs.
  static constexpr int kUnroll = G >= 4 || HD >= 256 ? 2 : 4;
  static constexpr int kStep = kStreams * kUnroll;  // keys per load batch
  // Plain (not append) kernels on 4-wave workgroups load two keys per
  // stream per batch instead of four: Qwen3's paged step 4.71 -> 4.93 TB/s,
  // its slab step +1%; the fused step lost 4% with two and keeps four.
  // Slab and paged variants sum in the same order either way.
  static constexpr int kPlainUnroll = W == 4 && kUnroll == 4 ? 2 : kUnroll;
  static constexpr int kPlainStep = kStreams * kPlainUnroll;
  // Waves per SIMD the register budget allows: four (128 VGPRs) up to four
  // query heads per kv head, two (256) for eight.
  static constexpr int kOcc = G >= 8 ? 2 : 4;
  // The cross-wave merge stages every wave's (G x HD) partial output in LDS,
  // and two waves per SIMD allow at most 8 waves per workgroup.
  static constexpr bool kFits = W * G * HD * 4 <= 65536 && (kOcc == 4 || W <= 8);
  static_assert(kLPK >= 1 && kLPK <= 64 && (64 % kLPK) == 0, "head_dim/lane mapping");
};

// q . k over one lane's 16-byte slices, accumulated in fp32.
template <typename T>
__device__ __forceinline__ float dot16(const uint4& q, const uint4& k);

template <>
__device__ __forceinline__ float dot16<float>(const uint4& q, const uint4& k) {
  float acc = __uint_as_float(q.x) * __uint_as_float(k.x);
  acc = fmaf(__uint_as_float(q.y), __uint_as_float(k.y), acc);
  acc = fmaf(__uint_as_float(q.z), __uint_as_float(k.z), acc);
  return fmaf(__uint_as_float(q.w), __uint_as_float(k.w), acc);
}

// bf16 pairs on v_dot2c_f32_bf16: the products of two bf16 values are exact
// in fp32, so this equals the unpacked fp32 dot product up to summation
// order.
template <>
__device__ __forceinline__ float dot16<bf16_raw>(const uint4& q, const uint4& k) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  auto pair = [](uint32_t x) { return __builtin_bit_cast(bf16x2_t, x); };
  float acc = __builtin_amdgcn_fdot2_f32_bf16(pair(q.x), pair(k.x), 0.f, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(pair(q.y), pair(k.y), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(pair(q.z), pair(k.z), acc, false);
  return __builtin_amdgcn_fdot2_f32_bf16(pair(q.w), pair(k.w), acc, false);
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

template <typename T>
__device__ __forceinline__ uint4 pack(const float* x);

template <>
__device__ __forceinline__ uint4 pack<float>(const float* x) {
  return make_uint4(__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]), __float_as_uint(x[3]));
}

template <>
__device__ __forceinline__ uint4 pack<bf16_raw>(const float* x) {
  return make_uint4(pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]), pack_bf16x2(x[4], x[5]), pack_bf16x2(x[6], x[7]));
}

// x rounded to T (and back): where the reference's element-wise ops round.
template <typename T>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (sizeof(T) == 2) return bf16_to_f32(f32_to_bf16(x));
  return x;
}

// Per-head RMSNorm and rotary embedding of one row slice -- lane `sub` of
// the LPK lanes holding a head_dim row, EPL elements -- in the reference's
// rounding order (qwen3_asr.py:322-330): the norm x * rsqrt(mean(x^2) +
// eps) * w in fp32, rounded once; the rotation x c + r s with r = (-x[d/2:],
// x[:d/2]) rounded after each product and after the sum.  Element e of lane
// sub pairs with element e of lane sub ^ LPK/2.  w, cs and sn are the
// lane's slices of the weights and tables (loaded by the caller); has_norm
// and has_rot are uniform over the grid.  All lanes of the wave must take
// part.
template <typename T, int HD, int LPK>
__device__ __forceinline__ uint4 norm_rotate(uint4 raw, bool has_norm, const uint4& w, bool has_rot, const uint4& cs,
                                             const uint4& sn, float eps, int sub) {
  constexpr int EPL = Elem<T>::kPerVec;
  float x[EPL];
  unpack<T>(raw, x);
  if (has_norm) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) ss = fmaf(x[e], x[e], ss);
    ss = group_sum<LPK>(ss);
    const float r = rsqrtf(ss * (1.f / HD) + eps);
    float wv[EPL];
    unpack<T>(w, wv);
#pragma unroll
    for (int e = 0; e < EPL; ++e) x[e] = round_to<T>(x[e] * r * wv[e]);
  }
  if (has_rot) {
    float cv[EPL], sv[EPL];
    unpack<T>(cs, cv);
    unpack<T>(sn, sv);
    const bool lower = sub < LPK / 2;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const float partner = __shfl_xor(x[e], LPK / 2, 64);
      const float rot = lower ? -partner : partner;
      x[e] = round_to<T>(round_to<T>(x[e] * cv[e]) + round_to<T>(rot * sv[e]));
    }
  }
  return pack<T>(x);
}

// RMS norm without weights (x / sqrt(mean(x^2) + eps), float32 sums,
// rounded once to T).
template <typename T, int HD, int LPK>
__device__ __forceinline__ uint4 rms_unweighted(uint4 raw, float eps) {
  constexpr int EPL = Elem<T>::kPerVec;
  float x[EPL];
  unpack<T>(raw, x);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) ss = fmaf(x[e], x[e], ss);
  ss = group_sum<LPK>(ss);
  const float r = rsqrtf(ss * (1.f / HD) + eps);
#pragma unroll
  for (int e = 0; e < EPL; ++e) x[e] = round_to<T>(x[e] * r);
  return pack<T>(x);
}

// Online-softmax state of one stream for the G query heads of a kv head.
template <typename T, int HD, int G, int W>
struct Stream {
  using S = DecodeShape<T, HD, G, W>;
  static constexpr int EPL = S::kEPL;
  uint4 q[G];   // the lane's raw 16-byte slice of each query head
  float c;      // scale * log2(e), applied to the reduced score
  float m[G], l[G], o[G][EPL];

  // Starts the state from one key (k, v) when `mine`; the dot products run
  // on every lane (their reductions need the whole wave).
  __device__ __forceinline__ void seed(const uint4& k, const uint4& v, bool mine) {
    float vf[EPL];
    unpack<T>(v, vf);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float s = group_sum<S::kLPK>(dot16<T>(q[g], k)) * c;
      if (mine) {
        m[g] = s;
        l[g] = 1.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) o[g][e] = vf[e];
      }
    }
  }

  __device__ __forceinline__ void init() {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m[g] = kNegInf;
      l[g] = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) o[g][e] = 0.f;
    }
  }

  // Folds one load batch (raw 16-byte lane slices of K and V); key u is
  // valid when bit u of valid_mask is set.
  template <int U = S::kUnroll>
  __device__ __forceinline__ void consume(const uint4* kr, const uint4* vr, unsigned valid_mask) {
    float s[U][G];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float acc = group_sum<S::kLPK>(dot16<T>(q[g], kr[u]));
        s[u][g] = (valid_mask >> u) & 1u ? acc * c : kNegInf;
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

  // Merges the wave's streams (lane groups LPK apart) with a butterfly of
  // lane swaps (lane_pair: the Whisper steps 1-1.5% shorter than with
  // ds_bpermute shuffles, outputs bit-identical); afterwards the first group
  // (lanes 0 .. LPK - 1, the ones the workgroup merge reads) holds the
  // wave's state.
  template <int OFF>
  __device__ __forceinline__ void merge_from() {
    if constexpr (OFF < 64) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float m1, m2, l1, l2;
        lane_pair<OFF>(m[g], m1, m2);
        lane_pair<OFF>(l[g], l1, l2);
        const float mn = fmaxf(m1, m2);
        const float mu = mn == kNegInf ? 0.f : mn;
        const float w1 = fast_exp2(m1 - mu);
        const float w2 = fast_exp2(m2 - mu);
        l[g] = l1 * w1 + l2 * w2;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          float o1, o2;
          lane_pair<OFF>(o[g][e], o1, o2);
          o[g][e] = o1 * w1 + o2 * w2;
        }
        m[g] = mn;
      }
      merge_from<OFF * 2>();
    }
  }
  __device__ __forceinline__ void merge_wave() { merge_from<S::kLPK>(); }
};

// At most 128 VGPRs, so that four waves fit per SIMD (two 8-wave workgroups
// per CU).
//
// APPEND: the fused prologue of asrattn_decode_append.  q and the step's key
// are normalized and rotated in registers; the cache supplies keys
// 0 .. positions[b] - 1 and the new key/value join from registers (the last
// split folds them into its state); the first split writes them to the
// cache at positions[b].  No workgroup reads that slot, so splits need no
// ordering among themselves.
//
// SPEC (plain launches with one split, no window, key counts in device
// memory and a cache of at least eight first batches; paged, a first page
// that holds the whole first batch; the launch chooses it): the first load
// batch, keys 0 .. STEP - 1, is issued before the row's key count is read,
// from buffer resources that end at the cache's capacity (paged: at the
// first page's end, the page read from the block table meanwhile); once the
// count is known, keys at or past it are masked and their values zeroed
// (cache slots past a row's keys may hold anything).
// The masked keys then add exactly zero, as the zeros of a resource ending
// at the count do, so the output is the same bit for bit; the launch is
// one round trip shorter at its start (Qwen3's step: 22.74 -> 22.37 us per
// launch, same box).  The fused step (its prologue's loads already cover
// that round trip) measured 2% slower with it and does not take it.
//
// PB (paged, one split, no window, pages of at least one load batch; SPEC
// on a paged cache implies it): batches start at multiples of STEP, and the
// page size is a power of two >= STEP, so each batch lies in one page: one
// block-table read and one pair of buffer resources per batch instead of
// one per slice (Qwen3's paged step 23.6 -> 22.9 us per launch, same box;
// the same loads in the same order, so the same bits).
template <typename T, int HD, int G, int W, bool APPEND, bool PAGED, bool SPEC = false, bool PB = false>
__global__ __launch_bounds__(64 * W, (DecodeShape<T, HD, G, W>::kOcc)) void decode_kernel(const DecodeArgs a) {
  static_assert(!SPEC || !APPEND, "speculative first batch: plain launches");
  static_assert(!PB || PAGED, "page-sized batches: paged caches");
  using S = DecodeShape<T, HD, G, W>;
  constexpr int EPL = S::kEPL, LPK = S::kLPK, NS = S::kStreams;
  // Keys per stream per load batch.
  constexpr int U = APPEND ? S::kUnroll : S::kPlainUnroll;
  constexpr int STEP = NS * U;
  constexpr bool kPageBatch = PAGED && (SPEC || PB);
  const asrattn_decode_params& p = a.p;

  const int split = blockIdx.x;
  const int hkv = blockIdx.y;
  const int b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = lane % LPK;
  const int stream = wave * S::kKPW + lane / LPK;

  // K and V of this (sequence, kv head).
  const int64_t kbatch = PAGED ? 0 : (int64_t)b * p.k_batch_stride;
  const int64_t vbatch = PAGED ? 0 : (int64_t)b * p.v_batch_stride;
  const char* kbase =
      reinterpret_cast<const char*>(static_cast<const T*>(p.k) + kbatch + (int64_t)hkv * p.k_head_stride);
  const char* vbase =
      reinterpret_cast<const char*>(static_cast<const T*>(p.v) + vbatch + (int64_t)hkv * p.v_head_stride);
  const uint32_t kts = (uint32_t)(p.k_token_stride * (int64_t)sizeof(T));
  const uint32_t vts = (uint32_t)(p.v_token_stride * (int64_t)sizeof(T));
  const uint32_t lane_bytes = sub * EPL * (uint32_t)sizeof(T);

  // q is used raw (no unpacking), so its load latency overlaps the first
  // K/V batch's; it and the prologue's inputs load before the key count is
  // read, which none of them needs (Qwen3's step 21.4 -> 20.9 us per launch,
  // the fused step 23.1 -> 22.6).  SPEC issues the first K/V batch there
  // too; without the scheduling barrier below, the compiler moves the
  // count's load and its wait above those loads.
  Stream<T, HD, G, W> st;
  {
    const T* qp = static_cast<const T*>(p.q) + (int64_t)b * p.q_batch_stride +
                  (int64_t)hkv * G * p.q_head_stride + sub * EPL;
#pragma unroll
    for (int g = 0; g < G; ++g) st.q[g] = *reinterpret_cast<const uint4*>(qp + (int64_t)g * p.q_head_stride);
  }
  st.c = a.c;
  st.init();
  // The prologue's inputs load here, before the first K/V batch; its
  // arithmetic runs after that batch is issued.
  const asrattn_append_params& ap = a.ap;
  const bool has_norm = APPEND && ap.q_norm != nullptr;
  const bool has_vnorm = APPEND && ap.v_norm != 0;
  const bool has_rot = APPEND && ap.cos != nullptr;
  uint4 knew = {}, vnew = {}, qw = {}, kw = {}, cs = {}, sn = {};
  if constexpr (APPEND) {
    const T* knp = static_cast<const T*>(ap.k_new) + (int64_t)b * ap.kn_batch_stride + (int64_t)hkv * ap.kn_head_stride;
    const T* vnp = static_cast<const T*>(ap.v_new) + (int64_t)b * ap.vn_batch_stride + (int64_t)hkv * ap.vn_head_stride;
    // Absent weights or tables read k_new's slice instead (and are unused):
    // the loads stay unconditional, so no branch joins their registers and
    // forces a wait before the first K/V batch.
    const T* qwp = has_norm ? static_cast<const T*>(ap.q_norm) : knp;
    const T* kwp = has_norm ? static_cast<const T*>(ap.k_norm) : knp;
    const T* csp = has_rot ? static_cast<const T*>(ap.cos) + (int64_t)b * ap.rope_batch_stride : knp;
    const T* snp = has_rot ? static_cast<const T*>(ap.sin) + (int64_t)b * ap.rope_batch_stride : knp;
    knew = *reinterpret_cast<const uint4*>(knp + sub * EPL);
    vnew = *reinterpret_cast<const uint4*>(vnp + sub * EPL);
    qw = *reinterpret_cast<const uint4*>(qwp + sub * EPL);
    kw = *reinterpret_cast<const uint4*>(kwp + sub * EPL);
    cs = *reinterpret_cast<const uint4*>(csp + sub * EPL);
    sn = *reinterpret_cast<const uint4*>(snp + sub * EPL);
  }

  // Two register batches in ping-pong: the next batch is in flight while the
  // current one is consumed.
  uint4 ka[U], va[U], kb[U], vb[U];
  // Paged: pool page of logical page pi of this sequence, or -1 when the
  // entry is missing or outside the pool (its keys are skipped).
  const int32_t* bt = PAGED ? a.pk.block_table + (int64_t)b * a.pk.bt_stride : nullptr;
  auto pool_page = [&](int pi) -> int {
    if (pi >= a.pk.bt_stride) return -1;
    const int e = bt[__builtin_amdgcn_readfirstlane(pi)];
    return e >= 0 && e < a.pk.num_pages ? e : -1;
  };

  int page0 = 0;  // SPEC, paged: the sequence's first pool page (-1: none)
  if constexpr (SPEC) {
    // Slab: resources up to the cache's capacity.  Paged: over the first
    // page (the launch makes sure the batch fits in one).
    const char* kp = kbase;
    const char* vp = vbase;
    uint32_t keys = (uint32_t)p.max_len_k;
    if constexpr (PAGED) {
      page0 = pool_page(0);
      const int64_t pg = page0 >= 0 ? page0 : 0;
      kp = kbase + pg * a.pk.k_page_stride * (int64_t)sizeof(T);
      vp = vbase + pg * a.pk.v_page_stride * (int64_t)sizeof(T);
      keys = page0 >= 0 ? (uint32_t)a.pk.page_size : 0u;
    }
    const __amdgpu_buffer_rsrc_t kcap = buffer_rsrc(kp, keys * kts);
    const __amdgpu_buffer_rsrc_t vcap = buffer_rsrc(vp, keys * vts);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t j = (uint32_t)(u * NS + stream);
      ka[u] = buffer_load16_stream(kcap, j * kts + lane_bytes);
      va[u] = buffer_load16_stream(vcap, j * vts + lane_bytes);
    }
    __builtin_amdgcn_sched_barrier(0);  // the batch's issue stays above the count's load
  }

  const int64_t pos = APPEND ? p.positions[b] : 0;
  const int n = APPEND ? (int)min(max(pos, (int64_t)0), (int64_t)p.max_len_k)
                       : decode_key_count(p.seqused_k, p.positions, b, p.max_len_k);
  // Sliding window: the query sees its last `window` keys (with the append
  // variant the new key is one of them): cache keys kfirst .. n - 1.
  const int kfirst = p.window > 0 ? max(0, n + (APPEND ? 1 : 0) - p.window) : 0;
  // Paged: splits start NS-aligned (slices stay inside pages); keys before
  // kfirst are masked.
  const int kbeg = PAGED ? kfirst / NS * NS : kfirst;
  int chunk = (n - kbeg + a.splits - 1) / a.splits;
  if constexpr (PAGED) chunk = (chunk + NS - 1) / NS * NS;
  const int k0 = min(n, kbeg + split * chunk);
  const int k1 = min(n, k0 + chunk);

  // Buffer resources that end at the split's last key: loads past it return
  // zeros without a branch, so the two load batches stay in flight across
  // the loop.  (Paged: the pool, past the sequence's first page.)
  const __amdgpu_buffer_rsrc_t krs = buffer_rsrc(kbase, (uint32_t)k1 * kts);
  const __amdgpu_buffer_rsrc_t vrs = buffer_rsrc(vbase, (uint32_t)k1 * vts);

  // Key u of the batch starting at `base` is base + u * NS + stream.
  auto load = [&](uint4* kr, uint4* vr, int base) -> unsigned {
    unsigned mask = 0;
    // kPageBatch: the batch's page, its first key and its resources.
    int bfirst = 0, bpage = -1;
    __amdgpu_buffer_rsrc_t kb_rs = krs, vb_rs = vrs;
    if constexpr (kPageBatch) {
      const int pi = base >> a.page_shift;
      bfirst = pi << a.page_shift;
      bpage = pool_page(pi);
      const uint32_t keys = bpage >= 0 ? (uint32_t)min(max(k1 - bfirst, 0), a.pk.page_size) : 0u;
      const int64_t pg = bpage >= 0 ? bpage : 0;
      kb_rs = buffer_rsrc(kbase + pg * a.pk.k_page_stride * (int64_t)sizeof(T), keys * kts);
      vb_rs = buffer_rsrc(vbase + pg * a.pk.v_page_stride * (int64_t)sizeof(T), keys * vts);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = base + u * NS + stream;
      if constexpr (kPageBatch) {
        kr[u] = buffer_load16_stream(kb_rs, (uint32_t)(j - bfirst) * kts + lane_bytes);
        vr[u] = buffer_load16_stream(vb_rs, (uint32_t)(j - bfirst) * vts + lane_bytes);
        mask |= (j < k1 && j >= kfirst && bpage >= 0 ? 1u : 0u) << u;
      } else if constexpr (PAGED) {
        const int j0 = base + u * NS;  // uniform; the slice lies in one page
        const int pi = j0 >> a.page_shift;
        const int first = pi << a.page_shift;
        const int page = pool_page(pi);
        const uint32_t keys = page >= 0 ? (uint32_t)min(max(k1 - first, 0), a.pk.page_size) : 0u;
        const int64_t pg = page >= 0 ? page : 0;
        const __amdgpu_buffer_rsrc_t kp = buffer_rsrc(kbase + pg * a.pk.k_page_stride * (int64_t)sizeof(T), keys * kts);
        const __amdgpu_buffer_rsrc_t vp = buffer_rsrc(vbase + pg * a.pk.v_page_stride * (int64_t)sizeof(T), keys * vts);
        kr[u] = buffer_load16_stream(kp, (uint32_t)(j - first) * kts + lane_bytes);
        vr[u] = buffer_load16_stream(vp, (uint32_t)(j - first) * vts + lane_bytes);
        mask |= (j < k1 && j >= kfirst && page >= 0 ? 1u : 0u) << u;
      } else {
        kr[u] = buffer_load16_stream(krs, (uint32_t)j * kts + lane_bytes);
        vr[u] = buffer_load16_stream(vrs, (uint32_t)j * vts + lane_bytes);
        mask |= (j < k1 ? 1u : 0u) << u;
      }
    }
    return mask;
  };

  // The first batch is issued unconditionally: with k0 >= k1 its offsets all
  // lie past the resource's end and read zeros.  SPEC's was issued above
  // (k0 = 0 with one split and no window); it is masked here.
  unsigned mb = 0;
  unsigned ma = 0;
  if constexpr (SPEC) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool valid = u * NS + stream < k1 && page0 >= 0;
      ma |= (valid ? 1u : 0u) << u;
      if (!valid) va[u] = make_uint4(0u, 0u, 0u, 0u);
    }
  } else {
    ma = load(ka, va, k0);
  }
  if constexpr (APPEND) {
    __builtin_amdgcn_sched_barrier(0);  // keep the prologue below the batch's issue
#pragma unroll
    for (int g = 0; g < G; ++g) st.q[g] = norm_rotate<T, HD, LPK>(st.q[g], has_norm, qw, has_rot, cs, sn, ap.eps, sub);
    knew = norm_rotate<T, HD, LPK>(knew, has_norm, kw, has_rot, cs, sn, ap.eps, sub);
    if (has_vnorm) vnew = rms_unweighted<T, HD, LPK>(vnew, ap.eps);
    st.seed(knew, vnew, split == a.splits - 1 && stream == 0);
  }
  for (int base = k0; base < k1; base += 2 * STEP) {
    mb = load(kb, vb, base + STEP);
    st.template consume<U>(ka, va, ma);
    if (base + STEP >= k1) break;
    ma = load(ka, va, base + 2 * STEP);
    st.template consume<U>(kb, vb, mb);
  }

  if constexpr (APPEND) {
    if (split == 0 && stream == 0 && pos >= 0 && pos < p.max_len_k) {
      int64_t koff = pos * kts, voff = pos * vts;
      bool write = true;
      if constexpr (PAGED) {
        const int pi = (int)(pos >> a.page_shift);
        const int page = pool_page(pi);
        const int64_t slot = pos - ((int64_t)pi << a.page_shift);
        write = page >= 0;
        koff = (int64_t)page * a.pk.k_page_stride * (int64_t)sizeof(T) + slot * kts;
        voff = (int64_t)page * a.pk.v_page_stride * (int64_t)sizeof(T) + slot * vts;
      }
      if (write) {
        *reinterpret_cast<uint4*>(const_cast<char*>(kbase) + koff + lane_bytes) = knew;
        *reinterpret_cast<uint4*>(const_cast<char*>(vbase) + voff + lane_bytes) = vnew;
      }
    }
  }

  st.merge_wave();

  // Merge the waves in LDS.
  __shared__ float sm_m[W][G];
  __shared__ float sm_l[W][G];
  __shared__ float sm_o[W][G][HD];
  if (lane < LPK) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (lane == 0) {
        sm_m[wave][g] = st.m[g];
        sm_l[wave][g] = st.l[g];
      }
#pragma unroll
      for (int e = 0; e < EPL; ++e) sm_o[wave][g][sub * EPL + e] = st.o[g][e];
    }
  }
  __syncthreads();

  for (int t = threadIdx.x; t < G * HD; t += S::kThreads) {
    const int g = t / HD;
    const int d = t % HD;
    float mx = kNegInf;
#pragma unroll
    for (int w = 0; w < W; ++w) mx = fmaxf(mx, sm_m[w][g]);
    const float mxu = mx == kNegInf ? 0.f : mx;
    float lsum = 0.f, osum = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float wt = fast_exp2(sm_m[w][g] - mxu);
      lsum = fmaf(sm_l[w][g], wt, lsum);
      osum = fmaf(sm_o[w][g][d], wt, osum);
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
  float lsum = 0.f, osum = 0.f;
  constexpr int kBatch = 8;  // splits whose partials are loaded in one round trip
  if (a.splits <= kBatch) {
    float m[kBatch], l[kBatch], o[kBatch];
#pragma unroll
    for (int s = 0; s < kBatch; ++s) {
      const int t = min(s, a.splits - 1);  // surplus slots repeat the last split, weighted 0
      m[s] = a.ws_ml[(idx0 + t) * 2];
      l[s] = a.ws_ml[(idx0 + t) * 2 + 1];
      o[s] = a.ws_o[(idx0 + t) * HD + d];
    }
    float mx = kNegInf;
#pragma unroll
    for (int s = 0; s < kBatch; ++s) mx = fmaxf(mx, m[s]);
    const float mxu = mx == kNegInf ? 0.f : mx;
#pragma unroll
    for (int s = 0; s < kBatch; ++s) {
      const float w = s < a.splits ? fast_exp2(m[s] - mxu) : 0.f;
      lsum = fmaf(l[s], w, lsum);
      osum = fmaf(o[s], w, osum);
    }
  } else {
    float mx = kNegInf;
    for (int s = 0; s < a.splits; ++s) mx = fmaxf(mx, a.ws_ml[(idx0 + s) * 2]);
    const float mxu = mx == kNegInf ? 0.f : mx;
    for (int s = 0; s < a.splits; ++s) {
      const float w = fast_exp2(a.ws_ml[(idx0 + s) * 2] - mxu);
      lsum = fmaf(a.ws_ml[(idx0 + s) * 2 + 1], w, lsum);
      osum = fmaf(a.ws_o[(idx0 + s) * HD + d], w, osum);
    }
  }
  T* op = static_cast<T*>(p.out) + (int64_t)b * p.o_batch_stride + (int64_t)hq * p.o_head_stride + d;
  Elem<T>::store1(op, lsum > 0.f ? osum / lsum : 0.f);
}

template <typename T, int HD, int G, int W>
hipError_t launch_typed(const DecodeArgs& a, bool append, hipStream_t stream) {
  const asrattn_decode_params& p = a.p;
  dim3 grid(a.splits, p.heads_kv, p.batch);
  const bool paged = a.pk.block_table != nullptr;
  // Key counts read from device memory, one split, no window, and a cache
  // of at least eight first batches: the first batch need not wait for the
  // count (SPEC).  Its resource ends at the capacity, not at the count, so a
  // batch as wide as the cache reads keys the row does not have: Whisper's
  // self-attention over a 256-key bucket, one 256-key batch, read 2.3x its
  // bytes and ran 3% slower with it.
  constexpr int kFirstBatch = DecodeShape<T, HD, G, W>::kPlainStep;
  const bool spec = !append && a.splits == 1 && p.window <= 0 &&
                    (p.seqused_k != nullptr || p.positions != nullptr) && p.max_len_k >= 8 * kFirstBatch &&
                    (!paged || a.pk.page_size >= kFirstBatch);
  // Paged appending steps whose batches each lie in one page (PB; the plain
  // steps get it with SPEC).
  const bool page_batch = paged && a.splits == 1 && p.window <= 0 &&
                          a.pk.page_size >= DecodeShape<T, HD, G, W>::kStep;
  if (append && paged && page_batch)
    hipLaunchKernelGGL((decode_kernel<T, HD, G, W, true, true, false, true>), grid, dim3(64 * W), 0, stream, a);
  else if (append && paged)
    hipLaunchKernelGGL((decode_kernel<T, HD, G, W, true, true>), grid, dim3(64 * W), 0, stream, a);
  else if (append)
    hipLaunchKernelGGL((decode_kernel<T, HD, G, W, true, false>), grid, dim3(64 * W), 0, stream, a);
  else if (paged && spec)
    hipLaunchKernelGGL((decode_kernel<T, HD, G, W, false, true, true>), grid, dim3(64 * W), 0, stream, a);
  else if (paged)
    hipLaunchKernelGGL((decode_kernel<T, HD, G, W, false, true>), grid, dim3(64 * W), 0, stream, a);
  else if (spec)
    hipLaunchKernelGGL((decode_kernel<T, HD, G, W, false, false, true>), grid, dim3(64 * W), 0, stream, a);
  else
    hipLaunchKernelGGL((decode_kernel<T, HD, G, W, false, false>), grid, dim3(64 * W), 0, stream, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || a.splits == 1) return err;
  hipLaunchKernelGGL((decode_combine_kernel<T, HD>), dim3(p.heads_q, p.batch), dim3(HD), 0, stream, a);
  return hipGetLastError();
}

// waves: 4, 8 or 16, lowered to what the merge's LDS allows.
template <typename T, int HD, int G>
hipError_t launch_waves(const DecodeArgs& a, int waves, bool append, hipStream_t stream) {
  if constexpr (DecodeShape<T, HD, G, 16>::kFits) {
    if (waves >= 16) return launch_typed<T, HD, G, 16>(a, append, stream);
  }
  if constexpr (DecodeShape<T, HD, G, 8>::kFits) {
    if (waves >= 8) return launch_typed<T, HD, G, 8>(a, append, stream);
  }
  static_assert(DecodeShape<T, HD, G, 4>::kFits, "four waves fit");
  return launch_typed<T, HD, G, 4>(a, append, stream);
}

template <typename T, int HD>
hipError_t launch_hd(const DecodeArgs& a, int group, int waves, bool append, hipStream_t stream) {
  switch (group) {
    case 1: return launch_waves<T, HD, 1>(a, waves, append, stream);
    case 2: return launch_waves<T, HD, 2>(a, waves, append, stream);
    case 4: return launch_waves<T, HD, 4>(a, waves, append, stream);
    case 8: return launch_waves<T, HD, 8>(a, waves, append, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace
}  // namespace asrattn
