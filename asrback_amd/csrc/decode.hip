// Decoder-step attention: kernel choice and launch (the kernels live in
// decode_kernels.hpp, instantiated per element type in decode_bf16.hip and
// decode_f32.hip).
#include "decode_args.hpp"
#include "kernels.hpp"

namespace asrattn {

bool decode_supported(int dtype, int head_dim, int group) {
  const bool dt = dtype == ASRATTN_F32 || dtype == ASRATTN_BF16;
  // A key row is read by at most one wave: 64 lanes x 16 bytes.
  const bool hd = head_dim == 64 || head_dim == 128 || head_dim == 256 || (head_dim == 512 && dtype == ASRATTN_BF16);
  const bool g = group == 1 || group == 2 || group == 4 || group == 8;
  return dt && hd && g;
}

int decode_keys_per_wave(int dtype, int head_dim) {
  return 64 / (head_dim * (dtype == ASRATTN_BF16 ? 2 : 4) / 16);
}

int decode_waves(const asrattn_decode_params& p, int splits, int page_size) {
  // About 2048 waves over the grid (two per SIMD): on one MI355X, Qwen3's
  // 512 workgroups ran 6% faster on 4 waves than on 8, Gemma 4's 256 5%
  // faster on 8 than on 16, Whisper's 192 the same on 8 and 16.  No more
  // waves than one load batch of the split's keys needs (Whisper's 256-key
  // self-attention bucket: 8 waves, 4% faster than 16).
  const long long groups = (long long)p.batch * p.heads_kv * splits;
  const int keys_per_split = (p.max_len_k + splits - 1) / splits;
  int waves = 16;
  while (waves > 4 && groups * waves > 2048) waves /= 2;
  // A wave loads 64 / LPK rows per instruction (8 for bf16 x 64, 4 for 128),
  // and a batch takes 4 of them (2 with four or more query heads per kv
  // head, or head_dim 256 and up: DecodeShape::kUnroll).
  const int rows_per_wave = 64 / (p.head_dim * (p.dtype == ASRATTN_BF16 ? 2 : 4) / 16);
  const int group = p.heads_q / p.heads_kv;
  const int unroll = group >= 4 || p.head_dim >= 256 ? 2 : 4;
  while (waves > 4 && waves * rows_per_wave * unroll > keys_per_split) waves /= 2;
  // Paged: a slice (one key per stream of the workgroup) within one page.
  while (page_size > 0 && waves > 4 && waves * rows_per_wave > page_size) waves /= 2;
  return waves;
}

hipError_t launch_decode(const asrattn_decode_params& p, const asrattn_append_params* append,
                         const asrattn_paged_kv* paged, int splits, float* ws_o, float* ws_ml, hipStream_t stream) {
  DecodeArgs a;
  a.p = p;
  a.ap = append != nullptr ? *append : asrattn_append_params{};
  a.pk = paged != nullptr ? *paged : asrattn_paged_kv{};
  a.page_shift = 0;
  while (paged != nullptr && (1 << a.page_shift) < paged->page_size) ++a.page_shift;
  const bool app = append != nullptr;
  a.ws_o = ws_o;
  a.ws_ml = ws_ml;
  a.splits = splits;
  a.c = p.scale * kLog2e;
  const int group = p.heads_q / p.heads_kv;
  const int waves = decode_waves(p, splits, paged != nullptr ? paged->page_size : 0);
  return p.dtype == ASRATTN_BF16 ? launch_decode_bf16(a, p.head_dim, group, waves, app, stream)
                                 : launch_decode_f32(a, p.head_dim, group, waves, app, stream);
}

}  // namespace asrattn
