// Inner loops shared by the split-K linears and the LM head (gfx950).
#pragma once
#include "common.h"

// One 64-wide k group of a q4 tile-32 weight for NT n-tiles (see q4_linear.hip
// for the layout and the exact-integer B construction).
//   a[t], al[t] : ACT_F16P hi / lo fragments of this lane's row, words t = 0..3
//   xsr[r]      : group sums (hi + lo) of the 16 rows this lane holds in the result
template <int NT>
DRT_DEV void q4_group_mma(f32x16 (&acc)[NT], const f16x8 (&a)[4], const f16x8 (&al)[4],
                          const float (&xsr)[16], const u32x4 (&w)[NT],
                          const uint32_t (&sbv)[NT]) {
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    f32x16 c = f32x16{};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t wt = w[j][t];
      u32x4 bw;
      bw[0] = q4_pair_to_f16((wt >> 0) & 0x000F000Fu);
      bw[1] = q4_pair_to_f16((wt >> 4) & 0x000F000Fu);
      bw[2] = q4_pair_to_f16((wt >> 8) & 0x000F000Fu);
      bw[3] = q4_pair_to_f16((wt >> 12) & 0x000F000Fu);
      const f16x8 b = __builtin_bit_cast(f16x8, bw);
      c = mfma_f16(a[t], b, c);
      c = mfma_f16(al[t], b, c);
    }
    const float s = bf16_bits_to_float(sbv[j] & 0xffffu);
    const float b = bf16_bits_to_float(sbv[j] >> 16);
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = fmaf(s, c[r], fmaf(b, xsr[r], acc[j][r]));
  }
}

// Address helpers of the device weight layouts.
DRT_DEV const u32x4* q4_tile_words(const uint32_t* qw, int64_t nt, int G, int g, int lane) {
  return (const u32x4*)(qw + (((nt * G + g) * 64) + lane) * 4);
}
DRT_DEV uint32_t q4_tile_sb(const uint32_t* sb, int64_t nt, int G, int g, int lane) {
  return sb[(nt * G + g) * 32 + (lane & 31)];
}
// bf16 tile layout: wb[((nt*KC + kc)*64 + l)*8 + e] = W[32nt + (l&31)][16kc + 8(l>>5) + e]
DRT_DEV const bf16x8* bf16_tile_frag(const uint16_t* wb, int64_t nt, int KC, int kc, int lane) {
  return (const bf16x8*)(wb + (((nt * KC + kc) * 64) + lane) * 8);
}
