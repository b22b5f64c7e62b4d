// Device helpers shared by the linear kernels (fused_linear.hip, skinny_linear.hip).
#pragma once
#include "fused.h"

namespace {

DRT_DEV void q4_group_mma1(f32x16& acc, const f16x8 (&a)[4], const float (&xsr)[16],
                           const u32x4 w, const uint32_t sbv) {
  f32x16 c = f32x16{};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t wt = w[t];
    u32x4 bw;
    bw[0] = (wt & 0x000F000Fu) | 0x64006400u;
    bw[1] = ((wt >> 4) & 0x000F000Fu) | 0x64006400u;
    bw[2] = ((wt >> 8) & 0x000F000Fu) | 0x64006400u;
    bw[3] = ((wt >> 12) & 0x000F000Fu) | 0x64006400u;
    c = mfma_f16(a[t], __builtin_bit_cast(f16x8, bw), c);
  }
  const float s = bf16_bits_to_float(sbv & 0xffffu);
  const float b = bf16_bits_to_float(sbv >> 16);
  const float bp = fmaf(-1024.f, s, b);
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = fmaf(s, c[r], fmaf(bp, xsr[r], acc[r]));
}

// Same as q4_group_mma1 with the group sum of each row computed here from the
// A fragments (lane l holds 32 of the 64 values of row l & 31; the two halves
// are added by one shuffle) and fetched by shuffle as the rows are consumed.
DRT_DEV void q4_group_mma1_lane(f32x16& acc, const u32x4 (&a)[4], const u32x4 w,
                                const uint32_t sbv, int lane) {
  float xs_lane = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const f16x8 h = __builtin_bit_cast(f16x8, a[t]);
#pragma unroll
    for (int e = 0; e < 8; ++e) xs_lane += (float)h[e];
  }
  xs_lane += __shfl_xor(xs_lane, 32, 64);
  f32x16 c = f32x16{};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t wt = w[t];
    u32x4 bw;
    bw[0] = (wt & 0x000F000Fu) | 0x64006400u;
    bw[1] = ((wt >> 4) & 0x000F000Fu) | 0x64006400u;
    bw[2] = ((wt >> 8) & 0x000F000Fu) | 0x64006400u;
    bw[3] = ((wt >> 12) & 0x000F000Fu) | 0x64006400u;
    c = mfma_f16(__builtin_bit_cast(f16x8, a[t]), __builtin_bit_cast(f16x8, bw), c);
  }
  const float s = bf16_bits_to_float(sbv & 0xffffu);
  const float b = bf16_bits_to_float(sbv >> 16);
  const float bp = fmaf(-1024.f, s, b);
#pragma unroll
  for (int r = 0; r < 16; ++r)
    acc[r] = fmaf(s, c[r], fmaf(bp, __shfl(xs_lane, mfma_row(r, lane), 64), acc[r]));
}

template <typename T> DRT_DEV T cvt_to(float f);
template <> DRT_DEV _Float16 cvt_to<_Float16>(float f) { return (_Float16)f; }
template <> DRT_DEV __bf16 cvt_to<__bf16>(float f) {
  return __builtin_bit_cast(__bf16, float_to_bf16_bits(f));
}

// Epilogue of one head: x0/x1 are this lane's elements l and l + 64 of row m.
template <typename T>
DRT_DEV void qkv_head_store(const FusedArgs& a, int head, int m, int pos, float x0, float x1,
                            int lane) {
  const int Hq = a.Hq, Hkv = a.Hkv;
  const bool is_q = head < Hq, is_k = !is_q && head < Hq + Hkv;
  if (is_q || is_k) {
    const uint16_t* nw = is_q ? a.q_norm : a.k_norm;
    if (nw) {
      const float ms = wave_sum(x0 * x0 + x1 * x1) / 128.f;
      const float inv = 1.f / sqrtf(ms + a.eps);
      x0 = (x0 * inv) * bf16_bits_to_float(nw[lane]);
      x1 = (x1 * inv) * bf16_bits_to_float(nw[lane + 64]);
    }
    const float c = a.rope_cos[(int64_t)pos * 64 + lane];
    const float s = a.rope_sin[(int64_t)pos * 64 + lane];
    const float r0 = x0 * c - x1 * s;
    const float r1 = x1 * c + x0 * s;
    x0 = r0;
    x1 = r1;
  }
  if (is_q) {
    T* qo = (T*)a.q_out + ((int64_t)m * Hq + head) * 128;
    qo[lane] = cvt_to<T>(x0);
    qo[lane + 64] = cvt_to<T>(x1);
    return;
  }
  const int kvh = is_k ? head - Hq : head - Hq - Hkv;
  T* tile = (T*)a.kv_layer + (int64_t)kvh * a.kv_head_stride + (int64_t)(pos >> 5) * 8192;
  const int kk = pos & 31;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int hd = lane + 64 * e;
    const float val = e ? x1 : x0;
    if (is_k) {
      tile[(((hd >> 4) * 2 + ((hd >> 3) & 1)) * 32 + kk) * 8 + (hd & 7)] = cvt_to<T>(val);
    } else {
      const int q16 = kk & 15;
      tile[4096 + ((((hd >> 5) * 2 + (kk >> 4)) * 2 + ((q16 >> 2) & 1)) * 32 + (hd & 31)) * 8 +
           (q16 & 3) + 4 * (q16 >> 3)] = cvt_to<T>(val);
    }
  }
}

}  // namespace
