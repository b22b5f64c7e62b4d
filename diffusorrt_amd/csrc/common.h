// Shared device-side helpers for the gfx950 (CDNA4) kernels of the denoise step.
//
// Conventions used by every kernel in this library:
//  * wave64; MFMA v_mfma_f32_32x32x16_{f16,bf16}: lane l supplies A row (l & 31)
//    and B column (l & 31), each with 8 k-slots [8*(l>>5), 8*(l>>5)+8); the
//    32x32 fp32 result leaves lane l holding column (l & 31) of rows
//    8*(r>>2) + 4*(l>>5) + (r & 3) for r = 0..15.
//  * Any permutation of the k-slots is harmless as long as A and B use the same
//    one; the q4 and attention layouts below exploit that to make every lane's
//    loads 16-byte contiguous and every wave instruction a contiguous 1 KiB.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define DRT_DEV __device__ __forceinline__

DRT_DEV f32x16 mfma_f16(const f16x8 a, const f16x8 b, const f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
DRT_DEV f32x16 mfma_bf16(const bf16x8 a, const bf16x8 b, const f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Row of the 32x32 MFMA result held in accumulator r by this lane.
DRT_DEV int mfma_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

DRT_DEV float bf16_bits_to_float(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// float -> bf16 bits, round to nearest even (NaN kept quiet).
DRT_DEV uint16_t float_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
DRT_DEV float round_bf16(float f) { return bf16_bits_to_float(float_to_bf16_bits(f)); }

DRT_DEV uint16_t half_bits(_Float16 h) { return __builtin_bit_cast(uint16_t, h); }
// a in bits 0-15, b in bits 16-31
DRT_DEV uint32_t pack_half2(_Float16 a, _Float16 b) {
  return (uint32_t)half_bits(a) | ((uint32_t)half_bits(b) << 16);
}

// Wave-level reductions (64 lanes) via cross-lane shuffles.
DRT_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
DRT_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
DRT_DEV double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Activation formats written by producers and read by the linear kernels.
//  ACT_F16P: an fp32 value x carried as two fp16 planes of [M][K] each, hi =
//    fp16(x) first, then lo = fp16(x - hi) at + M*K elements (x - hi is exact in
//    fp32, so hi + lo holds x to about 22 significant bits); each 8-element chunk
//    of a row stored in the order (0,4,1,5,2,6,3,7). Group sums, where a
//    producer writes them, are fp32 sums of hi + lo over 64-wide k groups.
//  ACT_BF16: bf16, natural order (bf16-weight linears: the reference rounds
//    their inputs to bf16 itself).
enum ActFmt : int {
  ACT_F16P = 0,
  ACT_BF16 = 1,
};

// hi/lo fp16 pair of a float (ACT_F16P, and the Q planes of the attention)
DRT_DEV _Float16 f16_lo(float x, _Float16 hi) { return (_Float16)(x - (float)hi); }
template <typename T> DRT_DEV T lo_part(float x, T hi);
template <> DRT_DEV _Float16 lo_part<_Float16>(float x, _Float16 hi) { return f16_lo(x, hi); }
template <> DRT_DEV __bf16 lo_part<__bf16>(float x, __bf16 hi) {
  const float r = x - bf16_bits_to_float(__builtin_bit_cast(uint16_t, hi));
  return __builtin_bit_cast(__bf16, float_to_bf16_bits(r));
}

// Bit set in the runtime's error word when a producer met a value beyond the
// fp16 range (|x| >= 65520 rounds to infinity): the forward's results are not
// valid and the host reports it.
constexpr int DRT_ERR_F16_RANGE = 4;
DRT_DEV bool f16_overflows(float x) { return !(fabsf(x) < 65504.f); }

// Scale c of a row's pre-scaled norm input (the split-K q4 path: a residual
// update writes w * h * c as fp16 hi / lo planes for the next RMSNorm, and the
// linear that reads them multiplies its output rows by rinv / c): the largest
// power of two <= the row's norm factor rinv (exact to apply and to undo), over
// 16, so the planes stay 16-32x below the normalised values unless the row's
// RMS grew more than 16-fold since rinv was measured.
DRT_DEV float pre_scale_of(float rinv) {
  return __uint_as_float(__float_as_uint(rinv) & 0x7f800000u) * 0.0625f;
}

// Two q4 nibbles at bits 0-3 and 16-19 of w as a pair of exact fp16 integers
// q: the nibble placed under the exponent of 1024 is the fp16 1024 + q, and one
// packed fp16 subtraction of 1024 (exact) leaves q.
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
DRT_DEV uint32_t q4_pair_to_f16(uint32_t w) {
  const f16x2 k = {(_Float16)-1024.f, (_Float16)-1024.f};
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, w | 0x64006400u) + k);
}

// The constants of q4_word_to_f16x8 held in registers (VOP3 forms take no
// literal operand on gfx9, so literals would cost a separate and + or each).
struct Q4Consts {
  uint32_t magic, n1024, sixteenth, n64;
};
DRT_DEV Q4Consts q4_consts() {
  uint32_t m = 0x64006400u, a = 0xE400E400u, s = 0x2C002C00u, b = 0xD400D400u;
  asm volatile("" : "+v"(m), "+s"(a), "+s"(s), "+v"(b));
  return Q4Consts{m, a, s, b};
}

// One q4 weight word (nibbles n0..n7, n0 lowest) as the fp16 B fragment
// (n0, n4, n1, n5, n2, n6, n3, n7), the element order of four q4_pair_to_f16
// calls on w, w >> 4, w >> 8, w >> 12, in 9 instructions instead of 15: the
// nibbles at bits 4-7 / 20-23 are placed one position higher under the
// exponent of 1024 (fp16 1024 + 16 q), which one packed fma with 1/16 and -64
// turns into q (exact: (1024 + 16 q) / 16 - 64 = q, one rounding of an exact
// value).
DRT_DEV u32x4 q4_word_to_f16x8(uint32_t w, const Q4Consts& k) {
  const uint32_t w8 = w >> 8;
  const f16x2 n1024 = __builtin_bit_cast(f16x2, k.n1024);
  const f16x2 s16 = __builtin_bit_cast(f16x2, k.sixteenth);
  const f16x2 n64 = __builtin_bit_cast(f16x2, k.n64);
  u32x4 r;
  r[0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, (w & 0x000F000Fu) | k.magic) + n1024);
  r[1] = __builtin_bit_cast(
      uint32_t,
      __builtin_elementwise_fma(__builtin_bit_cast(f16x2, (w & 0x00F000F0u) | k.magic), s16, n64));
  r[2] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, (w8 & 0x000F000Fu) | k.magic) + n1024);
  r[3] = __builtin_bit_cast(
      uint32_t,
      __builtin_elementwise_fma(__builtin_bit_cast(f16x2, (w8 & 0x00F000F0u) | k.magic), s16, n64));
  return r;
}

// Position of element k within an ACT_F16P row: chunk order (0,4,1,5,2,6,3,7).
DRT_DEV int f16p_index(int k) {
  const int j = k & 7;
  return (k & ~7) | ((j & 3) << 1) | (j >> 2);
}

// Per-forward parameters read by the kernels from device memory, so that one
// captured HIP graph can serve every decode step (the host rewrites this small
// struct before each replay; shapes stay fixed).
struct StepDesc {
  int32_t row0;             // absolute position of row 0 of this forward
  int32_t n_rows;           // rows forwarded
  int32_t n_keys;           // keys [0, n_keys) are attended
  int32_t n_lm;             // LM-head rows (<= 32 per tile)
  int32_t mask_kind;        // 0 none, 1 d2f_hybrid
  int32_t mask_prompt_len;
  int32_t mask_block;
  int32_t step;             // sampling forward index
  uint64_t seed;
  float temperature;
  int32_t exclude_col;      // vocabulary column left out of the scoring (-1: none)
  // rows [row0, row0 + seg_rows) form a first mask segment that sees only keys
  // [0, row0 + seg_rows); the rest see [0, n_keys) (0: one segment)
  int32_t seg_rows;
  // the fixed-quota choice made on the device after the LM head: this many of
  // the n_lm LM rows whose canvas token is still the mask take their proposed
  // token (highest scores first, equal scores lower row first; 0: none)
  int32_t quota;
};
// Entries of a device block's quota table (indexed by step modulo this; a block
// runs fewer steps).
constexpr int QUOTA_TAB = 64;
