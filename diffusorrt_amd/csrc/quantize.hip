// 4-bit affine group-64 quantization of a linear weight on the device: the
// load-time step that turns a package's floating-point projection weights into
// the QuantizedWeight bundle of backends/mlx_ops.py:63-94 (`mx.quantize(w,
// group_size=64, bits=4)`, run once per load by backends/mlx_dream.py:2073-2108).
//
// Per group of 64 weights along K (the values first rounded to bf16, the
// resident weight dtype of the q4 configurations), in fp32:
//   scale = max((w_max - w_min) / 15, 1e-7)
//   the edge is the extreme of larger magnitude: w_min (scale > 0) when
//   |w_min| > |w_max|, else w_max (scale negated);
//   q0 = round(edge / scale); unless q0 == 0, scale = edge / q0 and bias = edge
//   (so the edge value sits exactly on the grid), else bias = 0;
//   q = clamp(round((w - bias) / scale), 0, 15)   (round: half away from zero)
// then scale and bias are stored as bf16 (round to nearest even). This is MLX's
// published affine quantization (mlx 0.31, the version the reference pins); fp32
// division is IEEE (correctly rounded) here.
//
// Output is the MLX packing: w_q[N][K/8] uint32 (word j of row n holds
// k = 8j..8j+7, low nibble first), scales/biases[N][K/64] bf16.
//
// One thread per output word (8 weights: one 16-byte bf16 load, or two for fp32
// input), eight consecutive lanes per group, so loads and word stores are fully
// coalesced; the group's min/max are three xor exchanges.
#include "common.h"
#include "launch.h"

namespace {

__global__ __launch_bounds__(256) void q4_quantize_kernel(const void* __restrict__ w, int w_f32,
                                                          uint32_t* __restrict__ w_q,
                                                          uint16_t* __restrict__ scales,
                                                          uint16_t* __restrict__ biases,
                                                          int64_t n_words) {
  const int64_t word = (int64_t)blockIdx.x * 256 + threadIdx.x;
  // the grid covers whole groups (n_words is a multiple of 8 and so is every
  // block's first word), so all eight lanes of a group are live or none is
  if (word >= n_words) return;
  float v[8];
  if (w_f32) {
    const f32x4* p = (const f32x4*)((const float*)w + word * 8);
    const f32x4 a = p[0], b = p[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = round_bf16(a[i]);
      v[4 + i] = round_bf16(b[i]);
    }
  } else {
    const u32x4 r = *(const u32x4*)((const uint16_t*)w + word * 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = bf16_bits_to_float(r[i] & 0xffffu);
      v[2 * i + 1] = bf16_bits_to_float(r[i] >> 16);
    }
  }
  float mx = v[0], mn = v[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) {
    mx = fmaxf(mx, v[i]);
    mn = fminf(mn, v[i]);
  }
#pragma unroll
  for (int x = 1; x < 8; x <<= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, x, 64));
    mn = fminf(mn, __shfl_xor(mn, x, 64));
  }
  float scale = fmaxf((mx - mn) / 15.f, 1e-7f);
  const bool side = fabsf(mn) > fabsf(mx);
  scale = side ? scale : -scale;
  const float edge = side ? mn : mx;
  const float q0 = roundf(edge / scale);
  const bool at_zero = q0 == 0.f;
  scale = at_zero ? scale : edge / q0;
  const float bias = at_zero ? 0.f : edge;
  uint32_t out = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float q = fminf(fmaxf(roundf((v[i] - bias) / scale), 0.f), 15.f);
    out |= (uint32_t)q << (4 * i);
  }
  w_q[word] = out;
  if ((threadIdx.x & 7) == 0) {
    scales[word >> 3] = float_to_bf16_bits(scale);
    biases[word >> 3] = float_to_bf16_bits(bias);
  }
}

}  // namespace

namespace drt {

void q4_quantize(const void* w, bool w_f32, int N, int K, uint32_t* w_q, uint16_t* scales,
                 uint16_t* biases, hipStream_t s) {
  require(N > 0 && K > 0 && K % 64 == 0, "q4 quantization needs K % 64 == 0");
  const int64_t n_words = (int64_t)N * (K / 8);
  const int64_t blocks = (n_words + 255) / 256;
  require(blocks <= 0x7fffffff, "weight too large for one quantization launch");
  hipLaunchKernelGGL(q4_quantize_kernel, dim3((unsigned)blocks), dim3(256), 0, s, w, (int)w_f32,
                     w_q, scales, biases, n_words);
  DRT_HIP(hipGetLastError());
}

}  // namespace drt
