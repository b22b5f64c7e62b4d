// 4-bit affine group-64 quantized linear (MLX packing) for gfx950.
//
// y[m, n] = sum_k x[m, k] * (scale[n, g] * q[n, k] + bias[n, g]),  g = k / 64
//         = sum_g ( scale[n,g] * sum_{k in g} x[m,k] * q[n,k]  +  bias[n,g] * xsum[m,g] )
//
// The nibbles q enter the MFMA as exact fp16 integers: each 16-bit half is built
// as 0x6400 | q, the fp16 value 1024 + q, by one shift and one and-or per two
// nibbles, and one packed fp16 subtraction of 1024 (exact) leaves q. Scale and
// bias are applied in fp32 per group:
//   y += scale * acc_g + bias * xsum[m, g]
// so the weights are never rounded, and acc_g = sum x q stays small (no large
// offset for the fp32 accumulation to lose bits against). The activation enters
// as an fp16 hi + lo pair (each MFMA step runs twice), so the only differences
// from an fp32 reference are ~2^-22 relative on the activation and the fp32
// summation order.

// Device weight layout ("tile32-g64"), produced once by q4_repack_kernel from
// the MLX layout w_q[N][K/8] (word j of row n holds k = 8j..8j+7, low nibble
// first) and scales/biases[N][K/64] (bf16):
//   qw[((nt*G + g)*64 + l)*4 + t] = w_q[32*nt + (l&31)][8*g + 4*(l>>5) + t]
//   sb[(nt*G + g)*32 + r]         = scale_bits | bias_bits << 16   (row 32nt + r)
// so one n-tile x group is a contiguous 1 KiB of words (one dwordx4 per lane)
// plus 128 B of scale/bias.
//
// The activation is ACT_F16P: hi and lo planes of fp16 rows whose 8-chunks are
// stored in the order (0,4,1,5,2,6,3,7), which is exactly the k order of the B
// halves above, plus xsum[m][g] = sum over the group of hi + lo (fp32).
#include "common.h"
#include "launch.h"

extern "C" __global__ void q4_repack_kernel(const uint32_t* __restrict__ w_q,
                                            const uint16_t* __restrict__ scales,
                                            const uint16_t* __restrict__ biases,
                                            uint32_t* __restrict__ qw, uint32_t* __restrict__ sb,
                                            int N, int K) {
  const int G = K >> 6;
  const int words = K >> 3;
  const int64_t total = (int64_t)N * words;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i & 3;
    const int64_t l = (i >> 2) & 63;
    const int64_t tg = i >> 8;  // nt*G + g
    const int64_t nt = tg / G, g = tg % G;
    const int64_t n = 32 * nt + (l & 31);
    const int64_t j = 8 * g + 4 * (l >> 5) + t;
    qw[i] = w_q[n * words + j];
  }
  const int64_t total_sb = (int64_t)N * G;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total_sb;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i & 31;
    const int64_t tg = i >> 5;
    const int64_t nt = tg / G, g = tg % G;
    const int64_t n = 32 * nt + r;
    sb[i] = (uint32_t)scales[n * G + g] | ((uint32_t)biases[n * G + g] << 16);
  }
}

// fp32 (or bf16) activation rows -> ACT_F16P (hi plane, lo plane at + M*K) +
// group sums of hi + lo. One wave per (row, group).
extern "C" __global__ void q4_act_prep_kernel(const void* __restrict__ x, int x_is_bf16,
                                              _Float16* __restrict__ xp,
                                              float* __restrict__ xsum, int M, int K) {
  const int G = K >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t wid = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
  if (wid >= (int64_t)M * G) return;
  const int64_t m = wid / G, g = wid % G;
  const int k = (int)g * 64 + lane;
  float v;
  if (x_is_bf16) v = bf16_bits_to_float(((const uint16_t*)x)[m * K + k]);
  else v = ((const float*)x)[m * K + k];
  const _Float16 h = (_Float16)v, lo = f16_lo(v, h);
  xp[m * K + f16p_index(k)] = h;
  xp[(int64_t)M * K + m * K + f16p_index(k)] = lo;
  const float s = wave_sum((float)h + (float)lo);
  if (lane == 0) xsum[m * G + g] = s;
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
namespace drt {

void q4_repack(const uint32_t* w_q, const uint16_t* scales, const uint16_t* biases, int N, int K,
               uint32_t* qw, uint32_t* sb, hipStream_t s) {
  require(N % 32 == 0 && K % 64 == 0, "q4 linear needs N % 32 == 0 and K % 64 == 0");
  const int64_t work = (int64_t)N * (K / 8);
  const int blocks = (int)std::min<int64_t>((work + 255) / 256, 65536);
  hipLaunchKernelGGL(q4_repack_kernel, dim3(blocks), dim3(256), 0, s, w_q, scales, biases, qw, sb,
                     N, K);
  DRT_HIP(hipGetLastError());
}

void q4_act_prep(const void* x, bool x_bf16, int M, int K, _Float16* xp, float* xsum,
                 hipStream_t s) {
  const int64_t waves = (int64_t)M * (K / 64);
  hipLaunchKernelGGL(q4_act_prep_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, x,
                     (int)x_bf16, xp, xsum, M, K);
  DRT_HIP(hipGetLastError());
}

}  // namespace drt
