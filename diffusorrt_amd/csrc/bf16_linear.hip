// bf16-weight linear support for gfx950 (the GEMM itself is fused_linear.hip):
// y = bf16(x) @ W^T with fp32 accumulation, rounded to bf16 like the reference's
// bf16 matmul output (backends/mlx_ops.py:122-125).
//
// Device weight layout (produced once at upload from row-major W[N][K]):
//   wb[((nt*KC + kc)*64 + l)*8 + e] = W[32*nt + (l&31)][16*kc + 8*(l>>5) + e],  KC = K/16
// one n-tile x 16-k chunk is a contiguous 1 KiB (one 16-byte load per lane).
// The activation is ACT_BF16 (natural order).
#include "common.h"
#include "launch.h"

extern "C" __global__ void bf16_repack_kernel(const uint16_t* __restrict__ w,
                                              uint16_t* __restrict__ wb, int N, int K) {
  const int KC = K >> 4;
  const int64_t total = (int64_t)N * K / 8;  // 16-byte chunks
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t l = i & 63;
    const int64_t tk = i >> 6;  // nt*KC + kc
    const int64_t nt = tk / KC, kc = tk % KC;
    const int64_t n = 32 * nt + (l & 31);
    const int64_t k = 16 * kc + 8 * (l >> 5);
    *(u32x4*)(wb + i * 8) = *(const u32x4*)(w + n * K + k);
  }
}

namespace drt {

void bf16_repack(const uint16_t* w, int N, int K, uint16_t* wb, hipStream_t s) {
  require(N % 32 == 0 && K % 16 == 0, "bf16 linear needs N % 32 == 0 and K % 16 == 0");
  const int64_t work = (int64_t)N * K / 8;
  const int blocks = (int)std::min<int64_t>((work + 255) / 256, 65536);
  hipLaunchKernelGGL(bf16_repack_kernel, dim3(blocks), dim3(256), 0, s, w, wb, N, K);
  DRT_HIP(hipGetLastError());
}

}  // namespace drt

// ---- small fp32 <-> bf16 helpers used by the per-op entry points ----
extern "C" __global__ void round_bf16_bias_kernel(float* __restrict__ y, int64_t n,
                                                  const uint16_t* __restrict__ bias, int N) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    float v = round_bf16(y[i]);
    if (bias) v += bf16_bits_to_float(bias[i % N]);
    y[i] = v;
  }
}

extern "C" __global__ void to_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ o,
                                          int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    o[i] = float_to_bf16_bits(x[i]);
}

namespace drt {

void round_bf16_inplace(float* y, int64_t n, const uint16_t* bias, int N, hipStream_t s) {
  const int blocks = (int)std::min<int64_t>((n + 255) / 256, 8192);
  hipLaunchKernelGGL(round_bf16_bias_kernel, dim3(blocks), dim3(256), 0, s, y, n, bias, N);
  DRT_HIP(hipGetLastError());
}

void to_bf16(const float* x, uint16_t* o, int64_t n, hipStream_t s) {
  const int blocks = (int)std::min<int64_t>((n + 255) / 256, 8192);
  hipLaunchKernelGGL(to_bf16_kernel, dim3(blocks), dim3(256), 0, s, x, o, n);
  DRT_HIP(hipGetLastError());
}

}  // namespace drt
