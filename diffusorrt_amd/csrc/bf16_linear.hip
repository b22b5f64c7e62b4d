// bf16-weight linear for gfx950: y = bf16(x) @ W^T with fp32 accumulation,
// the reference's bf16 path (backends/mlx_ops.py:122-125). The epilogue that
// consumes the split-K partials rounds the sum to bf16, as the reference's bf16
// matmul output is rounded.
//
// Device weight layout (produced once at upload from row-major W[N][K]):
//   wb[((nt*KC + kc)*64 + l)*8 + e] = W[32*nt + (l&31)][16*kc + 8*(l>>5) + e],  KC = K/16
// one n-tile x 16-k chunk is a contiguous 1 KiB (one 16-byte load per lane).
// The activation is ACT_BF16 (natural order).
#include "gemm_core.h"
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

// Grid: x = ceil(N / (32*NT*WAVES)), y = K splits (chunks_per_split 16-k chunks
// each), z = ceil(M / 32); the activation is staged in LDS stage_chunks at a
// time. out: partials [splits][M][N] fp32.
template <int NT, int WAVES, int P>
__global__ __launch_bounds__(64 * WAVES) void bf16_gemm_kernel(
    const uint16_t* __restrict__ wb, const uint16_t* __restrict__ x, float* __restrict__ out,
    int M, int N, int K, int chunks_per_split, int stage_chunks) {
  const int KC = K >> 4;
  const int NTILES = N >> 5;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int split = blockIdx.y;
  const int c0 = split * chunks_per_split;
  const int nc = min(KC - c0, chunks_per_split);
  const int m0 = blockIdx.z * 32;
  const int nt0 = (blockIdx.x * WAVES + wave) * NT;
  const bool active = nt0 < NTILES;

  extern __shared__ __align__(16) char smem[];
  const int row_h = stage_chunks * 16 + 8;
  uint16_t* xs = (uint16_t*)smem;
  int ntv[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) ntv[j] = min(nt0 + j, NTILES - 1);
  f32x16 acc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[j] = f32x16{};
  const uint16_t* arow = xs + (lane & 31) * row_h + 8 * (lane >> 5);

  for (int s0 = 0; s0 < nc; s0 += stage_chunks) {
    const int snc = min(stage_chunks, nc - s0);
    const int cbase = c0 + s0;
    __syncthreads();
    const int cpr = snc * 2;  // 16-byte pieces per row
    for (int c = threadIdx.x; c < 32 * cpr; c += 64 * WAVES) {
      const int r = c / cpr, cc = c - r * cpr;
      const int m = m0 + r;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (m < M) v = *(const u32x4*)(x + (int64_t)m * K + (int64_t)cbase * 16 + cc * 8);
      *(u32x4*)(xs + r * row_h + cc * 8) = v;
    }
    __syncthreads();
    if (!active) continue;
    bf16x8 wbuf[P][NT];
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int j = 0; j < NT; ++j) wbuf[p][j] = *bf16_tile_frag(wb, ntv[j], KC, cbase + min(p, snc - 1), lane);
    for (int cb = 0; cb < snc; cb += P) {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const int cc = cb + p;
        if (cc < snc) {
          const bf16x8 a = *(const bf16x8*)(arow + cc * 16);
#pragma unroll
          for (int j = 0; j < NT; ++j) acc[j] = mfma_bf16(a, wbuf[p][j], acc[j]);
          const int cn = cc + P;
          if (cn < snc) {
#pragma unroll
            for (int j = 0; j < NT; ++j) wbuf[p][j] = *bf16_tile_frag(wb, ntv[j], KC, cbase + cn, lane);
          }
        }
      }
    }
  }
  if (!active) return;
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    if (nt0 + j >= NTILES) break;
    const int n = (nt0 + j) * 32 + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = m0 + mfma_row(r, lane);
      if (m < M) out[((int64_t)split * M + m) * N + n] = acc[j][r];
    }
  }
}

template __global__ void bf16_gemm_kernel<1, 4, 8>(const uint16_t*, const uint16_t*, float*, int,
                                                   int, int, int, int);

namespace drt {

void bf16_repack(const uint16_t* w, int N, int K, uint16_t* wb, hipStream_t s) {
  require(N % 32 == 0 && K % 16 == 0, "bf16 linear needs N % 32 == 0 and K % 16 == 0");
  const int64_t work = (int64_t)N * K / 8;
  const int blocks = (int)std::min<int64_t>((work + 255) / 256, 65536);
  hipLaunchKernelGGL(bf16_repack_kernel, dim3(blocks), dim3(256), 0, s, w, wb, N, K);
  DRT_HIP(hipGetLastError());
}

void bf16_linear_partials(const uint16_t* wb, const uint16_t* x, int M, int N, int K, float* part,
                          int splits, int chunks_per_split, hipStream_t s) {
  const int m_tiles = (M + 31) / 32;
  const int stage = std::min(chunks_per_split, 64);  // <= 1024 k staged (~66 KB LDS)
  const size_t lds = (size_t)32 * (stage * 16 + 8) * 2;
  auto fn = bf16_gemm_kernel<1, 4, 8>;
  static size_t granted = 0;
  grant_lds((const void*)fn, lds, granted);
  hipLaunchKernelGGL(fn, dim3((N / 32 + 3) / 4, splits, m_tiles), dim3(256), lds, s, wb, x, part,
                     M, N, K, chunks_per_split, stage);
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
