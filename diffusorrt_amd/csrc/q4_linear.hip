// 4-bit affine group-64 quantized linear (MLX packing) for gfx950.
//
// y[m, n] = sum_k x[m, k] * (scale[n, g] * q[n, k] + bias[n, g]),  g = k / 64
//         = sum_g ( scale[n,g] * sum_{k in g} x[m,k] * q[n,k]  +  bias[n,g] * xsum[m,g] )
//
// The nibbles q enter the MFMA as exact fp16 integers: each 16-bit half is built
// as 0x6400 | q, i.e. the fp16 value 1024 + q, by one shift and one and-or per
// two nibbles. The 1024 offset is removed in fp32 together with the bias:
//   y += scale * acc_g + (bias - 1024 * scale) * xsum[m, g]
// so the weights are never rounded; the only rounding versus an fp32 reference
// is the fp16 activation (2^-12 relative) and fp32 accumulation order.
//
// Device weight layout ("tile32-g64"), produced once by q4_repack_kernel from
// the MLX layout w_q[N][K/8] (word j of row n holds k = 8j..8j+7, low nibble
// first) and scales/biases[N][K/64] (bf16):
//   qw[((nt*G + g)*64 + l)*4 + t] = w_q[32*nt + (l&31)][8*g + 4*(l>>5) + t]
//   sb[(nt*G + g)*32 + r]         = scale_bits | bias_bits << 16   (row 32nt + r)
// so one n-tile x group is a contiguous 1 KiB of words (one dwordx4 per lane)
// plus 128 B of scale/bias.
//
// The activation is ACT_F16P: fp16 rows whose 8-chunks are stored in the order
// (0,4,1,5,2,6,3,7), which is exactly the k order of the B halves above, plus
// xsum[m][g] = sum over the group of the fp16-rounded values (fp32).
#include "gemm_core.h"
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

// fp32 (or bf16) activation rows -> ACT_F16P + group sums. One wave per (row, group).
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
  const _Float16 h = (_Float16)v;
  xp[m * K + f16p_index(k)] = h;
  const float s = wave_sum((float)h);
  if (lane == 0) xsum[m * G + g] = s;
}

// Split-K q4 GEMM for a 32-row tile: each wave owns NT consecutive 32-column
// n-tiles; the WG's WAVES waves share the activation slice, staged in LDS in
// chunks of at most CHUNK groups. Grid: x = ceil(N / (32*NT*WAVES)),
// y = K splits, z = ceil(M / 32).
// out: partial sums [splits][M][N] fp32 (deterministic, reduced by the epilogue).
template <int NT, int WAVES, int P>
__global__ __launch_bounds__(64 * WAVES) void q4_gemm_kernel(
    const uint32_t* __restrict__ qw, const uint32_t* __restrict__ sb,
    const _Float16* __restrict__ xp, const float* __restrict__ xsum,
    float* __restrict__ out, int M, int N, int K, int groups_per_split, int chunk_groups) {
  const int G = K >> 6;
  const int NTILES = N >> 5;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int split = blockIdx.y;
  const int g0 = split * groups_per_split;
  const int ng = min(G - g0, groups_per_split);
  const int m0 = blockIdx.z * 32;
  const int nt0 = (blockIdx.x * WAVES + wave) * NT;
  const bool active = nt0 < NTILES;

  extern __shared__ __align__(16) char smem[];
  const int row_h = chunk_groups * 64 + 8;  // 16 B pad keeps b128 reads conflict-free
  _Float16* xs = (_Float16*)smem;
  float* xss = (float*)(smem + (size_t)32 * row_h * 2);

  int ntv[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) ntv[j] = min(nt0 + j, NTILES - 1);  // clamp: loads stay in bounds
  f32x16 acc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[j] = f32x16{};
  const _Float16* arow = xs + (lane & 31) * row_h + 32 * (lane >> 5);

  for (int c0 = 0; c0 < ng; c0 += chunk_groups) {
    const int cng = min(chunk_groups, ng - c0);
    const int gc = g0 + c0;  // first group of this chunk
    __syncthreads();
    const int cpr = cng * 8;  // 16-byte chunks per row
    for (int c = threadIdx.x; c < 32 * cpr; c += 64 * WAVES) {
      const int r = c / cpr, cc = c - r * cpr;
      const int m = m0 + r;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (m < M) v = *(const u32x4*)(xp + (int64_t)m * K + (int64_t)gc * 64 + cc * 8);
      *(u32x4*)(xs + r * row_h + cc * 8) = v;
    }
    for (int c = threadIdx.x; c < 32 * cng; c += 64 * WAVES) {
      const int gg = c >> 5, r = c & 31;
      const int m = m0 + r;
      xss[c] = (m < M) ? xsum[(int64_t)m * G + gc + gg] : 0.f;
    }
    __syncthreads();
    if (!active) continue;

    u32x4 wbuf[P][NT];
    uint32_t sbuf[P][NT];
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int g = gc + min(p, cng - 1);
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        wbuf[p][j] = *q4_tile_words(qw, ntv[j], G, g, lane);
        sbuf[p][j] = q4_tile_sb(sb, ntv[j], G, g, lane);
      }
    }
    for (int gb = 0; gb < cng; gb += P) {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const int gg = gb + p;
        if (gg < cng) {
          f16x8 a[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) a[t] = *(const f16x8*)(arow + gg * 64 + 8 * t);
          float xsr[16];
#pragma unroll
          for (int r = 0; r < 16; ++r) xsr[r] = xss[gg * 32 + mfma_row(r, lane)];
          q4_group_mma<NT>(acc, a, xsr, wbuf[p], sbuf[p]);
          const int gn = gg + P;
          if (gn < cng) {
#pragma unroll
            for (int j = 0; j < NT; ++j) {
              wbuf[p][j] = *q4_tile_words(qw, ntv[j], G, gc + gn, lane);
              sbuf[p][j] = q4_tile_sb(sb, ntv[j], G, gc + gn, lane);
            }
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

// Sum split-K partials (+ optional bf16 bias) into fp32 y[M][N].
extern "C" __global__ void splitk_reduce_kernel(const float* __restrict__ part, int splits,
                                                const uint16_t* __restrict__ bias,
                                                float* __restrict__ y, int M, int N) {
  const int64_t total = (int64_t)M * N;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.f;
    for (int p = 0; p < splits; ++p) s += part[(int64_t)p * total + i];
    if (bias) s += bf16_bits_to_float(bias[i % N]);
    y[i] = s;
  }
}

template __global__ void q4_gemm_kernel<1, 4, 4>(const uint32_t*, const uint32_t*, const _Float16*,
                                                 const float*, float*, int, int, int, int, int);

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

// Pick K splits so that the grid has enough waves to keep HBM busy while each
// split still streams several groups (each split costs an M x N partial write).
SplitPlan plan_linear(const LinearW& w, int M) {
  SplitPlan p;
  const int m_tiles = (M + 31) / 32;
  const int units = w.q4 ? w.K / 64 : w.K / 16;     // groups or 16-k chunks
  const int min_per_split = w.q4 ? 2 : 8;
  const int col_blocks = (w.N / 32 + 3) / 4;         // NT = 1, 4 waves
  const int target_wgs = 1024;
  int splits = std::max(1, target_wgs / std::max(1, col_blocks * m_tiles));
  splits = std::min(splits, std::max(1, units / min_per_split));
  int per = (units + splits - 1) / splits;
  per = std::max(per, 1);
  p.per_split = per;
  p.splits = (units + per - 1) / per;
  return p;
}

void linear_partials(const LinearW& w, const void* act, const float* xsum, int M, float* part,
                     const SplitPlan& plan, hipStream_t s) {
  if (!w.q4) {
    bf16_linear_partials(w.wb.as<uint16_t>(), (const uint16_t*)act, M, w.N, w.K, part,
                         plan.splits, plan.per_split, s);
    return;
  }
  const int m_tiles = (M + 31) / 32;
  const int ng = plan.per_split;
  const int chunk = std::min(ng, 16);  // <= 16 groups staged at a time (~68 KB LDS)
  const size_t lds = (size_t)32 * (chunk * 64 + 8) * 2 + (size_t)32 * chunk * 4;
  const dim3 grid((w.N / 32 + 3) / 4, plan.splits, m_tiles);
  auto fn = q4_gemm_kernel<1, 4, 4>;
  static size_t granted = 0;
  grant_lds((const void*)fn, lds, granted);
  hipLaunchKernelGGL(fn, grid, dim3(256), lds, s, w.qw.as<uint32_t>(), w.sb.as<uint32_t>(),
                     (const _Float16*)act, xsum, part, M, w.N, w.K, ng, chunk);
  DRT_HIP(hipGetLastError());
}

void splitk_reduce(const float* part, int splits, const uint16_t* bias, float* y, int M, int N,
                   hipStream_t s) {
  const int64_t total = (int64_t)M * N;
  const int blocks = (int)std::min<int64_t>((total + 255) / 256, 8192);
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, s, part, splits, bias, y, M,
                     N);
  DRT_HIP(hipGetLastError());
}

}  // namespace drt
