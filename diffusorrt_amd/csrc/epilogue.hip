// Elementwise and epilogue kernels of the decoder layer (gfx950).
//
//   * embed_kernel:         token rows of the bf16 table -> fp32 residual stream.
//   * residual_norm_kernel: (optional split partials added to) the residual
//     stream, then RMSNorm(h) * w of selected rows in an activation format:
//     the final norm of the LM-head rows, and the reduce + next norm of the
//     large-M forwards' split-K projections.
//   * per-op fp32 kernels of the kernel-table seam: rms_norm, rope, swiglu.
// The decoder layer's other epilogues are fused into fused_linear.hip.
// Reference math: backends/mlx_ops.py:21-35 (rms_norm), :97-130 (linear
// dtypes), :133-144 (rope), :147-154 (swiglu); backends/mlx_forward.py:1164-1361.
#include "common.h"
#include "launch.h"

namespace {

constexpr int KV_TILE = 8192;

template <typename T> DRT_DEV T cvt(float f);
template <> DRT_DEV _Float16 cvt<_Float16>(float f) { return (_Float16)f; }
template <> DRT_DEV __bf16 cvt<__bf16>(float f) {
  return __builtin_bit_cast(__bf16, float_to_bf16_bits(f));
}

DRT_DEV float block_sum_256(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
  const int nw = blockDim.x >> 6;
  for (int i = 0; i < nw; ++i) t += red[i];
  return t;
}

}  // namespace

// tokens[M] -> hidden fp32 [M][d] (bf16 embedding rows cast to fp32,
// backends/mlx_forward.py:1538-1557).
// Also writes, when ss_out is set, the rows' partial sums of squares per 32
// columns for the next RMSNorm, one [d/32][32] block per 32-row tile
// (ss_out[(m / 32) * d + c * 32 + m % 32], c = column / 32); grid rows M .. up to
// the end of the last tile (when launched) write zero partials.
// With pre (and ss_out), the first layer's pre-scaled norm input as well: the
// planes of w * h * c (ACT_F16P, [M][d] hi then lo), c from this row's own norm
// factor (pre_scale_of), c into pre_sc[m], and the planes' per-32-column sums
// laid out like ss_out (zero rows past M).
// With row_desc the token of row m is tokens[row_desc->row0 + m] (a canvas on the
// device that a graph-replayed forward reads at its step's rows).
extern "C" __global__ __launch_bounds__(256) void embed_kernel(
    const int32_t* __restrict__ tokens, const uint16_t* __restrict__ table,
    float* __restrict__ hidden, int M, int d, float* __restrict__ ss_out,
    const StepDesc* __restrict__ row_desc, const uint16_t* __restrict__ pre_norm, float eps,
    uint16_t* __restrict__ pre, float* __restrict__ pre_xs, float* __restrict__ pre_sc,
    int* __restrict__ err) {
  // thread c owns columns 32c .. 32c + 31 (d % 32 == 0, d <= 32 * 256); every
  // load is issued before the first store (a wait for a load also waits for the
  // stores issued before it)
  const int m = blockIdx.x, c = threadIdx.x, ng = d >> 5;
  const bool live = c < ng;
  if (row_desc) tokens += row_desc->row0;
  float* ss_row = ss_out ? ss_out + (int64_t)(m >> 5) * d + (m & 31) : nullptr;
  float* xs_row = pre ? pre_xs + (int64_t)(m >> 5) * d + (m & 31) : nullptr;
  if (m >= M) {
    if (ss_out && live) {
      ss_row[c * 32] = 0.f;
      if (xs_row) xs_row[c * 32] = 0.f;
    }
    return;
  }
  const int64_t tok = tokens[m];
  const int k0 = min(c, ng - 1) * 32;
  const uint16_t* trow = table + tok * d + k0;
  u32x4 tv[4], wv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) tv[j] = *(const u32x4*)(trow + 8 * j);
  if (pre) {
#pragma unroll
    for (int j = 0; j < 4; ++j) wv[j] = *(const u32x4*)(pre_norm + k0 + 8 * j);
  }
  float x[32];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[8 * j + 2 * e] = bf16_bits_to_float(tv[j][e] & 0xffffu);
      x[8 * j + 2 * e + 1] = bf16_bits_to_float(tv[j][e] >> 16);
    }
  float q = 0.f;
#pragma unroll
  for (int e = 0; e < 32; ++e) q += x[e] * x[e];
  if (!live) q = 0.f;
  if (pre) {
    __shared__ float red[4];
    const float sc = pre_scale_of(1.f / sqrtf(block_sum_256(q, red) / (float)d + eps));
    u32x4 ph[4], pl[4];
    float xsum = 0.f;
    bool over = false;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int w = 0; w < 4; ++w) {  // word w of chunk j holds elements (w, w + 4)
        const int e0 = 8 * j + w, e1 = e0 + 4;
        const uint32_t w0 = wv[j][(e0 & 7) >> 1], w1 = wv[j][(e1 & 7) >> 1];
        const float g0 = bf16_bits_to_float((e0 & 1) ? w0 >> 16 : w0 & 0xffffu);
        const float g1 = bf16_bits_to_float((e1 & 1) ? w1 >> 16 : w1 & 0xffffu);
        const float v0 = (x[e0] * sc) * g0, v1 = (x[e1] * sc) * g1;
        const _Float16 h0 = (_Float16)v0, h1 = (_Float16)v1;
        const _Float16 l0 = f16_lo(v0, h0), l1 = f16_lo(v1, h1);
        ph[j][w] = pack_half2(h0, h1);
        pl[j][w] = pack_half2(l0, l1);
        over = over || f16_overflows(v0) || f16_overflows(v1);
        xsum += ((float)h0 + (float)l0) + ((float)h1 + (float)l1);
      }
    if (live) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        *(u32x4*)(pre + (int64_t)m * d + k0 + 8 * j) = ph[j];
        *(u32x4*)(pre + (int64_t)(M + m) * d + k0 + 8 * j) = pl[j];
      }
      xs_row[c * 32] = xsum;
      if (over && err)
        __hip_atomic_fetch_or(err, DRT_ERR_F16_RANGE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (threadIdx.x == 0) pre_sc[m] = sc;
  }
  if (live) {
    f32x4* hrow = (f32x4*)(hidden + (int64_t)m * d + k0);
#pragma unroll
    for (int j = 0; j < 8; ++j) hrow[j] = f32x4{x[4 * j], x[4 * j + 1], x[4 * j + 2], x[4 * j + 3]};
    if (ss_out) ss_row[c * 32] = q;
  }
}

// WPR waves per output row (4 / WPR rows per 256-thread work-group). Wave w of
// a row owns the 8-element chunks of lanes l + 64 (w + WPR j) of the row
// (d % 64 == 0, d <= 4096), loaded and stored 16 bytes at a time; the 8 chunks
// of a 64-wide group are 8 consecutive lanes. One wave per row suits d <= 1024
// (every chunk's loads in flight at once); four waves per row split the chunks
// of wider rows so that theirs are too, and add the row's sum of squares in LDS.
//   src row  = src_rows ? src_rows[i] : i
//   v        = hidden[src] + R(sum_s part[s][src])          (part may be null)
//   hidden_out[src] = v                                     (if write_hidden)
//   act[i]   = fmt(v * rsqrt(mean(v^2) + eps) * w)          (if norm_w non-null)
// (backends/mlx_ops.py:21-35 for the norm; R rounds to bf16 when rnd_bf16.)
constexpr int RN_MAX_SPLITS = 9;  // partial slices a reduce takes

template <int WPR>
DRT_DEV void residual_norm_rows(float* __restrict__ hidden, const float* __restrict__ part,
                                int splits, int M_part, int rnd_bf16,
                                const int32_t* __restrict__ src_rows, int write_hidden,
                                const uint16_t* __restrict__ norm_w, float eps, int d, int fmt,
                                void* __restrict__ act, float* __restrict__ xsum, int n_rows,
                                int* __restrict__ err) {
  constexpr int NC = 8 / WPR;  // chunks per lane for d <= 4096
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, w = wave % WPR;
  const int i = blockIdx.x * (4 / WPR) + wave / WPR;
  if (i >= n_rows) return;  // whole rows (with WPR = 4, the whole work-group)
  const int src = src_rows ? src_rows[i] : i;
  // chunk j of this wave: lanes' 8-element chunks lane + 64 (w + WPR j)
  auto kof = [&](int j) { return (lane + 64 * (w + WPR * j)) * 8; };
  auto has = [&](int j) { return 512 * (w + WPR * j) < d; };  // uniform across the wave
  // Every load is issued before the first store: a wait for a load also waits
  // for the stores issued before it. Within a last, partial chunk the
  // addresses are clamped and the lanes past d are zeroed.
  f32x4 v[NC][2];
  u32x4 wv[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    v[c][0] = v[c][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    wv[c] = u32x4{0u, 0u, 0u, 0u};
    if (has(c)) {
      const int k = min(kof(c), d - 8);
      const f32x4* hp = (const f32x4*)(hidden + (int64_t)src * d + k);
      v[c][0] = hp[0];
      v[c][1] = hp[1];
    }
  }
  if (norm_w) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
      if (has(c)) wv[c] = *(const u32x4*)(norm_w + min(kof(c), d - 8));
  }
  if (part) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (has(c)) {
        const int k = min(kof(c), d - 8);
        // every slice's loads are issued before the first add (one latency)
        f32x4 ps[RN_MAX_SPLITS][2];
#pragma unroll
        for (int p = 0; p < RN_MAX_SPLITS; ++p) {
          const f32x4* pp =
              (const f32x4*)(part + ((int64_t)min(p, splits - 1) * M_part + src) * d + k);
          ps[p][0] = pp[0];
          ps[p][1] = pp[1];
        }
        f32x4 s0 = f32x4{0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
        for (int p = 0; p < RN_MAX_SPLITS; ++p) {
          if (p < splits) {
            s0 += ps[p][0];
            s1 += ps[p][1];
          }
        }
        if (rnd_bf16) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s0[e] = round_bf16(s0[e]);
            s1[e] = round_bf16(s1[e]);
          }
        }
        v[c][0] += s0;
        v[c][1] += s1;
      }
    }
  }
#pragma unroll
  for (int c = 0; c < NC; ++c)
    if (kof(c) >= d) v[c][0] = v[c][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (part && write_hidden) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int k = kof(c);
      if (k < d) {
        f32x4* hp = (f32x4*)(hidden + (int64_t)src * d + k);
        hp[0] = v[c][0];
        hp[1] = v[c][1];
      }
    }
  }
  if (!norm_w) return;  // (uniform across the work-group)
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) ss += v[c][0][e] * v[c][0][e] + v[c][1][e] * v[c][1][e];
  ss = wave_sum(ss);
  if (WPR > 1) {  // the row's waves in wave order
    __shared__ float rsum[4];
    if (lane == 0) rsum[wave] = ss;
    __syncthreads();
    ss = rsum[0];
#pragma unroll
    for (int q = 1; q < WPR; ++q) ss += rsum[q];
  }
  const float inv = 1.f / sqrtf(ss / (float)d + eps);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int k = kof(c);
    if (k >= d) break;  // uniform across each 8-lane group (d % 64 == 0)
    float n[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      n[2 * e] = (v[c][e >> 1][(2 * e) & 3] * inv) * bf16_bits_to_float(wv[c][e] & 0xffffu);
      n[2 * e + 1] = (v[c][e >> 1][(2 * e + 1) & 3] * inv) * bf16_bits_to_float(wv[c][e] >> 16);
    }
    if (fmt == ACT_F16P) {  // hi plane, lo plane at + n_rows * d
      _Float16 h[8], lo[8];
      float gs = 0.f;
      bool over = false;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const _Float16 he = (_Float16)n[e], le = f16_lo(n[e], he);
        h[f16p_index(e)] = he;
        lo[f16p_index(e)] = le;
        gs += (float)he + (float)le;
        over = over || f16_overflows(n[e]);
      }
      _Float16* dst = (_Float16*)act + (int64_t)i * d + k;
      *(u32x4*)dst = __builtin_bit_cast(u32x4, h);
      *(u32x4*)(dst + (int64_t)n_rows * d) = __builtin_bit_cast(u32x4, lo);
      if (over && err) atomicOr(err, DRT_ERR_F16_RANGE);
      if (xsum) {
        gs += __shfl_xor(gs, 1, 64);
        gs += __shfl_xor(gs, 2, 64);
        gs += __shfl_xor(gs, 4, 64);
        if ((lane & 7) == 0) xsum[(int64_t)i * (d >> 6) + (k >> 6)] = gs;
      }
    } else if (fmt == ACT_BF16) {
      uint16_t h[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) h[e] = float_to_bf16_bits(n[e]);
      *(u32x4*)((uint16_t*)act + (int64_t)i * d + k) = __builtin_bit_cast(u32x4, h);
    } else {
      f32x4* o = (f32x4*)((float*)act + (int64_t)i * d + k);
      o[0] = f32x4{n[0], n[1], n[2], n[3]};
      o[1] = f32x4{n[4], n[5], n[6], n[7]};
    }
  }
}

#define DRT_RN_ARGS                                                                            \
  float *__restrict__ hidden, const float *__restrict__ part, int splits, int M_part,            \
      int rnd_bf16, const int32_t *__restrict__ src_rows, int write_hidden,                     \
      const uint16_t *__restrict__ norm_w, float eps, int d, int fmt, void *__restrict__ act,   \
      float *__restrict__ xsum, int n_rows, int *__restrict__ err
extern "C" __global__ __launch_bounds__(256) void residual_norm_kernel(DRT_RN_ARGS) {
  residual_norm_rows<1>(hidden, part, splits, M_part, rnd_bf16, src_rows, write_hidden, norm_w,
                        eps, d, fmt, act, xsum, n_rows, err);
}
extern "C" __global__ __launch_bounds__(256) void residual_norm_wide_kernel(DRT_RN_ARGS) {
  residual_norm_rows<4>(hidden, part, splits, M_part, rnd_bf16, src_rows, write_hidden, norm_w,
                        eps, d, fmt, act, xsum, n_rows, err);
}
#undef DRT_RN_ARGS

// ---- per-op kernels for the KernelTable seam (fp32 tensors) ----

// RMSNorm over the last axis of x [rows][d] (d <= 4096), bf16 weight.
extern "C" __global__ void rms_norm_rows_kernel(const float* __restrict__ x,
                                                const uint16_t* __restrict__ w, float eps,
                                                float* __restrict__ y, int d) {
  __shared__ float red[8];
  const int64_t r = blockIdx.x;
  float ss = 0.f;
  for (int k = threadIdx.x; k < d; k += blockDim.x) {
    const float v = x[r * d + k];
    ss += v * v;
  }
  const float tot = block_sum_256(ss, red);
  const float inv = 1.f / sqrtf(tot / (float)d + eps);
  for (int k = threadIdx.x; k < d; k += blockDim.x)
    y[r * d + k] = (x[r * d + k] * inv) * bf16_bits_to_float(w[k]);
}

// Split-half RoPE on x [rows][H][hd] fp32 with per-row tables cos/sin [rows][hd].
extern "C" __global__ void rope_rows_kernel(const float* __restrict__ x,
                                            const float* __restrict__ cos_t,
                                            const float* __restrict__ sin_t,
                                            float* __restrict__ y, int rows, int H, int hd) {
  const int64_t total = (int64_t)rows * H * hd;
  const int half = hd >> 1;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int e = (int)(i % hd);
    const int64_t r = i / ((int64_t)H * hd);
    const float xv = x[i];
    const float rot = e < half ? -x[i + half] : x[i - half];
    y[i] = xv * cos_t[r * hd + e] + rot * sin_t[r * hd + e];
  }
}

// silu(g) * u elementwise on fp32.
extern "C" __global__ void swiglu_rows_kernel(const float* __restrict__ g,
                                              const float* __restrict__ u,
                                              float* __restrict__ y, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float gv = g[i];
    y[i] = gv * (1.f / (1.f + expf(-gv))) * u[i];
  }
}

namespace drt {

void embed(const int32_t* tokens, const uint16_t* table, float* hidden, int M, int d,
           float* ss_out, hipStream_t s, const StepDesc* row_desc, const PreOut* pre) {
  require(d % 32 == 0 && d <= 32 * 256, "embed needs d % 32 == 0 and d <= 8192");
  require(!pre || ss_out, "pre-scaled planes need the row statistics");
  // with ss_out, whole 32-row tiles are launched so unused rows get zero partials
  const int grid = ss_out ? (M + 31) / 32 * 32 : M;
  hipLaunchKernelGGL(embed_kernel, dim3(grid), dim3(256), 0, s, tokens, table, hidden, M, d,
                     ss_out, row_desc, pre ? pre->norm : nullptr, pre ? pre->eps : 0.f,
                     pre ? pre->planes : nullptr, pre ? pre->xs : nullptr,
                     pre ? pre->sc : nullptr, pre ? pre->err : nullptr);
  DRT_HIP(hipGetLastError());
}

void residual_norm(float* hidden, const float* part, int splits, int M_part, bool rnd_bf16,
                   const int32_t* src_rows, bool write_hidden, const uint16_t* norm_w, float eps,
                   int d, int fmt, void* act, float* xsum, int n_out_rows, hipStream_t s,
                   int* err) {
  require(d % 64 == 0 && d <= 4096, "residual_norm needs d % 64 == 0 and d <= 4096");
  require(!part || (splits >= 1 && splits <= RN_MAX_SPLITS), "residual_norm takes 1..9 slices");
  if (n_out_rows <= 0) return;
  if (d > 1024)  // one row per work-group, its chunks over four waves
    hipLaunchKernelGGL(residual_norm_wide_kernel, dim3(n_out_rows), dim3(256), 0, s, hidden, part,
                       splits, M_part, (int)rnd_bf16, src_rows, (int)write_hidden, norm_w, eps, d,
                       fmt, act, xsum, n_out_rows, err);
  else
    hipLaunchKernelGGL(residual_norm_kernel, dim3((n_out_rows + 3) / 4), dim3(256), 0, s, hidden,
                       part, splits, M_part, (int)rnd_bf16, src_rows, (int)write_hidden, norm_w,
                       eps, d, fmt, act, xsum, n_out_rows, err);
  DRT_HIP(hipGetLastError());
}

void rms_norm_rows(const float* x, const uint16_t* w, float eps, float* y, int rows, int d,
                   hipStream_t s) {
  hipLaunchKernelGGL(rms_norm_rows_kernel, dim3(rows), dim3(256), 0, s, x, w, eps, y, d);
  DRT_HIP(hipGetLastError());
}

void rope_rows(const float* x, const float* cos_t, const float* sin_t, float* y, int rows, int H,
               int hd, hipStream_t s) {
  const int64_t n = (int64_t)rows * H * hd;
  const int blocks = (int)std::min<int64_t>((n + 255) / 256, 8192);
  hipLaunchKernelGGL(rope_rows_kernel, dim3(blocks), dim3(256), 0, s, x, cos_t, sin_t, y, rows, H,
                     hd);
  DRT_HIP(hipGetLastError());
}

void swiglu_rows(const float* g, const float* u, float* y, int64_t n, hipStream_t s) {
  const int blocks = (int)std::min<int64_t>((n + 255) / 256, 8192);
  hipLaunchKernelGGL(swiglu_rows_kernel, dim3(blocks), dim3(256), 0, s, g, u, y, n);
  DRT_HIP(hipGetLastError());
}

}  // namespace drt
