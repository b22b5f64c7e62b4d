// Elementwise and epilogue kernels of the decoder layer (gfx950).
//
//   * embed_kernel:         token rows of the bf16 table -> fp32 residual stream.
//   * residual_norm_kernel: (optional split partials added to) the residual
//     stream, then RMSNorm(h) * w of selected rows in an activation format;
//     the runtime uses it for the final norm of the LM-head rows.
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

// Write one activation element. F16P also needs a wave-wide group sum, done by
// the caller (each wave covers exactly one 64-wide group per call).
DRT_DEV void write_act(int fmt, void* row, int k, float v, float* xsum_row, int lane) {
  if (fmt == ACT_F16P) {
    const _Float16 h = (_Float16)v;
    ((_Float16*)row)[f16p_index(k)] = h;
    const float s = wave_sum((float)h);
    if (lane == 0) xsum_row[k >> 6] = s;
  } else if (fmt == ACT_BF16) {
    ((uint16_t*)row)[k] = float_to_bf16_bits(v);
  } else {
    ((float*)row)[k] = v;
  }
}

DRT_DEV size_t act_row_bytes(int fmt, int d) { return fmt == 2 ? (size_t)d * 4 : (size_t)d * 2; }

}  // namespace

// tokens[M] -> hidden fp32 [M][d] (bf16 embedding rows cast to fp32,
// backends/mlx_forward.py:1538-1557).
// Also writes, when ss_out is set, the rows' partial sums of squares per 32
// columns (ss_out[c*32 + m], c = column / 32) for the next RMSNorm; grid rows
// M .. 31 (when launched) write zero partials.
extern "C" __global__ void embed_kernel(const int32_t* __restrict__ tokens,
                                        const uint16_t* __restrict__ table,
                                        float* __restrict__ hidden, int M, int d,
                                        float* __restrict__ ss_out) {
  const int m = blockIdx.x;
  if (m >= M) {
    if (ss_out)
      for (int c = threadIdx.x; c < d / 32; c += blockDim.x) ss_out[c * 32 + m] = 0.f;
    return;
  }
  const int64_t tok = tokens[m];
  for (int k = threadIdx.x; k < d; k += blockDim.x)
    hidden[(int64_t)m * d + k] = bf16_bits_to_float(table[tok * d + k]);
  if (ss_out) {
    for (int c = threadIdx.x; c < d / 32; c += blockDim.x) {
      float q = 0.f;
      for (int k = 0; k < 32; ++k) {
        const float v = bf16_bits_to_float(table[tok * d + c * 32 + k]);
        q += v * v;
      }
      ss_out[c * 32 + m] = q;
    }
  }
}

// One 256-thread WG per output row. Requires d % 256 == 0 (true for every
// geometry here: 1024, 3584 = 14 * 256).
//   src row  = src_rows ? src_rows[i] : i
//   v        = hidden[src] + R(sum_s part[s][src])          (part may be null)
//   hidden_out[src] = v                                     (if non-null)
//   act[i]   = fmt(v * rsqrt(mean(v^2) + eps) * w)          (if norm_w non-null)
extern "C" __global__ void residual_norm_kernel(
    float* __restrict__ hidden, const float* __restrict__ part, int splits, int M_part,
    int rnd_bf16, const int32_t* __restrict__ src_rows, int write_hidden,
    const uint16_t* __restrict__ norm_w, float eps, int d, int fmt, void* __restrict__ act,
    float* __restrict__ xsum) {
  __shared__ float red[8];
  const int i = blockIdx.x;
  const int src = src_rows ? src_rows[i] : i;
  const int lane = threadIdx.x & 63;
  constexpr int MAXV = 14;  // d <= 3584
  float v[MAXV];
  const int nv = d / 256;
  float ss = 0.f;
  for (int j = 0; j < nv; ++j) {
    const int k = j * 256 + threadIdx.x;
    float x = hidden[(int64_t)src * d + k];
    if (part) {
      float s = 0.f;
      for (int p = 0; p < splits; ++p) s += part[((int64_t)p * M_part + src) * d + k];
      if (rnd_bf16) s = round_bf16(s);
      x += s;
    }
    v[j] = x;
    ss += x * x;
  }
  if (write_hidden)
    for (int j = 0; j < nv; ++j) hidden[(int64_t)src * d + j * 256 + threadIdx.x] = v[j];
  if (!norm_w) return;
  const float tot = block_sum_256(ss, red);
  const float inv = 1.f / sqrtf(tot / (float)d + eps);
  char* arow = (char*)act + (size_t)i * act_row_bytes(fmt, d);
  float* xs_row = xsum ? xsum + (int64_t)i * (d >> 6) : nullptr;
  for (int j = 0; j < nv; ++j) {
    const int k = j * 256 + threadIdx.x;
    const float n = (v[j] * inv) * bf16_bits_to_float(norm_w[k]);
    write_act(fmt, arow, k, n, xs_row, lane);
  }
}

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
           float* ss_out, hipStream_t s) {
  // with ss_out, rows up to 32 are launched so unused rows get zero partials
  const int grid = ss_out ? std::max(M, 32) : M;
  hipLaunchKernelGGL(embed_kernel, dim3(grid), dim3(256), 0, s, tokens, table, hidden, M, d,
                     ss_out);
  DRT_HIP(hipGetLastError());
}

void residual_norm(float* hidden, const float* part, int splits, int M_part, bool rnd_bf16,
                   const int32_t* src_rows, bool write_hidden, const uint16_t* norm_w, float eps,
                   int d, int fmt, void* act, float* xsum, int n_out_rows, hipStream_t s) {
  require(d % 256 == 0 && d <= 14 * 256, "residual_norm needs d % 256 == 0 and d <= 3584");
  if (n_out_rows <= 0) return;
  hipLaunchKernelGGL(residual_norm_kernel, dim3(n_out_rows), dim3(256), 0, s, hidden, part, splits,
                     M_part, (int)rnd_bf16, src_rows, (int)write_hidden, norm_w, eps, d, fmt, act,
                     xsum);
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
