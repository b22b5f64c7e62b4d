// Elementwise and epilogue kernels of the decoder layer (gfx950).
//
// Every split-K linear writes fp32 partials [splits][M][N]; the kernels here
// reduce them in a fixed order (deterministic) and fuse the op that follows:
//   * residual_norm_kernel: h += sum(partials) [bf16-rounded for bf16 weights,
//     as the reference's bf16 matmul output is], then RMSNorm(h) * w written
//     in the activation format the next linear reads.
//   * qkv_epilogue_kernel:  q/k/v reduce (+ bias), per-head q/k RMSNorm,
//     split-half RoPE, Q out for attention, K/V into the tiled KV cache.
//   * swiglu_kernel:        gate/up reduce, silu(g) * u, activation for down.
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
extern "C" __global__ void embed_kernel(const int32_t* __restrict__ tokens,
                                        const uint16_t* __restrict__ table,
                                        float* __restrict__ hidden, int M, int d) {
  const int m = blockIdx.x;
  if (m >= M) return;
  const int64_t tok = tokens[m];
  for (int k = threadIdx.x; k < d; k += blockDim.x)
    hidden[(int64_t)m * d + k] = bf16_bits_to_float(table[tok * d + k]);
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

// QKV epilogue. One WG (4 waves) per row; each wave takes whole heads, lane l
// holding head elements l and l + 64 (the RoPE pair). Heads 0..Hq-1 are q,
// then Hkv k heads, then Hkv v heads, matching the fused [q | k | v] linear.
template <typename T>
__global__ void qkv_epilogue_kernel(const float* __restrict__ part, int splits, int M,
                                    const uint16_t* __restrict__ bias, int rnd_bf16,
                                    const uint16_t* __restrict__ q_norm,
                                    const uint16_t* __restrict__ k_norm, float eps,
                                    const float* __restrict__ rope_cos,
                                    const float* __restrict__ rope_sin, int row_pos0, int Hq,
                                    int Hkv, T* __restrict__ q_out, T* __restrict__ kv_layer,
                                    int64_t kv_head_stride) {
  const int m = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int N = (Hq + 2 * Hkv) * 128;
  const int pos = row_pos0 + m;
  const float c = rope_cos[(int64_t)pos * 64 + lane];
  const float s = rope_sin[(int64_t)pos * 64 + lane];
  for (int h = wave; h < Hq + 2 * Hkv; h += blockDim.x >> 6) {
    const int col0 = h * 128 + lane, col1 = col0 + 64;
    float x0 = 0.f, x1 = 0.f;
    for (int p = 0; p < splits; ++p) {
      const float* pr = part + ((int64_t)p * M + m) * N;
      x0 += pr[col0];
      x1 += pr[col1];
    }
    if (rnd_bf16) {
      x0 = round_bf16(x0);
      x1 = round_bf16(x1);
    }
    if (bias) {
      x0 += bf16_bits_to_float(bias[col0]);
      x1 += bf16_bits_to_float(bias[col1]);
    }
    const bool is_q = h < Hq, is_k = !is_q && h < Hq + Hkv;
    if (is_q || is_k) {
      const uint16_t* nw = is_q ? q_norm : k_norm;
      if (nw) {
        const float ms = wave_sum(x0 * x0 + x1 * x1) / 128.f;
        const float inv = 1.f / sqrtf(ms + eps);
        x0 = (x0 * inv) * bf16_bits_to_float(nw[lane]);
        x1 = (x1 * inv) * bf16_bits_to_float(nw[lane + 64]);
      }
      // split-half RoPE: out = x*cos + rotate_half(x)*sin, rotate_half = [-x2, x1]
      const float r0 = x0 * c - x1 * s;
      const float r1 = x1 * c + x0 * s;
      x0 = r0;
      x1 = r1;
    }
    if (is_q) {
      T* qo = q_out + ((int64_t)m * Hq + h) * 128;
      qo[lane] = cvt<T>(x0);
      qo[lane + 64] = cvt<T>(x1);
    } else {
      const int kvh = is_k ? h - Hq : h - Hq - Hkv;
      T* tile = kv_layer + (int64_t)kvh * kv_head_stride + (int64_t)(pos >> 5) * KV_TILE;
      const int kk = pos & 31;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int hd = lane + 64 * e;
        const float val = e ? x1 : x0;
        if (is_k) {
          const int ko = (((hd >> 4) * 2 + ((hd >> 3) & 1)) * 32 + kk) * 8 + (hd & 7);
          tile[ko] = cvt<T>(val);
        } else {
          const int q16 = kk & 15;
          const int vo =
              ((((hd >> 5) * 2 + (kk >> 4)) * 2 + ((q16 >> 2) & 1)) * 32 + (hd & 31)) * 8 +
              (q16 & 3) + 4 * (q16 >> 3);
          tile[4096 + vo] = cvt<T>(val);
        }
      }
    }
  }
}

// SwiGLU epilogue: part [splits][M][2F] of the fused [gate | up] linear.
// One wave per (row, 64-column group) of the F outputs.
extern "C" __global__ void swiglu_kernel(const float* __restrict__ part, int splits, int M, int F,
                                         int rnd_bf16, int fmt, void* __restrict__ act,
                                         float* __restrict__ xsum) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
  const int groups = F >> 6;
  if (wid >= (int64_t)M * groups) return;
  const int m = (int)(wid / groups), g = (int)(wid % groups);
  const int f = g * 64 + lane;
  float gv = 0.f, uv = 0.f;
  for (int p = 0; p < splits; ++p) {
    const float* pr = part + ((int64_t)p * M + m) * (2 * F);
    gv += pr[f];
    uv += pr[F + f];
  }
  if (rnd_bf16) {
    gv = round_bf16(gv);
    uv = round_bf16(uv);
  }
  const float sig = 1.f / (1.f + expf(-gv));
  const float y = gv * sig * uv;
  char* arow = (char*)act + (size_t)m * act_row_bytes(fmt, F);
  write_act(fmt, arow, f, y, xsum ? xsum + (int64_t)m * groups : nullptr, lane);
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

template __global__ void qkv_epilogue_kernel<_Float16>(const float*, int, int, const uint16_t*,
                                                       int, const uint16_t*, const uint16_t*,
                                                       float, const float*, const float*, int,
                                                       int, int, _Float16*, _Float16*, int64_t);
template __global__ void qkv_epilogue_kernel<__bf16>(const float*, int, int, const uint16_t*, int,
                                                     const uint16_t*, const uint16_t*, float,
                                                     const float*, const float*, int, int, int,
                                                     __bf16*, __bf16*, int64_t);

namespace drt {

void embed(const int32_t* tokens, const uint16_t* table, float* hidden, int M, int d,
           hipStream_t s) {
  hipLaunchKernelGGL(embed_kernel, dim3(M), dim3(256), 0, s, tokens, table, hidden, M, d);
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

void qkv_epilogue(bool kv_bf16, const float* part, int splits, int M, const uint16_t* bias,
                  bool rnd_bf16, const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                  const float* rope_cos, const float* rope_sin, int row_pos0, int Hq, int Hkv,
                  void* q_out, void* kv_layer, int64_t kv_head_stride, hipStream_t s) {
  if (kv_bf16)
    hipLaunchKernelGGL(qkv_epilogue_kernel<__bf16>, dim3(M), dim3(256), 0, s, part, splits, M,
                       bias, (int)rnd_bf16, q_norm, k_norm, eps, rope_cos, rope_sin, row_pos0, Hq,
                       Hkv, (__bf16*)q_out, (__bf16*)kv_layer, kv_head_stride);
  else
    hipLaunchKernelGGL(qkv_epilogue_kernel<_Float16>, dim3(M), dim3(256), 0, s, part, splits, M,
                       bias, (int)rnd_bf16, q_norm, k_norm, eps, rope_cos, rope_sin, row_pos0, Hq,
                       Hkv, (_Float16*)q_out, (_Float16*)kv_layer, kv_head_stride);
  DRT_HIP(hipGetLastError());
}

void swiglu(const float* part, int splits, int M, int F, bool rnd_bf16, int fmt, void* act,
            float* xsum, hipStream_t s) {
  require(F % 64 == 0, "swiglu needs F % 64 == 0");
  const int64_t waves = (int64_t)M * (F / 64);
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, part,
                     splits, M, F, (int)rnd_bf16, fmt, act, xsum);
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
