// Fused LM head + vocab softmax statistics + scoring for gfx950.
//
// Scoring restated from backends/diffusion_runtime.py:179-192 (greedy) and
// :203-275 (temperature sampling):
//   greedy:  p = softmax_f64(logits); score = max p = 1 / sum_v exp(l_v - max),
//            token = first argmax (np.argmax keeps the lowest index).
//   T > 0:   token = argmax(l + T * g) with Gumbel g = -log(-log u) in float32,
//            u from a splitmix64 counter hash of (seed, forward, position, token);
//            the product and the sum are rounded separately in float64;
//            score = exp(l_token - max) / sum.
//
// lmhead_kernel computes a 32-row x 64-column logits block per wave (q4 or bf16
// weights) and reduces it to per-row block statistics (max, first argmax,
// sum of exp(l - block max) in fp32, sampling candidate), so the logits only
// leave the chip when the caller asks for them. lmhead_finalize_kernel joins
// the blocks of a row in float64.
#include "gemm_core.h"
#include "launch.h"

struct LmStat {
  float m;       // block max logit
  float s;       // sum exp(l - m) over the block (fp32)
  int arg;       // first column attaining m
  int sarg;      // sampling: column of the best key
  double skey;   // sampling: best l + T * g
  float sl;      // sampling: logit at sarg
  float pad;
};

namespace {

constexpr uint64_t GOLDEN = 0x9E3779B97F4A7C15ull;

DRT_DEV uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

DRT_DEV uint64_t sampling_row_key(uint64_t seed, int step, int position) {
  uint64_t key = mix64(seed + GOLDEN);
  key = mix64(key + (uint64_t)(int64_t)(step + 1) * GOLDEN);
  return mix64(key + (uint64_t)(int64_t)(position + 1) * GOLDEN);
}

DRT_DEV float gumbel(uint64_t row_key, int token) {
  const uint64_t bits = mix64(row_key + (uint64_t)(token + 1) * GOLDEN);
  const float u = ((float)(uint32_t)(bits >> 41) + 0.5f) * 0x1p-23f;
  return -logf(-logf(u));
}

}  // namespace

// WK = 0: q4 tile32-g64 weights + ACT_F16P activation (hi and lo planes of M
// rows, group sums of hi + lo); WK = 1: bf16 tile weights
// + ACT_BF16 activation (logits rounded to bf16, as the reference's bf16 matmul).
// Grid: x = ceil(N / (64 * WAVES)), y = 1, z = ceil(M / 32). NT is fixed to 2.
template <int WK, int WAVES, int P>
__global__ __launch_bounds__(64 * WAVES) void lmhead_kernel(
    const uint32_t* __restrict__ qw, const uint32_t* __restrict__ sb,
    const uint16_t* __restrict__ wb, const void* __restrict__ x,
    const float* __restrict__ xsum, int M, int N, int K, int chunk_k,
    float* __restrict__ logits_out, LmStat* __restrict__ stats, float temperature_arg,
    uint64_t seed_arg, int step_arg, const int32_t* __restrict__ positions,
    const StepDesc* __restrict__ desc, int exclude_arg) {
  // sampling controls come from the step descriptor when one is given (graph replays)
  const float temperature = desc ? desc->temperature : temperature_arg;
  const uint64_t seed = desc ? desc->seed : seed_arg;
  const int step = desc ? desc->step : step_arg;
  // a column left out of the statistics (the canvas MASK token of threshold
  // policies, backends/diffusion_runtime.py:256-282): -inf for max, sum and draw
  const int excl = desc ? desc->exclude_col : exclude_arg;
  constexpr int NT = 2;
  const int G = K >> 6, KC = K >> 4;
  const int NTILES = N >> 5, NB = N >> 6;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m0 = blockIdx.z * 32;
  const int wblk = blockIdx.x * WAVES + wave;  // 64-column block of this wave
  const bool active = wblk < NB;
  const int nt0 = active ? wblk * NT : 0;

  extern __shared__ __align__(16) char smem[];
  const int row_h = chunk_k + 8;
  constexpr int PLANES = WK == 0 ? 2 : 1;  // ACT_F16P: hi rows, then lo rows
  char* xs_raw = smem;                      // [PLANES][32][row_h]
  float* xss = (float*)(smem + (size_t)PLANES * 32 * row_h * 2);
  float* ttile = (float*)(smem + (size_t)PLANES * 32 * row_h * 2 +
                          (size_t)32 * (chunk_k >> 6) * 4) +
                 wave * (32 * 65);

  f32x16 acc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[j] = f32x16{};

  for (int k0 = 0; k0 < K; k0 += chunk_k) {
    const int ck = min(chunk_k, K - k0);
    __syncthreads();
    const int cpr = ck / 8;
    for (int c = threadIdx.x; c < PLANES * 32 * cpr; c += 64 * WAVES) {
      const int pr = c / cpr, cc = c - pr * cpr;  // pr = plane * 32 + row
      const int m = m0 + (pr & 31);
      u32x4 v = {0u, 0u, 0u, 0u};
      if (m < M)
        v = *(const u32x4*)((const uint16_t*)x + ((int64_t)(pr >> 5) * M + m) * K + k0 + cc * 8);
      *(u32x4*)((uint16_t*)xs_raw + pr * row_h + cc * 8) = v;
    }
    if (WK == 0) {
      const int ngc = ck >> 6;
      for (int c = threadIdx.x; c < 32 * ngc; c += 64 * WAVES) {
        const int gg = c >> 5, r = c & 31;
        const int m = m0 + r;
        xss[c] = (m < M) ? xsum[(int64_t)m * G + (k0 >> 6) + gg] : 0.f;
      }
    }
    __syncthreads();
    if (!active) continue;
    if (WK == 0) {
      const int gbase = k0 >> 6, ng = ck >> 6;
      const _Float16* arow = (const _Float16*)xs_raw + (lane & 31) * row_h + 32 * (lane >> 5);
      u32x4 wbuf[P][NT];
      uint32_t sbuf[P][NT];
#pragma unroll
      for (int p = 0; p < P; ++p)
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          const int g = gbase + min(p, ng - 1);
          wbuf[p][j] = __builtin_nontemporal_load(q4_tile_words(qw, nt0 + j, G, g, lane));
          sbuf[p][j] = __builtin_nontemporal_load(&sb[((int64_t)(nt0 + j) * G + g) * 32 + (lane & 31)]);
        }
      for (int gb = 0; gb < ng; gb += P) {
#pragma unroll
        for (int p = 0; p < P; ++p) {
          const int gg = gb + p;
          if (gg < ng) {
            f16x8 a[4], al[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              a[t] = *(const f16x8*)(arow + gg * 64 + 8 * t);
              al[t] = *(const f16x8*)(arow + 32 * row_h + gg * 64 + 8 * t);
            }
            float xsr[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) xsr[r] = xss[gg * 32 + mfma_row(r, lane)];
            q4_group_mma<NT>(acc, a, al, xsr, wbuf[p], sbuf[p]);
            const int gn = gg + P;
            if (gn < ng) {
#pragma unroll
              for (int j = 0; j < NT; ++j) {
                wbuf[p][j] = __builtin_nontemporal_load(q4_tile_words(qw, nt0 + j, G, gbase + gn, lane));
                sbuf[p][j] = __builtin_nontemporal_load(
                    &sb[((int64_t)(nt0 + j) * G + gbase + gn) * 32 + (lane & 31)]);
              }
            }
          }
        }
      }
    } else {
      const int cbase = k0 >> 4, nc = ck >> 4;
      const uint16_t* arow = (const uint16_t*)xs_raw + (lane & 31) * row_h + 8 * (lane >> 5);
      bf16x8 wbuf[P][NT];
#pragma unroll
      for (int p = 0; p < P; ++p)
#pragma unroll
        for (int j = 0; j < NT; ++j) wbuf[p][j] = *bf16_tile_frag(wb, nt0 + j, KC, cbase + min(p, nc - 1), lane);
      for (int cb = 0; cb < nc; cb += P) {
#pragma unroll
        for (int p = 0; p < P; ++p) {
          const int cc = cb + p;
          if (cc < nc) {
            const bf16x8 a = *(const bf16x8*)(arow + cc * 16);
#pragma unroll
            for (int j = 0; j < NT; ++j) acc[j] = mfma_bf16(a, wbuf[p][j], acc[j]);
            const int cn = cc + P;
            if (cn < nc) {
#pragma unroll
              for (int j = 0; j < NT; ++j) wbuf[p][j] = *bf16_tile_frag(wb, nt0 + j, KC, cbase + cn, lane);
            }
          }
        }
      }
    }
  }

  // Epilogue: logits block -> LDS transpose -> per-row statistics.
  if (active) {
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float v = acc[j][r];
        if (WK == 1) v = round_bf16(v);
        const int row = mfma_row(r, lane);
        ttile[row * 65 + j * 32 + (lane & 31)] =
            (nt0 + j) * 32 + (lane & 31) == excl ? -INFINITY : v;
        if (logits_out && m0 + row < M)
          logits_out[(int64_t)(m0 + row) * N + (nt0 + j) * 32 + (lane & 31)] = v;
      }
  }
  __syncthreads();
  if (!active) return;
  const int row = lane >> 1, half = lane & 1;
  const float* tv = ttile + row * 65 + half * 32;
  const int col0 = wblk * 64 + half * 32;
  float mx = tv[0];
  int arg = col0;
  for (int c = 1; c < 32; ++c) {
    const float v = tv[c];
    if (v > mx) { mx = v; arg = col0 + c; }
  }
  float se = 0.f;
  for (int c = 0; c < 32; ++c) se += expf(tv[c] - mx);
  double skey = -INFINITY;
  int sarg = col0;
  float sl = tv[0];
  if (temperature > 0.f && m0 + row < M) {
    const uint64_t rk = sampling_row_key(seed, step, positions[m0 + row]);
    const double T = (double)temperature;
    for (int c = 0; c < 32; ++c) {
      const double key = __dadd_rn((double)tv[c], __dmul_rn(T, (double)gumbel(rk, col0 + c)));
      if (key > skey) { skey = key; sarg = col0 + c; sl = tv[c]; }
    }
  }
  // Join with the partner lane (the other 32 columns of this row).
  const float mx2 = __shfl_xor(mx, 1, 64);
  const int arg2 = __shfl_xor(arg, 1, 64);
  const float se2 = __shfl_xor(se, 1, 64);
  const double skey2 = __shfl_xor(skey, 1, 64);
  const int sarg2 = __shfl_xor(sarg, 1, 64);
  const float sl2 = __shfl_xor(sl, 1, 64);
  if (half == 0 && m0 + row < M) {
    LmStat st;
    st.m = fmaxf(mx, mx2);
    st.arg = mx >= mx2 ? arg : arg2;  // this lane holds the lower columns
    st.s = se * expf(mx - st.m) + se2 * expf(mx2 - st.m);
    const bool take2 = skey2 > skey;
    st.skey = take2 ? skey2 : skey;
    st.sarg = take2 ? sarg2 : sarg;
    st.sl = take2 ? sl2 : sl;
    st.pad = 0.f;
    stats[(int64_t)(m0 + row) * NB + wblk] = st;
  }
}

// One 256-thread WG per row: join the N/64 block statistics in float64. scores
// and tokens may be pinned host memory (the session's landing area: no copy
// after the forward); scores_d / tokens_d (optional) get the same values in
// device memory; err_host, when given, receives the forward's placement and
// bounded-wait flags (*err_dev, final once the earlier kernels are done).
extern "C" __global__ void lmhead_finalize_kernel(const LmStat* __restrict__ stats, int NB,
                                                  int sampling_arg,
                                                  const StepDesc* __restrict__ desc,
                                                  double* __restrict__ scores,
                                                  int32_t* __restrict__ tokens,
                                                  double* __restrict__ scores_d,
                                                  int32_t* __restrict__ tokens_d,
                                                  const int* __restrict__ err_dev,
                                                  int* __restrict__ err_host) {
  const int sampling = desc ? (desc->temperature > 0.f) : sampling_arg;
  __shared__ float red_f[4];
  __shared__ int red_i[4];
  __shared__ double red_d[4];
  __shared__ int red_j[4];
  const int row = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (err_host && row == 0 && threadIdx.x == 0)
    *err_host = __hip_atomic_load(err_dev, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const LmStat* st = stats + (int64_t)row * NB;
  // pass 1: global max and its first block
  float mx = -INFINITY;
  int mb = 0x7fffffff;
  for (int b = threadIdx.x; b < NB; b += blockDim.x) {
    if (st[b].m > mx) { mx = st[b].m; mb = b; }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(mx, o, 64);
    const int b2 = __shfl_xor(mb, o, 64);
    if (m2 > mx || (m2 == mx && b2 < mb)) { mx = m2; mb = b2; }
  }
  if (lane == 0) { red_f[wave] = mx; red_i[wave] = mb; }
  __syncthreads();
  mx = red_f[0];
  mb = red_i[0];
  for (int w = 1; w < 4; ++w)
    if (red_f[w] > mx || (red_f[w] == mx && red_i[w] < mb)) { mx = red_f[w]; mb = red_i[w]; }
  if (mb < 0 || mb >= NB) mb = 0;  // all-NaN row: keep the index in bounds
  const double M = (double)mx;
  // pass 2: float64 sum and (optional) the best sampling key
  double s = 0.0;
  double bk = -INFINITY;
  int bj = 0x7fffffff;
  for (int b = threadIdx.x; b < NB; b += blockDim.x) {
    s += (double)st[b].s * exp((double)st[b].m - M);
    if (sampling && st[b].skey > bk) { bk = st[b].skey; bj = b; }
  }
  s = wave_sum_d(s);
  for (int o = 32; o > 0; o >>= 1) {
    const double k2 = __shfl_xor(bk, o, 64);
    const int j2 = __shfl_xor(bj, o, 64);
    if (k2 > bk || (k2 == bk && j2 < bj)) { bk = k2; bj = j2; }
  }
  __syncthreads();
  __shared__ double red_k[4];
  if (lane == 0) { red_d[wave] = s; red_j[wave] = bj; red_k[wave] = bk; }
  __syncthreads();
  if (threadIdx.x == 0) {
    double tot = 0.0;
    for (int w = 0; w < 4; ++w) tot += red_d[w];
    double sc;
    int32_t tk;
    if (!sampling) {
      sc = 1.0 / tot;
      tk = st[mb].arg;
    } else {
      double k = red_k[0];
      int j = red_j[0];
      for (int w = 1; w < 4; ++w)
        if (red_k[w] > k || (red_k[w] == k && red_j[w] < j)) { k = red_k[w]; j = red_j[w]; }
      if (j < 0 || j >= NB) j = 0;  // all keys NaN: keep the index in bounds
      tk = st[j].sarg;
      sc = exp((double)st[j].sl - M) / tot;
    }
    scores[row] = sc;
    tokens[row] = tk;
    if (scores_d) {
      scores_d[row] = sc;
      tokens_d[row] = tk;
    }
  }
}

// The fixed-quota choice of one block step on the device
// (backends/diffusion_runtime.py:290-299, the top-k of the confidences, and
// :1200-1346, its commit): of the desc->n_lm LM rows (positions[r]) whose canvas
// token is still the mask, the desc->quota with the highest scores take their
// proposed token; equal scores go to the lower row (the lower position), as the
// host loop's stable order does. One wave, n_lm <= 64; rows are distinct
// positions, and every canvas read happens before any write.
extern "C" __global__ void block_commit_kernel(const double* __restrict__ scores,
                                               const int32_t* __restrict__ tokens,
                                               const int32_t* __restrict__ positions,
                                               int32_t* __restrict__ canvas, int mask_id,
                                               const StepDesc* __restrict__ desc) {
  const int quota = desc->quota, n = min(desc->n_lm, 64);
  if (quota <= 0) return;
  const int r = threadIdx.x;
  const bool row = r < n;
  const int pos = row ? positions[r] : 0;
  const bool masked = row && canvas[pos] == mask_id;
  const double sc = row ? scores[r] : 0.0;
  int rank = 0;
  for (int j = 0; j < n; ++j) {
    const double sj = __shfl(sc, j, 64);
    const int mj = __shfl((int)masked, j, 64);
    rank += (mj && (sj > sc || (sj == sc && j < r))) ? 1 : 0;
  }
  if (masked && rank < quota) canvas[pos] = tokens[r];
}

template __global__ void lmhead_kernel<0, 4, 4>(const uint32_t*, const uint32_t*, const uint16_t*,
                                                const void*, const float*, int, int, int, int,
                                                float*, LmStat*, float, uint64_t, int,
                                                const int32_t*, const StepDesc*, int);
template __global__ void lmhead_kernel<1, 4, 8>(const uint32_t*, const uint32_t*, const uint16_t*,
                                                const void*, const float*, int, int, int, int,
                                                float*, LmStat*, float, uint64_t, int,
                                                const int32_t*, const StepDesc*, int);

namespace drt {

size_t lmhead_stats_bytes(int M, int N) { return (size_t)M * (N / 64) * sizeof(LmStat); }

void lmhead(const LinearW& w, const void* act, const float* xsum, int M, float* logits_out,
            void* stats, float temperature, uint64_t seed, int step, const int32_t* positions,
            double* scores, int32_t* tokens, hipStream_t s, const StepDesc* desc,
            int exclude_col, const int* err_dev, int* err_host, double* scores_d,
            int32_t* tokens_d) {
  require(w.N % 64 == 0, "lm head needs vocab % 64 == 0");
  require(M >= 1, "lm head needs at least one row");
  // k per LDS chunk: q4 stages hi and lo rows, so half the k of bf16 keeps the
  // work-group at <= 66 KiB of LDS (two per CU)
  const int chunk_k = std::min(w.q4 ? 256 : 512, w.K);
  require(w.K % chunk_k == 0 || w.K % 64 == 0, "lm head K must be a multiple of 64");
  const int NB = w.N / 64;
  constexpr int WAVES = 4;
  const size_t lds = (size_t)(w.q4 ? 2 : 1) * 32 * (chunk_k + 8) * 2 +
                     (size_t)32 * (chunk_k / 64) * 4 + (size_t)WAVES * 32 * 65 * 4;
  const dim3 grid((NB + WAVES - 1) / WAVES, 1, (M + 31) / 32);
  if (w.q4) {
    auto fn = lmhead_kernel<0, WAVES, 4>;
    static size_t granted = 0;
    grant_lds((const void*)fn, lds, granted);
    const double bytes = (double)w.N * w.K / 2 + (double)w.N * w.K / 16 + 2.0 * M * w.K;
    DRT_LAUNCH(Profiler::LMHEAD, bytes, fn, grid, dim3(64 * WAVES), lds, s, w.qw.as<uint32_t>(),
               w.sb.as<uint32_t>(), (const uint16_t*)nullptr, act, xsum, M, w.N, w.K, chunk_k,
               logits_out, (LmStat*)stats, temperature, seed, step, positions, desc,
               exclude_col);
  } else {
    auto fn = lmhead_kernel<1, WAVES, 8>;
    static size_t granted = 0;
    grant_lds((const void*)fn, lds, granted);
    const double bytes = 2.0 * w.N * w.K + 2.0 * M * w.K;
    DRT_LAUNCH(Profiler::LMHEAD, bytes, fn, grid, dim3(64 * WAVES), lds, s,
               (const uint32_t*)nullptr, (const uint32_t*)nullptr, w.wb.as<uint16_t>(), act, xsum,
               M, w.N, w.K, chunk_k, logits_out, (LmStat*)stats, temperature, seed, step,
               positions, desc, exclude_col);
  }
  DRT_HIP(hipGetLastError());
  if (scores && tokens) {
    hipLaunchKernelGGL(lmhead_finalize_kernel, dim3(M), dim3(256), 0, s, (const LmStat*)stats, NB,
                       (int)(temperature > 0.f), desc, scores, tokens, scores_d, tokens_d,
                       err_dev, err_host);
    DRT_HIP(hipGetLastError());
  }
}

void block_commit(const double* scores_d, const int32_t* tokens_d, const int32_t* positions,
                  int32_t* canvas, int mask_id, const StepDesc* desc, hipStream_t s) {
  require(desc && scores_d && tokens_d && positions && canvas,
          "block_commit needs the step descriptor, device scores, tokens, positions and canvas");
  hipLaunchKernelGGL(block_commit_kernel, dim3(1), dim3(64), 0, s, scores_d, tokens_d, positions,
                     canvas, mask_id, desc);
  DRT_HIP(hipGetLastError());
}

}  // namespace drt
