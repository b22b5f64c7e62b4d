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
#include "fused.h"
#include "gemm_core.h"
#include "launch.h"
#include "lmstat.h"

#include <cstdlib>
#include <type_traits>

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
  // work-group b of the one-dimensional grid takes (column group x, row tile z)
  // = (t / Z, t % Z) with t dealt to the XCDs in contiguous runs (work-group b
  // runs on XCD b % 8; t = (b % 8) * T8 / 8 + b / 8, the last T - T8 as they
  // come): the row tiles of a column group run on one XCD together, so its
  // weights come from HBM once and from that XCD's L2 for the other row tiles
  const int Z = (M + 31) / 32, T = (int)gridDim.x, T8 = T & ~7, b = (int)blockIdx.x;
  const int t = b < T8 ? (b & 7) * (T8 >> 3) + (b >> 3) : b;
  const int m0 = (t % Z) * 32;
  const int wblk = (t / Z) * WAVES + wave;  // 64-column block of this wave
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

// ---------------------------------------------------------------------------
// q4 LM head over a persistent grid (K = 1024): one 8-wave work-group per CU
// owns a contiguous range of 32-column tiles and stages the 32-row activation
// tile (hi and lo planes, 128 KiB) into LDS once, with direct-to-LDS loads; its
// waves take the tiles in turn (wave w: tiles w, w + 8, ...), each keeping the
// next tile's 16 groups of weights in flight while it multiplies the current
// one. The bias term sum_g b_g * xsum_g goes through three bf16 MFMAs per tile
// (the group sums split into three bf16 planes, exact), so the per-group VALU
// work is the dequantisation and one scale fma per result. Statistics are
// joined per row over the work-group's columns: one LmStat per (row,
// work-group), in column order, for lmhead_finalize_kernel.
namespace {

constexpr int LMP_WAVES = 8;
constexpr int LMP_G = 16;                    // 64-k groups: K = 1024
constexpr int LMP_PF = 8;                    // weight groups in flight per wave
constexpr int LMP_ROW = LMP_G * 64 + 8;      // halves per LDS activation row (+16 B)
constexpr int LMP_TRS = 40;                  // floats per transpose row
constexpr int LMP_TR = 16 * LMP_TRS;         // floats of a wave's half-tile transpose
constexpr size_t LMP_ACT_BYTES = (size_t)2 * 32 * LMP_ROW * 2;
constexpr size_t LMP_XS_OFF = LMP_ACT_BYTES + (size_t)LMP_WAVES * LMP_TR * 4;
constexpr size_t LMP_LDS = LMP_XS_OFF + 3 * 64 * 16;  // + the bias product's A planes
constexpr float LMP_L2E = 1.44269504088896340736f;

// Running statistics of one row over the columns seen so far (in increasing
// column order): max, sum of exp(l - max), first column of the max, and the
// sampling draw (best l + T g, its column and logit).
struct RowRun {
  float m, s;
  int arg;
  int sarg;
  double skey;
  float sl;
};

DRT_DEV RowRun rowrun_empty() { return RowRun{-INFINITY, 0.f, 0x7fffffff, 0x7fffffff, -INFINITY, 0.f}; }

// a and b cover disjoint column sets; equal maxima (and equal keys) go to the
// lower column, so the join does not depend on the order of its operands.
DRT_DEV RowRun rowrun_join(const RowRun& a, const RowRun& b) {
  RowRun r;
  r.m = fmaxf(a.m, b.m);
  const float ea = a.m == r.m ? 1.f : __builtin_amdgcn_exp2f((a.m - r.m) * LMP_L2E);
  const float eb = b.m == r.m ? 1.f : __builtin_amdgcn_exp2f((b.m - r.m) * LMP_L2E);
  r.s = a.s * ea + b.s * eb;
  r.arg = (a.m > b.m || (a.m == b.m && a.arg < b.arg)) ? a.arg : b.arg;
  const bool ka = a.skey > b.skey || (a.skey == b.skey && a.sarg < b.sarg);
  r.skey = ka ? a.skey : b.skey;
  r.sarg = ka ? a.sarg : b.sarg;
  r.sl = ka ? a.sl : b.sl;
  return r;
}

DRT_DEV RowRun rowrun_shfl_xor(const RowRun& a, int o) {
  RowRun r;
  r.m = __shfl_xor(a.m, o, 64);
  r.s = __shfl_xor(a.s, o, 64);
  r.arg = __shfl_xor(a.arg, o, 64);
  r.sarg = __shfl_xor(a.sarg, o, 64);
  r.skey = __shfl_xor(a.skey, o, 64);
  r.sl = __shfl_xor(a.sl, o, 64);
  return r;
}

}  // namespace

// WK = 0 (q4): x is ACT_F16P (hi + lo planes) with group sums xsum. WK = 1
// (bf16 tile weights in qw's place, sb unused): x is ACT_BF16 (one plane), four
// bf16 MFMAs per 64-k group, the logits rounded to bf16 before the statistics
// (the reference's bf16 matmul output), four groups in flight per wave.
template <int WK>
__global__ __launch_bounds__(64 * LMP_WAVES) void lmhead_q4p_kernel(
    const uint32_t* __restrict__ qw, const uint32_t* __restrict__ sb,
    const uint16_t* __restrict__ x, const float* __restrict__ xsum, int M, int N,
    float* __restrict__ logits_out, LmStat* __restrict__ stats, float temperature_arg,
    uint64_t seed_arg, int step_arg, const int32_t* __restrict__ positions,
    const StepDesc* __restrict__ desc, int exclude_arg) {
  constexpr bool BF = WK == 1;
  constexpr int G = LMP_G, K = G * 64, W = LMP_WAVES;
  constexpr int PF = BF ? 4 : LMP_PF;  // weight groups in flight per wave
  constexpr int FR = BF ? 4 : 1;       // 16-byte fragments per group and lane
  constexpr int PLANES = BF ? 1 : 2;
  const float temperature = desc ? desc->temperature : temperature_arg;
  const uint64_t seed = desc ? desc->seed : seed_arg;
  const int step = desc ? desc->step : step_arg;
  const int excl = desc ? desc->exclude_col : exclude_arg;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int m0 = blockIdx.z * 32;
  const int U = N >> 5, nwg = gridDim.x, wg = blockIdx.x;
  const uint16_t* wb = (const uint16_t*)qw;
  // group g of tile nt, fragment f: q4 words or a bf16 16-k MFMA fragment
  auto wfrag = [&](int nt, int g, int f) {
    return BF ? (const u32x4*)bf16_tile_frag(wb, nt, K >> 4, 4 * g + f, lane)
              : q4_tile_words(qw, nt, G, g, lane);
  };
  const int ub = (int)((int64_t)U * wg / nwg), ue = (int)((int64_t)U * (wg + 1) / nwg);
  const int n_mine = ue - ub > wave ? (ue - ub - wave + W - 1) / W : 0;
  extern __shared__ __align__(16) char smem[];
  uint16_t* act = (uint16_t*)smem;  // [2 planes][32 rows][LMP_ROW]
  float* tr = (float*)(smem + LMP_ACT_BYTES) + wave * LMP_TR;

  // 1. the first tile's weights (a wave without tiles loads a valid one, unused)
  // weights in flight: a ring of PF groups (group g in slot g % PF)
  u32x4 wq[PF][FR];
  uint32_t wsb[PF];
  {
    const int nt = min(ub + wave, U - 1);
#pragma unroll
    for (int g = 0; g < PF; ++g) {
#pragma unroll
      for (int f = 0; f < FR; ++f) wq[g][f] = __builtin_nontemporal_load(wfrag(nt, g, f));
      wsb[g] = BF ? 0u : __builtin_nontemporal_load(&sb[((int64_t)nt * G + g) * 32 + (lane & 31)]);
    }
  }
  // 2. the activation tile into LDS: 128 chunks of 1 KiB (plane, row, half row);
  // rows past M repeat row M - 1 (their results are never stored)
#pragma unroll
  for (int i = 0; i < 64 * PLANES / W; ++i) {
    const int ch = wave + W * i, p = ch >> 6, r = (ch >> 1) & 31, hf = ch & 1;
    const int m = min(m0 + r, M - 1);
    const uint16_t* src = x + ((int64_t)p * M + m) * K + hf * 512 + lane * 8;
    __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)(
                                         act + (p * 32 + r) * LMP_ROW + hf * 512),
                                     16, 0, 0);
  }
  // 3. the group sums as three bf16 planes (exact split of the fp32 value) in
  // the A layout of the bias product: lane l, row l & 31, groups 8 (l >> 5) .. +7
  u32x4* xsp = (u32x4*)(smem + LMP_XS_OFF);  // [3 planes][64 lanes]
  if (!BF && wave == 0) {
    const int mr = m0 + (lane & 31);
    f32x4 xa = f32x4{0.f, 0.f, 0.f, 0.f}, xb = xa;
    if (mr < M) {
      const f32x4* xp = (const f32x4*)(xsum + (int64_t)mr * G + 8 * (lane >> 5));
      xa = xp[0];
      xb = xp[1];
    }
    uint32_t ph[8], pm[8], pl[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = e < 4 ? xa[e] : xb[e - 4];
      ph[e] = float_to_bf16_bits(v);
      const float r1 = v - bf16_bits_to_float(ph[e]);
      pm[e] = float_to_bf16_bits(r1);
      pl[e] = float_to_bf16_bits(r1 - bf16_bits_to_float(pm[e]));
    }
    u32x4 h, md, lo;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h[j] = ph[2 * j] | (ph[2 * j + 1] << 16);
      md[j] = pm[2 * j] | (pm[2 * j + 1] << 16);
      lo[j] = pl[2 * j] | (pl[2 * j + 1] << 16);
    }
    xsp[lane] = h;
    xsp[64 + lane] = md;
    xsp[128 + lane] = lo;
  }
  // sampling: the row keys of this lane's two rows (lane >> 2 and 16 + lane >> 2)
  const bool sampling = temperature > 0.f;
  const int rowa = m0 + (lane >> 2), rowb = rowa + 16;
  const bool va = rowa < M, vb = rowb < M;
  uint64_t rka = 0, rkb = 0;
  if (sampling && va) rka = sampling_row_key(seed, step, positions[rowa]);
  if (sampling && vb) rkb = sampling_row_key(seed, step, positions[rowb]);
  __builtin_amdgcn_s_waitcnt(0);  // this wave's LDS chunks (and the first weights) landed
  __builtin_amdgcn_s_barrier();   // ... and every other wave's
  asm volatile("" ::: "memory");

  const Q4Consts kq = q4_consts();
  const _Float16* arow = (const _Float16*)act + (lane & 31) * LMP_ROW + 32 * (lane >> 5);
  RowRun runa = rowrun_empty(), runb = rowrun_empty();

  // statistics of one half tile (rows 16 PH .. +15) through the wave's LDS
  // area: lane takes row lane >> 2, columns 8 (lane & 3) .. +7 of the tile
  auto half_tile = [&](const f32x16& acc, int nt, auto ph_c, RowRun& run, uint64_t rk, bool rv) {
    constexpr int PH = decltype(ph_c)::value;
    const bool ex = nt * 32 + (lane & 31) == excl;
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) {
      const int r = 8 * PH + rr;
      tr[(mfma_row(r, lane) - 16 * PH) * LMP_TRS + (lane & 31)] = ex ? -INFINITY : acc[r];
    }
    const int q = lane >> 2, j4 = lane & 3;
    const int c0 = nt * 32 + 8 * j4;
    const f32x4 v0 = *(const f32x4*)(tr + q * LMP_TRS + 8 * j4);
    const f32x4 v1 = *(const f32x4*)(tr + q * LMP_TRS + 8 * j4 + 4);
    float v[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = v0[e];
      v[e + 4] = v1[e];
    }
    RowRun t;
    t.m = v[0];
    t.arg = c0;
#pragma unroll
    for (int e = 1; e < 8; ++e)
      if (v[e] > t.m) { t.m = v[e]; t.arg = c0 + e; }
    const float mb = t.m * LMP_L2E;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += __builtin_amdgcn_exp2f(fmaf(v[e], LMP_L2E, -mb));
    t.s = s;
    t.skey = -INFINITY;
    t.sarg = 0x7fffffff;
    t.sl = 0.f;
    if (sampling && rv) {
      const double T = (double)temperature;
      for (int e = 0; e < 8; ++e) {
        const double key = __dadd_rn((double)v[e], __dmul_rn(T, (double)gumbel(rk, c0 + e)));
        if (key > t.skey) { t.skey = key; t.sarg = c0 + e; t.sl = v[e]; }
      }
    }
    run = rowrun_join(run, t);
  };

  // one 32-column tile: 16 groups (each: 8 MFMAs and one scale fma per result),
  // the next tile's weights loaded into the registers each group frees
  auto tile = [&](int nt, auto prefetch) {
    // the activation fragments are the same for every tile: without this
    // barrier the compiler would hoist their LDS reads out of the tile loop
    // and hold all 16 groups (512 registers) live
    asm volatile("" ::: "memory");
    f32x16 acc = f32x16{};
    uint32_t bpk[8];
    const int ntn = nt + W;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int sl = g % PF;
      // keep each group's work in its place: the LDS reads and the
      // dequantisation would otherwise be hoisted to the tile start for every
      // group at once (registers for all of them)
      asm volatile("" ::: "memory");
      if (BF) {  // k = 64 g + 16 t + 8 (lane >> 5) + e, natural order
        const uint16_t* brow = (const uint16_t*)arow - 32 * (lane >> 5) + 8 * (lane >> 5);
#pragma unroll
        for (int t = 0; t < FR; ++t) {
          u32x4 wv = wq[sl][t];
          asm volatile("" : "+v"(wv));
          acc = mfma_bf16(*(const bf16x8*)(brow + g * 64 + 16 * t), __builtin_bit_cast(bf16x8, wv), acc);
        }
      } else {
        u32x4 wv = wq[sl][0];
        asm volatile("" : "+v"(wv));
        f16x8 a[4], al[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          a[t] = *(const f16x8*)(arow + g * 64 + 8 * t);
          al[t] = *(const f16x8*)(arow + 32 * LMP_ROW + g * 64 + 8 * t);
        }
        f32x16 c = f32x16{};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const f16x8 b = __builtin_bit_cast(f16x8, q4_word_to_f16x8(wv[t], kq));
          c = mfma_f16(a[t], b, c);
          c = mfma_f16(al[t], b, c);
        }
        const float s = bf16_bits_to_float(wsb[sl] & 0xffffu);
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = fmaf(s, c[r], acc[r]);
        // bias of group g into the bf16 B operand of the bias product
        if (g & 1) bpk[g >> 1] |= wsb[sl] & 0xffff0000u;
        else bpk[g >> 1] = wsb[sl] >> 16;
      }
      // the slot's next group: g + PF of this tile, else g + PF - G of the next
      if (g + PF < G || decltype(prefetch)::value) {
        const int tn = g + PF < G ? nt : ntn, gn = g + PF < G ? g + PF : g + PF - G;
#pragma unroll
        for (int f = 0; f < FR; ++f) wq[sl][f] = __builtin_nontemporal_load(wfrag(tn, gn, f));
        if (!BF)
          wsb[sl] = __builtin_nontemporal_load(&sb[((int64_t)tn * G + gn) * 32 + (lane & 31)]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (BF) {
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = round_bf16(acc[r]);
    } else {
      const bool hi_half = lane >= 32;
      u32x4 bb;
#pragma unroll
      for (int j = 0; j < 4; ++j) bb[j] = hi_half ? bpk[4 + j] : bpk[j];
      const bf16x8 bv = __builtin_bit_cast(bf16x8, bb);
#pragma unroll
      for (int p = 0; p < 3; ++p)
        acc = mfma_bf16(__builtin_bit_cast(bf16x8, xsp[64 * p + lane]), bv, acc);
    }

    if (logits_out) {
      // rows m0 + 4 (lane >> 5) + 8 (r >> 2) + (r & 3): per-r offsets are uniform
      const int rl = m0 + 4 * (lane >> 5);
      float* lp = logits_out + (int64_t)rl * N + nt * 32 + (lane & 31);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int dr = 8 * (r >> 2) + (r & 3);
        if (rl + dr < M) lp[(int64_t)dr * N] = acc[r];
      }
    }
    half_tile(acc, nt, std::integral_constant<int, 0>{}, runa, rka, va);
    half_tile(acc, nt, std::integral_constant<int, 1>{}, runb, rkb, vb);
  };
  for (int i = 0; i < n_mine; ++i) {
    const int nt = ub + wave + W * i;
    if (i + 1 < n_mine) tile(nt, std::true_type{});
    else tile(nt, std::false_type{});
  }

  // the four column quarters of a row, then the waves, in LDS over the activation
  runa = rowrun_join(runa, rowrun_shfl_xor(runa, 1));
  runa = rowrun_join(runa, rowrun_shfl_xor(runa, 2));
  runb = rowrun_join(runb, rowrun_shfl_xor(runb, 1));
  runb = rowrun_join(runb, rowrun_shfl_xor(runb, 2));
  __syncthreads();  // every wave is done with the activation tile
  RowRun* js = (RowRun*)smem;  // [W][32]
  if ((lane & 3) == 0) {
    js[wave * 32 + (lane >> 2)] = runa;
    js[wave * 32 + 16 + (lane >> 2)] = runb;
  }
  __syncthreads();
  if (threadIdx.x < 32) {
    const int row = threadIdx.x;
    RowRun r = js[row];
#pragma unroll
    for (int w = 1; w < W; ++w) r = rowrun_join(r, js[w * 32 + row]);
    if (m0 + row < M) {
      LmStat st;
      st.m = r.m;
      st.s = r.s;
      st.arg = r.arg;
      st.sarg = r.sarg;
      st.skey = r.skey;
      st.sl = r.sl;
      st.pad = 0.f;
      stats[(int64_t)(m0 + row) * nwg + wg] = st;
    }
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
    // last: a wait for a load also waits for the stores before it, and this
    // one crosses the bus to host memory
    if (err_host && row == 0)
      *err_host = __hip_atomic_load(err_dev, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The fixed-quota choice of one block step on the device
// (backends/diffusion_runtime.py:290-299, the top-k of the confidences, and
// :1200-1346, its commit): of the desc->n_lm LM rows (positions[r]) whose canvas
// token is still the mask, the desc->quota with the highest scores take their
// proposed token; equal scores go to the lower row (the lower position), as the
// host loop's stable order does. One wave, n_lm <= 64; rows are distinct
// positions, and every canvas read happens before any write. A NaN score ranks
// below every number.
// The fixed-quota choice of one step: `quota` of the n LM rows whose canvas
// token is still the mask take their proposed token, highest scores first.
__device__ __forceinline__ void commit_quota(const double* __restrict__ scores,
                                             const int32_t* __restrict__ tokens,
                                             const int32_t* __restrict__ positions,
                                             int32_t* __restrict__ canvas, int mask_id,
                                             int quota, int n) {
  const int r = threadIdx.x;
  const bool row = r < n;
  const int pos = row ? positions[r] : 0;
  const bool masked = row && canvas[pos] == mask_id;
  // a NaN score ranks as -inf, as in the library's host loop (the comparisons
  // below then stay a strict order: score descending, row ascending)
  const double s0 = row ? scores[r] : 0.0;
  const double sc = s0 != s0 ? -INFINITY : s0;
  int rank = 0;
  for (int j = 0; j < n; ++j) {
    const double sj = __shfl(sc, j, 64);
    const int mj = __shfl((int)masked, j, 64);
    rank += (mj && (sj > sc || (sj == sc && j < r))) ? 1 : 0;
  }
  if (masked && rank < quota) canvas[pos] = tokens[r];
}

// One wave. `advance` (may be desc itself, so neither is restrict) receives the
// next step's sampling index and quota, from quota_tab indexed by step modulo
// QUOTA_TAB: a device block's later steps replay one graph on one descriptor.
extern "C" __global__ void block_commit_kernel(const double* __restrict__ scores,
                                               const int32_t* __restrict__ tokens,
                                               const int32_t* __restrict__ positions,
                                               int32_t* __restrict__ canvas, int mask_id,
                                               const StepDesc* desc, StepDesc* advance,
                                               const int32_t* __restrict__ quota_tab) {
  const int quota = desc->quota, n = min(desc->n_lm, 64), step = desc->step;
  if (quota > 0) commit_quota(scores, tokens, positions, canvas, mask_id, quota, n);
  // every lane's loads of desc completed before its values were used above
  if (advance && threadIdx.x == 0) {
    advance->step = step + 1;
    advance->quota = quota_tab[(step + 1) & (QUOTA_TAB - 1)];
  }
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
  int NB = w.N / 64;
  constexpr int WAVES = 4;
  // K = 1024 heads (q4 or bf16) run on the persistent kernel, other K on the
  // large-M GEMM (q4, more than 64 rows) or the chunked kernel
  if (w.K == LMP_G * 64) {
    int dev = 0, n_cu = 0;
    DRT_HIP(hipGetDevice(&dev));
    DRT_HIP(hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev));
    const int U = w.N / 32;
    NB = std::max(1, std::min(n_cu, U / LMP_WAVES));  // one work-group per CU
    if (w.q4) {
      auto fn = lmhead_q4p_kernel<0>;
      static size_t granted = 0;
      grant_lds((const void*)fn, LMP_LDS, granted);
      const double bytes = (double)w.N * w.K / 2 + (double)w.N * w.K / 16 + 2.0 * M * w.K;
      DRT_LAUNCH(Profiler::LMHEAD, bytes, fn, dim3(NB, 1, (M + 31) / 32), dim3(64 * LMP_WAVES),
                 LMP_LDS, s, w.qw.as<uint32_t>(), w.sb.as<uint32_t>(), (const uint16_t*)act,
                 xsum, M, w.N, logits_out, (LmStat*)stats, temperature, seed, step, positions,
                 desc, exclude_col);
    } else {
      auto fn = lmhead_q4p_kernel<1>;
      static size_t granted = 0;
      grant_lds((const void*)fn, LMP_LDS, granted);
      const double bytes = 2.0 * w.N * w.K + 2.0 * M * w.K;
      DRT_LAUNCH(Profiler::LMHEAD, bytes, fn, dim3(NB, 1, (M + 31) / 32), dim3(64 * LMP_WAVES),
                 LMP_LDS, s, (const uint32_t*)w.wb.as<uint16_t>(), (const uint32_t*)nullptr,
                 (const uint16_t*)act, xsum, M, w.N, logits_out, (LmStat*)stats, temperature,
                 seed, step, positions, desc, exclude_col);
    }
  } else if (w.q4 && M > 64) {
    // more than two 32-row tiles of a q4 head of another K (Dream's canvas rows):
    // the large-M GEMM, whose 128 x 256 tiles dequantize the weights once per
    // 128 rows, with the statistics epilogue (the same records, N / 64 per row).
    // Dream's head (N = 152064, K = 3584): 272 us for 65-128 rows, 462 us for
    // 129-256, against about 120 us per 32-row tile on the chunked kernel.
    FusedArgs f;
    f.qw = w.qw.as<uint32_t>();
    f.sb = w.sb.as<uint32_t>();
    f.M = M;
    f.N = w.N;
    f.K = w.K;
    f.act = act;
    f.act_fmt = ACT_F16P;
    f.desc = desc;
    f.lm_stats = stats;
    f.lm_logits = logits_out;
    f.lm_pos = positions;
    f.lm_temp = temperature;
    f.lm_seed = seed;
    f.lm_step = step;
    f.lm_excl = exclude_col;
    big_linear(f, FL_LMSTAT, 1, s);
  } else {
  const size_t lds = (size_t)(w.q4 ? 2 : 1) * 32 * (chunk_k + 8) * 2 +
                     (size_t)32 * (chunk_k / 64) * 4 + (size_t)WAVES * 32 * 65 * 4;
  const dim3 grid((unsigned)(((NB + WAVES - 1) / WAVES) * ((M + 31) / 32)));  // (column group, row tile) pairs
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
                  int32_t* canvas, int mask_id, const StepDesc* desc, hipStream_t s,
                  StepDesc* advance, const int32_t* quota_tab) {
  require(desc && scores_d && tokens_d && positions && canvas,
          "block_commit needs the step descriptor, device scores, tokens, positions and canvas");
  require(!advance || quota_tab, "block_commit: a descriptor advance needs the quota table");
  hipLaunchKernelGGL(block_commit_kernel, dim3(1), dim3(64), 0, s, scores_d, tokens_d, positions,
                     canvas, mask_id, desc, advance, quota_tab);
  DRT_HIP(hipGetLastError());
}

}  // namespace drt
