// The LM head's per-block softmax statistics record and the sampling hash,
// shared by every kernel that scores vocabulary columns (the LM head kernels
// and the large-M GEMM's statistics epilogue).
//
// Scoring restated from backends/diffusion_runtime.py:179-192 (greedy) and
// :203-275 (temperature sampling): the Gumbel draw g = -log(-log u) in float32,
// u from a splitmix64 counter hash of (seed, forward, position, token).
#pragma once
#include "common.h"

struct LmStat {
  float m;       // block max logit
  float s;       // sum exp(l - m) over the block (fp32)
  int arg;       // first column attaining m
  int sarg;      // sampling: column of the best key
  double skey;   // sampling: best l + T * g
  float sl;      // sampling: logit at sarg
  float pad;
};

constexpr uint64_t LM_GOLDEN = 0x9E3779B97F4A7C15ull;

DRT_DEV uint64_t lm_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

DRT_DEV uint64_t sampling_row_key(uint64_t seed, int step, int position) {
  uint64_t key = lm_mix64(seed + LM_GOLDEN);
  key = lm_mix64(key + (uint64_t)(int64_t)(step + 1) * LM_GOLDEN);
  return lm_mix64(key + (uint64_t)(int64_t)(position + 1) * LM_GOLDEN);
}

DRT_DEV float gumbel(uint64_t row_key, int token) {
  const uint64_t bits = lm_mix64(row_key + (uint64_t)(token + 1) * LM_GOLDEN);
  const float u = ((float)(uint32_t)(bits >> 41) + 0.5f) * 0x1p-23f;
  return -logf(-logf(u));
}

// Statistics of 32 consecutive columns col0 .. col0 + 31 of one row (v[c]; an
// excluded column already -inf), the row's sampling key rk when sampling: max
// and its first column, sum of exp(l - max) in column order, and the best
// l + T g (the first column on ties).
struct LmRun32 {
  float mx, se, sl;
  int arg, sarg;
  double skey;
};

DRT_DEV LmRun32 lm_run32(const float (&v)[32], int col0, bool sampling, float temperature,
                         uint64_t rk) {
  LmRun32 r;
  r.mx = v[0];
  r.arg = col0;
  for (int c = 1; c < 32; ++c)
    if (v[c] > r.mx) { r.mx = v[c]; r.arg = col0 + c; }
  r.se = 0.f;
  for (int c = 0; c < 32; ++c) r.se += expf(v[c] - r.mx);
  r.skey = -INFINITY;
  r.sarg = col0;
  r.sl = v[0];
  if (sampling) {
    const double T = (double)temperature;
    for (int c = 0; c < 32; ++c) {
      const double key = __dadd_rn((double)v[c], __dmul_rn(T, (double)gumbel(rk, col0 + c)));
      if (key > r.skey) { r.skey = key; r.sarg = col0 + c; r.sl = v[c]; }
    }
  }
  return r;
}

// One 64-column block's record from its two halves (a: the lower columns).
DRT_DEV LmStat lm_join64(const LmRun32& a, const LmRun32& b) {
  LmStat st;
  st.m = fmaxf(a.mx, b.mx);
  st.arg = a.mx >= b.mx ? a.arg : b.arg;
  st.s = a.se * expf(a.mx - st.m) + b.se * expf(b.mx - st.m);
  const bool take2 = b.skey > a.skey;
  st.skey = take2 ? b.skey : a.skey;
  st.sarg = take2 ? b.sarg : a.sarg;
  st.sl = take2 ? b.sl : a.sl;
  st.pad = 0.f;
  return st;
}
