// Weight-streaming q4 linears for decode-sized activations (M <= 32 rows) with
// large weights: the 7B-class decode linears, 7-76 MB of q4 weights each, which
// only reach the HBM roofline if the weight stream never waits on activation
// traffic. The split-K skinny kernels re-read (and re-normalise) a K slice of
// the activation for every 32-128 output columns; at these sizes that is more
// bytes than the weights.
//
// Here a work-group owns one K slice (ng groups of 64) and a range of nblk
// 128-column blocks. It stages the slice's activation (ACT_F16P hi + lo, 8 KB
// per group for 32 rows) in LDS once, computes the 32-row group sums from it,
// and streams its blocks' weights group by group: wave w takes n-tile w of
// every block of the range, so one read of the A fragments from LDS serves
// nblk MFMA chains, and the weights of the next LOOK groups are always in
// flight (a register ring, refilled as each group is consumed). The exact-q
// arithmetic of the other q4 kernels applies (q4_group_mma1: the nibble as an
// exact fp16 integer, y += s * sum(x q) + b * sum(x) in fp32).
//
// Slices of up to 16 groups sit in LDS whole (SINGLE). Longer slices (the
// down projection: K = 18944) go through LDS 16 groups at a time: while a chunk
// is consumed the next one is already loaded into registers, and written to
// LDS between the two (PREF); the weight ring runs on across the chunks.
//
// Output: fp32 K slices y[ks][M][N] (no bias); the consumer reduces them in
// slice order (residual_norm, the q|k|v epilogue, swiglu_slices_kernel,
// sum_slices), so results are deterministic run to run. Reference op:
// backends/mlx_ops.py:97-130 (the q4 affine group-64 linear).
#include "fused.h"
#include "gemm_core.h"
#include "launch.h"
#include "linear_dev.h"

namespace {

constexpr int ST_PAD = 8;     // halves of pad per LDS row (16 B: rows start on different banks)
constexpr int ST_SS_MAX = 8;  // partial sums of squares per thread: K / 32 <= 16 * 8

struct StreamArgs {
  const uint32_t* qw;
  const uint32_t* sb;
  const uint16_t* act;    // ACT: ACT_F16P [M][K] hi plane, lo plane at + M * K
  const float* hidden;    // NORM: fp32 rows [M][K], their RMSNorm weight and the
  const uint16_t* norm_w; // per-32-column partial sums of squares [K / 32][32]
  const float* ss_in;
  float eps;
  int* err;               // DRT_ERR_F16_RANGE when a normed value leaves the fp16 range
  float* y;               // [KS][M][N] fp32 slices
  int M, N, K, KS, R;     // K slices, block ranges
};

// One 64-wide group of one q4 n-tile without its bias term: acc += s * sum(x q),
// the nibbles as exact fp16 integers q (q4_word_to_f16x8), the activation as
// hi + lo fp16 fragments. The bias term b * sum(x) of the group is added later
// for a whole chunk of groups at once (st_bias_mma).
DRT_DEV void st_group_mma(f32x16& acc, const f16x8 (&a)[4], const f16x8 (&al)[4], const u32x4 w,
                          const uint32_t sbv, const Q4Consts& kq) {
  f32x16 c = f32x16{};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const f16x8 b = __builtin_bit_cast(f16x8, q4_word_to_f16x8(w[t], kq));
    c = mfma_f16(a[t], b, c);
    c = mfma_f16(al[t], b, c);
  }
  const float s = bf16_bits_to_float(sbv & 0xffffu);
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = fmaf(s, c[r], acc[r]);
}

// The group sums of a chunk in the A layout of the bias product (lane l: row
// l & 31, k-slots = chunk groups 8 (l >> 5) .. +7; groups past the chunk are
// zero), as three bf16 planes whose sum is the fp32 value exactly.
template <int CH>
DRT_DEV void st_bias_planes(const float* xss, int lane, bf16x8 (&ap)[3]) {
  uint32_t ph[8], pm[8], pl[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int p = 8 * (lane >> 5) + e;
    const float v = p < CH ? xss[min(p, CH - 1) * 32 + (lane & 31)] : 0.f;
    ph[e] = float_to_bf16_bits(v);
    const float r1 = v - bf16_bits_to_float(ph[e]);
    pm[e] = float_to_bf16_bits(r1);
    pl[e] = float_to_bf16_bits(r1 - bf16_bits_to_float(pm[e]));
  }
  u32x4 h, m, l;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h[j] = ph[2 * j] | (ph[2 * j + 1] << 16);
    m[j] = pm[2 * j] | (pm[2 * j + 1] << 16);
    l[j] = pl[2 * j] | (pl[2 * j + 1] << 16);
  }
  ap[0] = __builtin_bit_cast(bf16x8, h);
  ap[1] = __builtin_bit_cast(bf16x8, m);
  ap[2] = __builtin_bit_cast(bf16x8, l);
}

// acc += sum over the chunk's groups (those of parity `half`: the wave's own)
// of bias(g, column) * xsum(g, row): three bf16 MFMAs over k = group (bf16
// products are exact in fp32). bk[k]: the bias bits of chunk group 8 (l >> 5) +
// 2 k + half for this lane's column (zero where the group is not the wave's).
DRT_DEV void st_bias_mma(f32x16& acc, const bf16x8 (&ap)[3], const uint32_t (&bk)[4], int half) {
  u32x4 bw;
#pragma unroll
  for (int k = 0; k < 4; ++k) bw[k] = half ? bk[k] << 16 : bk[k];
  const bf16x8 b = __builtin_bit_cast(bf16x8, bw);
#pragma unroll
  for (int i = 0; i < 3; ++i) acc = mfma_bf16(ap[i], b, acc);
}

// Item j of this thread in a chunk of CH groups: row r, 8-element piece c8 of
// the chunk row (512 threads, CH / 2 items each; the 8 pieces of a group row
// are 8 consecutive lanes).
template <int CH>
DRT_DEV void st_item(int j, int& r, int& c8) {
  const int it = threadIdx.x + 512 * j;
  r = it / (CH * 8);
  c8 = it - r * (CH * 8);
}

// ACT: the chunk's ACT_F16P pieces (clamped to the slice and to row M - 1).
template <int CH>
DRT_DEV void st_load_act(const StreamArgs& a, int cg0, int g_hi, u32x4 (&hi)[CH / 2],
                         u32x4 (&lo)[CH / 2]) {
  const int64_t plane = (int64_t)a.M * a.K;
#pragma unroll
  for (int j = 0; j < CH / 2; ++j) {
    int r, c8;
    st_item<CH>(j, r, c8);
    const int g = min(cg0 + (c8 >> 3), g_hi - 1);
    const int64_t off = (int64_t)min(r, a.M - 1) * a.K + g * 64 + (c8 & 7) * 8;
    hi[j] = *(const u32x4*)(a.act + off);
    lo[j] = *(const u32x4*)(a.act + plane + off);
  }
}

// NORM: the chunk's fp32 rows and norm weights (loads only; st_norm_apply
// norms them once the row factors are known).
template <int CH>
struct NormRaw {
  f32x4 hv[CH / 2][2];
  u32x4 nw[CH / 2];
};
template <int CH>
DRT_DEV void st_norm_load(const StreamArgs& a, int cg0, int g_hi, NormRaw<CH>& raw) {
#pragma unroll
  for (int j = 0; j < CH / 2; ++j) {
    int r, c8;
    st_item<CH>(j, r, c8);
    const int k = min(cg0 + (c8 >> 3), g_hi - 1) * 64 + (c8 & 7) * 8;
    const f32x4* src = (const f32x4*)(a.hidden + (int64_t)min(r, a.M - 1) * a.K + k);
    raw.hv[j][0] = src[0];
    raw.hv[j][1] = src[1];
    raw.nw[j] = *(const u32x4*)(a.norm_w + k);
  }
}
// ... normed into hi / lo pieces (ACT_F16P chunk order 0,4,1,5,2,6,3,7), as the
// RMSNorm prologue of the split-K linears computes them (backends/mlx_ops.py:
// 21-35); true when a value leaves the fp16 range.
template <int CH>
DRT_DEV bool st_norm_apply(const StreamArgs& a, const NormRaw<CH>& raw, const float* rinv,
                           u32x4 (&hi)[CH / 2], u32x4 (&lo)[CH / 2]) {
  bool over = false;
#pragma unroll
  for (int j = 0; j < CH / 2; ++j) {
    int r, c8;
    st_item<CH>(j, r, c8);
    const float inv = r < a.M ? rinv[r] : 0.f;
    _Float16 h[8], l[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t wbits = (e & 1) ? raw.nw[j][e >> 1] >> 16 : raw.nw[j][e >> 1] & 0xffffu;
      const float x = (raw.hv[j][e >> 2][e & 3] * inv) * bf16_bits_to_float(wbits);
      h[e] = (_Float16)x;
      l[e] = f16_lo(x, h[e]);
      over = over || f16_overflows(x);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      hi[j][e] = (uint32_t)half_bits(h[e]) | ((uint32_t)half_bits(h[e + 4]) << 16);
      lo[j][e] = (uint32_t)half_bits(l[e]) | ((uint32_t)half_bits(l[e + 4]) << 16);
    }
  }
  return over;
}

// The chunk's pieces into LDS (rows of CH * 64 + ST_PAD halves) and its group
// sums xss[group][row] = sum of hi + lo over the group's 64 values.
template <int CH>
DRT_DEV void st_store(const u32x4 (&hi)[CH / 2], const u32x4 (&lo)[CH / 2], uint16_t* xs,
                      uint16_t* xsl, float* xss) {
  constexpr int ROWH = CH * 64 + ST_PAD;
#pragma unroll
  for (int j = 0; j < CH / 2; ++j) {
    int r, c8;
    st_item<CH>(j, r, c8);
    *(u32x4*)(xs + r * ROWH + c8 * 8) = hi[j];
    *(u32x4*)(xsl + r * ROWH + c8 * 8) = lo[j];
    const f16x8 h = __builtin_bit_cast(f16x8, hi[j]);
    const f16x8 l = __builtin_bit_cast(f16x8, lo[j]);
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += (float)h[e] + (float)l[e];
    s = sum8_dpp(s);
    if ((c8 & 7) == 0) xss[(c8 >> 3) * 32 + r] = s;
  }
}

}  // namespace

// NBLK: most blocks a work-group's range holds; CH: groups per LDS chunk; PREF:
// the slice takes several chunks, the next one held in registers while the
// current one is consumed; LOOK: steps of weights in flight per wave (divides
// CH / 2); NORM: the input is the fp32 residual stream, RMSNormed while staged.
// 8 waves: wave w takes n-tile w & 3 of every block and the groups of parity
// w >> 2 of each chunk (two waves per SIMD, so one's MFMAs run under the
// other's VALU work); the two halves' sums meet in LDS at the end.
template <int NBLK, int CH, int LOOK, bool NORM, bool PREF>
__global__ __launch_bounds__(512) void stream_q4_kernel(const StreamArgs a) {
  constexpr int HS = CH / 2;  // steps of one half per chunk
  static_assert(HS % LOOK == 0, "the weight ring must cycle within a chunk");
  constexpr int UNR = LOOK < 4 ? 4 : LOOK;  // steps unrolled (the bias slots stay static)
  static_assert(HS % UNR == 0, "the unrolled steps must tile a chunk");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar addressing
  const int tile = wave & 3, half = wave >> 2;
  const int G = a.K >> 6, NB = a.N >> 7, KS = a.KS, R = a.R;
  const int ks = blockIdx.x % KS, rg = blockIdx.x / KS;
  const int g_lo = ks * G / KS, g_hi = (ks + 1) * G / KS;
  const int b_lo = rg * NB / R, nblk = (rg + 1) * NB / R - b_lo;  // 1 .. NBLK (host-checked)
  constexpr int ROWH = CH * 64 + ST_PAD;
  extern __shared__ __align__(16) char smem[];
  uint16_t* xs = (uint16_t*)smem;          // [32][ROWH] hi
  uint16_t* xsl = xs + 32 * ROWH;          // [32][ROWH] lo
  float* xss = (float*)(xsl + 32 * ROWH);  // [CH][32] group sums
  float* rinv = xss + CH * 32;             // [32]
  const Q4Consts kq = q4_consts();

  // n-tile of block j of the range for this wave (blocks past the range repeat
  // the last one: their loads stay valid and their results are not stored)
  int nt[NBLK];
#pragma unroll
  for (int j = 0; j < NBLK; ++j) nt[j] = 4 * (b_lo + min(j, nblk - 1)) + tile;
  // the weight ring of this wave's groups g_lo + half + 2i: step i in slot i % LOOK
  u32x4 wq[LOOK][NBLK];
  uint32_t wsb[LOOK][NBLK];
  auto fetch = [&](int slot, int g) {
    const int gc = min(g, g_hi - 1);
#pragma unroll
    for (int j = 0; j < NBLK; ++j) {
      const int64_t u = (int64_t)nt[j] * G + gc;  // wave-uniform unit index
      wq[slot][j] = __builtin_nontemporal_load((const u32x4*)(a.qw + u * 256) + lane);
      wsb[slot][j] = a.sb[u * 32 + (lane & 31)];
    }
  };
  // the ring's first weights go out after the slice's activation loads: the
  // vector memory counter retires in order, so the staging (from L2) would
  // otherwise wait for the weights (from HBM) before it could start
  auto fill_ring = [&]() {
#pragma unroll
    for (int i = 0; i < LOOK; ++i) fetch(i, g_lo + half + 2 * i);
  };

  u32x4 nhi[HS], nlo[HS];
  NormRaw<CH> raw;  // NORM only (unused registers otherwise)
  auto flag_range = [&](bool over) {
    if (over && a.err)
      __hip_atomic_fetch_or(a.err, DRT_ERR_F16_RANGE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  if (NORM) {
    // the first chunk's rows and norm weights, then the row statistics (the K /
    // 32 partial sums of squares of each row), under one memory latency
    st_norm_load<CH>(a, g_lo, g_hi, raw);
    const int np = a.K >> 5, r = threadIdx.x & 31, p0 = threadIdx.x >> 5;
    float sv[ST_SS_MAX];
#pragma unroll
    for (int e = 0; e < ST_SS_MAX; ++e) sv[e] = a.ss_in[min(p0 + 16 * e, np - 1) * 32 + r];
    fill_ring();
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < ST_SS_MAX; ++e) q += sv[e] * (p0 + 16 * e < np ? 1.f : 0.f);
    float* part_ss = (float*)smem;  // [16][32] scratch (the chunk is staged later)
    part_ss[p0 * 32 + r] = q;
    __syncthreads();
    if (threadIdx.x < 32) {
      float t = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) t += part_ss[e * 32 + threadIdx.x];
      rinv[threadIdx.x] = 1.f / sqrtf(t / (float)a.K + a.eps);
    }
    __syncthreads();
    flag_range(st_norm_apply<CH>(a, raw, rinv, nhi, nlo));
  } else {
    st_load_act<CH>(a, g_lo, g_hi, nhi, nlo);
    fill_ring();
  }
  f32x16 acc[NBLK];
#pragma unroll
  for (int j = 0; j < NBLK; ++j) acc[j] = f32x16{};

  // this wave's groups of the chunk at cg0 (LDS holds it), then the bias term of
  // the chunk's groups
  auto consume = [&](int cg0) {
    uint32_t bk[NBLK][4];
#pragma unroll
    for (int j = 0; j < NBLK; ++j)
#pragma unroll
      for (int k = 0; k < 4; ++k) bk[j][k] = 0u;
    // unrolled over UNR steps (ring slots and bias slots static), looped over
    // the chunk's UNR-step periods (unrolling the whole chunk spills registers)
#pragma unroll 1
    for (int s0 = 0; s0 < HS; s0 += UNR) {
#pragma unroll
      for (int sj = 0; sj < UNR; ++sj) {
        const int si = s0 + sj, gi = 2 * si + half, g = cg0 + gi;
        // the lanes whose bias k-slots hold chunk group gi (8 (l >> 5) <= gi < + 8);
        // UNR is a multiple of 4, so si >> 2 and si & 3 split over s0 and sj
        const bool bias_lanes = (lane >> 5) == (s0 >> 2) + (sj >> 2);
        if (g >= g_hi) break;  // uniform per wave
        const int slot = sj % LOOK;
        const _Float16* arow =
            (const _Float16*)xs + (lane & 31) * ROWH + gi * 64 + 32 * (lane >> 5);
        f16x8 af[4], afl[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          af[t] = *(const f16x8*)(arow + 8 * t);
          afl[t] = *(const f16x8*)(arow + 32 * ROWH + 8 * t);
        }
        // (five blocks: one unit at a time; interleaving five MFMA chains holds
        // five sets of temporaries and spills, and the other wave on the SIMD
        // fills the MFMA gaps)
        // every block of NBLK runs (a range's missing last block repeats its
        // previous one and is never stored): no branches between the units, so
        // their MFMA chains and dequantisation interleave
#pragma unroll
        for (int j = 0; j < NBLK; ++j) {
          st_group_mma(acc[j], af, afl, wq[slot][j], wsb[slot][j], kq);
          if (bias_lanes) bk[j][sj & 3] = wsb[slot][j] >> 16;
        }
        fetch(slot, g + 2 * LOOK);
      }
    }
    bf16x8 ap[3];
    st_bias_planes<CH>(xss, lane, ap);
#pragma unroll
    for (int j = 0; j < NBLK; ++j)
      if (j < nblk) st_bias_mma(acc[j], ap, bk[j], half);
  };
  if (!PREF) {  // the whole slice is one chunk
    st_store<CH>(nhi, nlo, xs, xsl, xss);
    __syncthreads();
    consume(g_lo);
    __syncthreads();
  } else {
    for (int cg0 = g_lo; cg0 < g_hi; cg0 += CH) {
      st_store<CH>(nhi, nlo, xs, xsl, xss);
      __syncthreads();
      const bool more = cg0 + CH < g_hi;
      if (more) {  // the next chunk into registers while this one is consumed
        if (NORM) st_norm_load<CH>(a, cg0 + CH, g_hi, raw);
        else st_load_act<CH>(a, cg0 + CH, g_hi, nhi, nlo);
      }
      consume(cg0);
      if (NORM && more)
        flag_range(st_norm_apply<CH>(a, raw, rinv, nhi, nlo));
      __syncthreads();  // the chunk's LDS is read before the next one overwrites it
    }
  }

  // the two halves' sums meet in LDS: [block][tile][16][64] floats
  float* red = (float*)smem;
  if (half == 1) {
#pragma unroll
    for (int j = 0; j < NBLK; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) red[((j * 4 + tile) * 16 + r) * 64 + lane] = acc[j][r];
  }
  __syncthreads();
  if (half == 1) return;
  // the slice's partial tiles: lane l holds column l & 31 of rows mfma_row(r, l)
  float* yk = a.y + (int64_t)ks * a.M * a.N;
#pragma unroll
  for (int j = 0; j < NBLK; ++j) {
    if (j >= nblk) break;
    const int col = nt[j] * 32 + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = mfma_row(r, lane);
      const float v = acc[j][r] + red[((j * 4 + tile) * 16 + r) * 64 + lane];
      if (row < a.M) yk[(int64_t)row * a.N + col] = v;
    }
  }
}

// hidden += the KS fp32 slices [KS][M][N] of a projection (slice order), and
// the new rows' per-32-column partial sums of squares ss[N / 32][32] (the next
// RMSNorm's statistics, read by a NORM stream linear). Thread: row m, columns
// c0 .. c0 + 3; the 8 threads of a 32-column piece are 8 consecutive lanes.
__global__ __launch_bounds__(256) void residual_slices_kernel(const float* __restrict__ part,
                                                              int KS, int M, int N,
                                                              float* __restrict__ hidden,
                                                              float* __restrict__ ss) {
  const int C4 = N >> 2;
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int m = i / C4, c0 = (i - m * C4) * 4;
  const bool live = m < M;  // whole 8-lane pieces share it (N % 32 == 0)
  const int mr = live ? m : M - 1;
  constexpr int KMAX = 8;
  f32x4 pv[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; ++k)
    pv[k] = *(const f32x4*)(part + ((int64_t)min(k, KS - 1) * M + mr) * N + c0);
  f32x4 h = *(const f32x4*)(hidden + (int64_t)mr * N + c0);
  f32x4 sum = pv[0];
#pragma unroll
  for (int k = 1; k < KMAX; ++k)
    if (k < KS) sum += pv[k];
  h += sum;
  const float q = sum8_dpp(h[0] * h[0] + h[1] * h[1] + h[2] * h[2] + h[3] * h[3]);
  if (!live) return;
  *(f32x4*)(hidden + (int64_t)m * N + c0) = h;
  if ((c0 & 31) == 0) ss[(c0 >> 5) * 32 + m] = q;
}

// SwiGLU of a [gate 64 | up 64]-interleaved projection given as KS fp32 slices
// [KS][M][N] (summed in slice order), written as the ACT_F16P activation
// [M][N / 2] of the down projection (backends/mlx_ops.py:147-154). Thread:
// row m, outputs f0 .. f0 + 7 of one 8-column chunk.
__global__ __launch_bounds__(256) void swiglu_slices_kernel(const float* __restrict__ part, int KS,
                                                            int M, int N, uint16_t* __restrict__ act,
                                                            int* __restrict__ err) {
  const int F = N >> 1, C8 = F >> 3;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= M * C8) return;
  const int m = i / C8, f0 = (i - m * C8) * 8;
  const int col = (f0 >> 6) * 128 + (f0 & 63);
  constexpr int KMAX = 8;
  f32x4 gv[KMAX][2], uv[KMAX][2];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const float* p = part + ((int64_t)min(k, KS - 1) * M + m) * N + col;
    gv[k][0] = *(const f32x4*)p;
    gv[k][1] = *(const f32x4*)(p + 4);
    uv[k][0] = *(const f32x4*)(p + 64);
    uv[k][1] = *(const f32x4*)(p + 68);
  }
  f32x4 g0 = gv[0][0], g1 = gv[0][1], u0 = uv[0][0], u1 = uv[0][1];
#pragma unroll
  for (int k = 1; k < KMAX; ++k)
    if (k < KS) {
      g0 += gv[k][0];
      g1 += gv[k][1];
      u0 += uv[k][0];
      u1 += uv[k][1];
    }
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float g = e < 4 ? g0[e] : g1[e - 4], u = e < 4 ? u0[e] : u1[e - 4];
    y[e] = g * (1.f / (1.f + expf(-g))) * u;
  }
  u32x4 pk, pl;
  bool over = false;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const _Float16 h0 = (_Float16)y[e], h1 = (_Float16)y[e + 4];
    pk[e] = (uint32_t)half_bits(h0) | ((uint32_t)half_bits(h1) << 16);
    pl[e] = (uint32_t)half_bits(f16_lo(y[e], h0)) | ((uint32_t)half_bits(f16_lo(y[e + 4], h1)) << 16);
    over = over || f16_overflows(y[e]) || f16_overflows(y[e + 4]);
  }
  uint16_t* dst = act + (int64_t)m * F + f0;
  *(u32x4*)dst = pk;
  *(u32x4*)(dst + (int64_t)M * F) = pl;
  if (over && err) __hip_atomic_fetch_or(err, DRT_ERR_F16_RANGE, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
}

#define DRT_ST(NB, CH, LK)                                                            \
  template __global__ void stream_q4_kernel<NB, CH, LK, false, false>(const StreamArgs); \
  template __global__ void stream_q4_kernel<NB, CH, LK, true, false>(const StreamArgs);
DRT_ST(1, 16, 8) DRT_ST(2, 16, 8) DRT_ST(3, 16, 4) DRT_ST(4, 16, 4) DRT_ST(5, 16, 2)
// slices longer than one chunk take an ACT_F16P input only (a normed input has
// K = d <= 4096, which the planner always cuts into slices of <= 16 groups)
template __global__ void stream_q4_kernel<1, 16, 8, false, true>(const StreamArgs);
template __global__ void stream_q4_kernel<2, 16, 4, false, true>(const StreamArgs);
#undef DRT_ST

namespace drt {

namespace {
constexpr int ST_SINGLE_MAX_NBLK = 5, ST_PREF_MAX_NBLK = 2;
constexpr int ST_MAX_KS = 8;  // K slices the slice reductions take
// activation chunk (hi, lo), group sums and row factors; the halves' final sums
// (NBLK x 16 KiB) reuse it
size_t st_lds(int ch) {
  return (size_t)2 * 32 * (ch * 64 + ST_PAD) * 2 + (size_t)ch * 32 * 4 + 32 * 4;
}
// (the CU count of the first device asked; every device this library runs on
// is the same part; 256 where no device answers, e.g. a workspace query made
// without a GPU)
int n_cu_of_current_device() {
  static int cached = 0;
  if (!cached) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n < 1) {
      (void)hipGetLastError();
      return 256;
    }
    cached = n;
  }
  return cached;
}
}  // namespace

bool stream_supported(int M, int N, int K) {
  return M >= 1 && M <= 32 && N % 128 == 0 && K % 64 == 0 &&
         (int64_t)N * K >= STREAM_MIN_WEIGHTS;
}

// K slices and block ranges of a streaming linear (one 8-wave work-group per
// CU): the fewest units on the busiest CU, (groups + 4) per block (a block's
// partial tile costs about as much as four groups of weights), over the K
// slices 1 .. max_ks.
StreamPlan stream_plan(int M, int N, int K, int max_ks) {
  StreamPlan best;
  if (!stream_supported(M, N, K)) return best;
  const int G = K / 64, NB = N / 128, n_cu = n_cu_of_current_device();
  int64_t best_cost = -1;
  for (int ks = 1; ks <= std::min({max_ks, G, ST_MAX_KS}); ++ks) {
    const int ng = (G + ks - 1) / ks;
    const bool single = ng <= 16;
    const int max_nblk = single ? ST_SINGLE_MAX_NBLK : ST_PREF_MAX_NBLK;
    const int r = std::min(NB, n_cu / ks);
    if (r < 1) continue;
    const int nblk = (NB + r - 1) / r;
    if (nblk > max_nblk) continue;
    const int64_t cost = (int64_t)nblk * (ng + 4);
    if (best_cost < 0 || cost < best_cost) {
      best_cost = cost;
      best.KS = ks;
      best.R = r;
      best.nblk = nblk;
      best.single = single;
    }
  }
  return best;
}

size_t stream_part_floats(int M, int N, int K, int max_ks) {
  const StreamPlan p = stream_plan(M, N, K, max_ks);
  return p.KS ? (size_t)p.KS * M * N : 0;
}

void stream_linear(const FusedArgs& f, const StreamPlan& p, hipStream_t s) {
  const bool norm = f.hidden != nullptr;
  require(p.KS >= 1 && f.qw && f.sb && f.y && f.M <= 32 && f.N % 128 == 0 && f.K % 64 == 0 &&
              (norm ? f.norm_w && f.ss_in && f.K / 32 <= 16 * ST_SS_MAX : f.act != nullptr),
          "streaming linear: unsupported arguments");
  StreamArgs a{f.qw, f.sb, (const uint16_t*)f.act, f.hidden, f.norm_w, f.ss_in, f.eps,
               f.placement_err, f.y, f.M, f.N, f.K, p.KS, p.R};
  const dim3 grid((unsigned)(p.R * p.KS));
  const double bytes = (double)f.N * f.K * 0.5625 + 4.0 * f.M * f.K + 4.0 * p.KS * f.M * f.N;
#define DRT_STL(NB, CH, LK)                                                             \
  {                                                                                      \
    auto fn = norm ? stream_q4_kernel<NB, CH, LK, true, false>                           \
                   : stream_q4_kernel<NB, CH, LK, false, false>;                         \
    static size_t granted = 0;                                                           \
    grant_lds((const void*)fn, st_lds(CH), granted);                                     \
    DRT_LAUNCH(Profiler::GEMM, bytes, fn, grid, dim3(512), st_lds(CH), s, a);            \
  }
#define DRT_STP(NB, CH, LK)                                                             \
  {                                                                                      \
    auto fn = stream_q4_kernel<NB, CH, LK, false, true>;                                 \
    static size_t granted = 0;                                                           \
    grant_lds((const void*)fn, st_lds(CH), granted);                                     \
    DRT_LAUNCH(Profiler::GEMM, bytes, fn, grid, dim3(512), st_lds(CH), s, a);            \
  }
  if (p.single) {
    switch (p.nblk) {
      // (weights in flight: 8-16 units per wave, 72-144 KiB per CU)
      case 1: DRT_STL(1, 16, 8) break;
      case 2: DRT_STL(2, 16, 8) break;
      case 3: DRT_STL(3, 16, 4) break;
      case 4: DRT_STL(4, 16, 4) break;
      case 5: DRT_STL(5, 16, 2) break;
      default: fail(INTERNAL_ERROR, "streaming linear: bad plan");
    }
  } else {
    require(!norm, "streaming linear: a normed input must fit one chunk per slice");
    if (p.nblk == 1) DRT_STP(1, 16, 8) else if (p.nblk == 2) DRT_STP(2, 16, 4)
    else fail(INTERNAL_ERROR, "streaming linear: bad plan");
  }
#undef DRT_STP
#undef DRT_STL
  DRT_HIP(hipGetLastError());
}

void swiglu_slices(const float* part, int KS, int M, int N, void* act, int* err, hipStream_t s) {
  require(KS >= 1 && KS <= 8 && N % 128 == 0 && M >= 1, "swiglu_slices: 1..8 slices, N % 128");
  const int n = M * (N / 16);
  hipLaunchKernelGGL(swiglu_slices_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     part, KS, M, N, (uint16_t*)act, err);
  DRT_HIP(hipGetLastError());
}

void residual_slices(const float* part, int KS, int M, int N, float* hidden, float* ss,
                     hipStream_t s) {
  require(KS >= 1 && KS <= 8 && N % 32 == 0 && M >= 1 && M <= 32,
          "residual_slices: 1..8 slices, N % 32, <= 32 rows");
  const int n = M * (N / 4);
  hipLaunchKernelGGL(residual_slices_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     part, KS, M, N, hidden, ss);
  DRT_HIP(hipGetLastError());
}

}  // namespace drt
