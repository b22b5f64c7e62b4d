// Fused linear for gfx950: prologue -> split-K GEMM inside one work-group ->
// fused epilogue. One kernel per linear of the decoder layer.
//
// A work-group owns a 32-row tile and WN n-tiles of 32 columns; its WN*WK
// waves split the K range WK ways, so every output tile is complete inside
// the work-group (reduced through LDS in a fixed order: deterministic) and no
// fp32 partials travel through global memory.
//
// Prologues (what is staged in LDS as the A operand, 1024 k at a time):
//   PRO_ACT : an activation already in the linear's format (ACT_F16P + group
//             sums for q4, ACT_BF16 for bf16 weights).
//   PRO_NORM: RMSNorm(hidden) * w computed on the fly from the fp32 residual
//             stream (backends/mlx_ops.py:21-35): the work-group reads its rows'
//             full K, so it computes the row statistic itself.
// Epilogues (on the final fp32 tile; bf16 weights round it to bf16 first, as the
// reference's bf16 matmul output is, backends/mlx_ops.py:122-125):
//   EPI_STORE : y = tile (+ bias)
//   EPI_RESID : hidden += tile                     (o_proj, down_proj residual adds)
//   EPI_QKV   : one head per work-group: (+ bias), per-head q/k RMSNorm, split-half
//               RoPE at the row's absolute position, Q out, K/V into the tiled cache
//               (backends/mlx_forward.py:1164-1361, mlx_ops.py:133-144)
//   EPI_SWIGLU: [gate 64 | up 64] column blocks -> silu(g) * u -> activation of the
//               down projection (mlx_ops.py:147-154)
#include "fused.h"
#include "gemm_core.h"
#include "launch.h"

#include "linear_dev.h"

// Stage RMSNorm(hidden[m0 .. m0+31][kc0 .. kc0+1023]) * w into LDS as the A
// operand (ACT_F16P + group sums, or ACT_BF16). Each thread owns 8 consecutive
// k of a row per item (two float4 loads, all issued before any use); rinv holds
// the rows' 1/rms. One latency instead of one per (row, group).
template <int WKIND, int NTHR, int JB, int ITEMS>
DRT_DEV void stage_norm_items(const FusedArgs& a, int m0, int kc0, int kcn, uint16_t* xs,
                              float* xss, const float* rinv, int row_h) {
  const int ipr = kcn / 8;                // items per row in this chunk
  f32x4 v[ITEMS][2];
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const int it = threadIdx.x + (JB + j) * NTHR;
    const int r = it >> 7, c8 = it & 127;
    const int m = m0 + r;
    if (c8 < ipr && m < a.M) {
      const f32x4* src = (const f32x4*)(a.hidden + (int64_t)m * a.K + kc0 + c8 * 8);
      v[j][0] = src[0];
      v[j][1] = src[1];
    } else {
      v[j][0] = f32x4{0.f, 0.f, 0.f, 0.f};
      v[j][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const int it = threadIdx.x + (JB + j) * NTHR;
    const int r = it >> 7, c8 = it & 127;
    const float inv = rinv[r];
    const int k = kc0 + c8 * 8;
    const uint32_t* wp = (const uint32_t*)(a.norm_w + (c8 < ipr ? k : kc0));
    const uint32_t w01 = wp[0], w23 = wp[1], w45 = wp[2], w67 = wp[3];
    float x[8];
    x[0] = (v[j][0][0] * inv) * bf16_bits_to_float(w01 & 0xffffu);
    x[1] = (v[j][0][1] * inv) * bf16_bits_to_float(w01 >> 16);
    x[2] = (v[j][0][2] * inv) * bf16_bits_to_float(w23 & 0xffffu);
    x[3] = (v[j][0][3] * inv) * bf16_bits_to_float(w23 >> 16);
    x[4] = (v[j][1][0] * inv) * bf16_bits_to_float(w45 & 0xffffu);
    x[5] = (v[j][1][1] * inv) * bf16_bits_to_float(w45 >> 16);
    x[6] = (v[j][1][2] * inv) * bf16_bits_to_float(w67 & 0xffffu);
    x[7] = (v[j][1][3] * inv) * bf16_bits_to_float(w67 >> 16);
    if (WKIND == W_Q4) {
      // ACT_F16P hi / lo planes (the lo plane 32 rows after the hi plane in
      // LDS): the 8-chunk stored in the order (0,4,1,5,2,6,3,7)
      _Float16 h[8], lo[8];
      bool over = false;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        h[e] = (_Float16)x[e];
        lo[e] = f16_lo(x[e], h[e]);
        over = over || f16_overflows(x[e]);
      }
      if (over && m0 + r < a.M && c8 < ipr) raise_range(a);
      u32x4 pk, pl;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pk[e] = (uint32_t)half_bits(h[e]) | ((uint32_t)half_bits(h[e + 4]) << 16);
        pl[e] = (uint32_t)half_bits(lo[e]) | ((uint32_t)half_bits(lo[e + 4]) << 16);
      }
      if (c8 < ipr) {
        *(u32x4*)(xs + r * row_h + c8 * 8) = pk;
        *(u32x4*)(xs + (32 + r) * row_h + c8 * 8) = pl;
      }
      float gs = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) gs += (float)h[e] + (float)lo[e];
      // a 64-k group is 8 consecutive items = 8 consecutive lanes
      gs += __shfl_xor(gs, 1, 64);
      gs += __shfl_xor(gs, 2, 64);
      gs += __shfl_xor(gs, 4, 64);
      if ((c8 & 7) == 0 && c8 < ipr) xss[(c8 >> 3) * 32 + r] = gs;
    } else {
      u32x4 pk;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        pk[e] = (uint32_t)float_to_bf16_bits(x[2 * e]) |
                ((uint32_t)float_to_bf16_bits(x[2 * e + 1]) << 16);
      if (c8 < ipr) *(u32x4*)(xs + r * row_h + c8 * 8) = pk;
    }
  }
}

// All items of a 1024-k chunk: at once for q4 (one latency); in two batches for
// bf16, whose prefetched weight fragments leave fewer free registers.
template <int WKIND, int NTHR>
DRT_DEV void stage_norm_chunk(const FusedArgs& a, int m0, int kc0, int kcn, uint16_t* xs,
                              float* xss, const float* rinv, int row_h) {
  constexpr int ITEMS = 32 * 128 / NTHR;  // 8-wide items per thread
  if constexpr (WKIND == W_Q4 || ITEMS < 2) {
    stage_norm_items<WKIND, NTHR, 0, ITEMS>(a, m0, kc0, kcn, xs, xss, rinv, row_h);
  } else {
    stage_norm_items<WKIND, NTHR, 0, ITEMS / 2>(a, m0, kc0, kcn, xs, xss, rinv, row_h);
    stage_norm_items<WKIND, NTHR, ITEMS / 2, ITEMS - ITEMS / 2>(a, m0, kc0, kcn, xs, xss, rinv,
                                                                 row_h);
  }
}

template <int WKIND, int WN, int WK, int PRO, int EPI>
__global__ __launch_bounds__(64 * WN * WK) void fused_linear_kernel(const FusedArgs a) {
  constexpr int NW = WN * WK;
  constexpr int NTHR = 64 * NW;
  constexpr int KPU = WKIND == W_Q4 ? 64 : 16;   // k per unit (q4 group / bf16 MFMA chunk)
  constexpr int CH = 1024 / KPU;                  // units per LDS chunk (1024 k)
  constexpr int UPW = CH / WK;                    // units per wave per chunk
  static_assert(CH % WK == 0, "WK must divide the chunk");
  constexpr int ROW_H = 1024 + 8;                 // 16-bit elements per LDS row (+16 B pad)
  // One n-tile per work-group and a ready-made activation: every wave reads its
  // own A fragments straight from global memory (nothing to share through LDS).
  constexpr bool DIRECT = PRO == PRO_ACT && WN == 1;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wn = wave % WN, wk = wave / WN;
  const int M = a.M, N = a.N, K = a.K;
  const int m0 = blockIdx.y * 32;
  const int NTILES = N >> 5;
  const int nt = blockIdx.x * WN + wn;
  const bool active = nt < NTILES;
  const int ntc = active ? nt : NTILES - 1;  // clamped: loads stay in bounds
  const int units = K / KPU;
  const int G = K >> 6;
  const int KC = K >> 4;

  extern __shared__ __align__(16) char smem[];
  uint16_t* xs = (uint16_t*)smem;                               // [2][32][ROW_H] (q4: hi, lo)
  float* xss = (float*)(smem + 2 * 32 * ROW_H * 2);              // [16][32]
  float* rinv = xss + 16 * 32;                                   // [32]
  float* rss = rinv + 32;                                        // [32][NW] row partials

  f32x16 acc = f32x16{};
  if constexpr (DIRECT) {
    // this wave's contiguous K slice, P units in flight (1024-thread work-groups
    // leave 128 VGPRs per lane: two q4 units of A fragments + weights fit)
    constexpr int P = WKIND == W_Q4 ? 2 : 4;
    const int u_lo = (int)((int64_t)units * wk / WK), u_hi = (int)((int64_t)units * (wk + 1) / WK);
    const int mrow = m0 + (lane & 31);
    const bool row_ok = mrow < M;
    const int mr = row_ok ? mrow : 0;
    u32x4 wq[P], af[P][4], afl[P][4];
    uint32_t wsb[P];
    bf16x8 wbf[P], ab[P];
    auto fetch = [&](int slot, int unit) {
      unit = min(unit, units - 1);
      if (WKIND == W_Q4) {
        wq[slot] = *q4_tile_words(a.qw, ntc, G, unit, lane);
        wsb[slot] = q4_tile_sb(a.sb, ntc, G, unit, lane);
        const u32x4* ap = (const u32x4*)((const uint16_t*)a.act + (int64_t)mr * K + unit * 64 +
                                         32 * (lane >> 5));
        const u32x4* apl = ap + (int64_t)M * K / 8;  // the lo plane
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          af[slot][t] = row_ok ? ap[t] : u32x4{0u, 0u, 0u, 0u};
          afl[slot][t] = row_ok ? apl[t] : u32x4{0u, 0u, 0u, 0u};
        }
      } else {
        wbf[slot] = *bf16_tile_frag(a.wb, ntc, KC, unit, lane);
        const bf16x8* ap = (const bf16x8*)((const uint16_t*)a.act + (int64_t)mr * K + unit * 16 +
                                           8 * (lane >> 5));
        ab[slot] = row_ok ? *ap : bf16x8{};
      }
    };
#pragma unroll
    for (int p = 0; p < P; ++p) fetch(p, u_lo + p);
    for (int ub = u_lo; ub < u_hi; ub += P) {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const int u = ub + p;
        if (u < u_hi) {
          if (WKIND == W_Q4) {
            // (the LDS staging area is unused on this path: 32 floats per wave)
            q4_group_mma1_lane(acc, af[p], afl[p], wq[p], wsb[p], lane,
                               (float*)smem + (threadIdx.x >> 6) * 32);
          } else {
            acc = mfma_bf16(ab[p], wbf[p], acc);
          }
          if (u + P < u_hi) fetch(p, u + P);
        }
      }
    }
  } else {
    // This wave's units of a chunk are wk*UPW .. wk*UPW+UPW-1; their weights
    // stream through a P-deep register ring that carries over into the next chunk.
    constexpr int P = UPW < 4 ? UPW : 4;
    u32x4 wq[P];
    uint32_t wsb[P];
    bf16x8 wbf[P];
    auto load_unit = [&](int slot, int unit) {
      unit = min(unit, units - 1);
      if (WKIND == W_Q4) {
        wq[slot] = *q4_tile_words(a.qw, ntc, G, unit, lane);
        wsb[slot] = q4_tile_sb(a.sb, ntc, G, unit, lane);
      } else {
        wbf[slot] = *bf16_tile_frag(a.wb, ntc, KC, unit, lane);
      }
    };
#pragma unroll
    for (int p = 0; p < P; ++p) load_unit(p, wk * UPW + p);

    if (PRO == PRO_NORM) {
      // row statistic over the full K: 8-wide items, one partial per (row, wave)
      float part[32 * 128 / NTHR];
      const int ipr_all = K / 8;
      for (int r = 0; r < 32; ++r) (void)r;
      for (int j = 0; j < 32 * 128 / NTHR; ++j) part[j] = 0.f;
      for (int kb = 0; kb < K; kb += 1024) {
#pragma unroll
        for (int j = 0; j < 32 * 128 / NTHR; ++j) {
          const int it = threadIdx.x + j * NTHR;
          const int r = it >> 7, c8 = (it & 127) + kb / 8;
          const int m = m0 + r;
          if (c8 < ipr_all && m < M) {
            const f32x4* src = (const f32x4*)(a.hidden + (int64_t)m * K + c8 * 8);
            const f32x4 p0 = src[0], p1 = src[1];
            part[j] += p0[0] * p0[0] + p0[1] * p0[1] + p0[2] * p0[2] + p0[3] * p0[3] +
                       p1[0] * p1[0] + p1[1] * p1[1] + p1[2] * p1[2] + p1[3] * p1[3];
          }
        }
      }
      // a row's 128 items are 128 consecutive threads = two full waves
#pragma unroll
      for (int j = 0; j < 32 * 128 / NTHR; ++j) {
        const float t = wave_sum(part[j]);
        const int r = (threadIdx.x + j * NTHR) >> 7;
        if (lane == 0) rss[r * 2 + ((threadIdx.x >> 6) & 1)] = t;
      }
      __syncthreads();
      if (threadIdx.x < 32)
        rinv[threadIdx.x] = 1.f / sqrtf((rss[threadIdx.x * 2] + rss[threadIdx.x * 2 + 1]) / (float)K + a.eps);
    }

    for (int c0u = 0; c0u < units; c0u += CH) {
      const int cu = min(CH, units - c0u);
      const int kc0 = c0u * KPU, kcn = cu * KPU;
      __syncthreads();  // rinv ready / previous chunk's LDS reads done
      if (PRO == PRO_ACT) {
        const int vpr = kcn / 8;
        const int planes = WKIND == W_Q4 ? 2 : 1;  // ACT_F16P: hi and lo planes
        for (int i = threadIdx.x; i < planes * 32 * vpr; i += NTHR) {
          const int pr = i / vpr, v = i - pr * vpr;  // pr = plane * 32 + row
          const int r = pr & 31, pl = pr >> 5;
          const int m = m0 + r;
          u32x4 val = {0u, 0u, 0u, 0u};
          if (m < M)
            val = *(const u32x4*)((const uint16_t*)a.act + ((int64_t)pl * M + m) * K + kc0 + v * 8);
          *(u32x4*)(xs + pr * ROW_H + v * 8) = val;
        }
        if (WKIND == W_Q4) {
          for (int i = threadIdx.x; i < 32 * (kcn / 64); i += NTHR) {
            const int gg = i >> 5, r = i & 31;
            const int m = m0 + r;
            xss[i] = (m < M) ? a.act_xsum[(int64_t)m * G + (kc0 >> 6) + gg] : 0.f;
          }
        }
      } else {
        stage_norm_chunk<WKIND, NTHR>(a, m0, kc0, kcn, xs, xss, rinv, ROW_H);
      }
      __syncthreads();
      if (active) {
#pragma unroll
        for (int ub = 0; ub < UPW; ub += P) {
#pragma unroll
          for (int p = 0; p < P; ++p) {
            const int u = ub + p;
            const int uc = wk * UPW + u;  // unit within the chunk
            if (uc < cu) {
              if (WKIND == W_Q4) {
                const _Float16* arow =
                    (const _Float16*)xs + (lane & 31) * ROW_H + uc * 64 + 32 * (lane >> 5);
                f16x8 af[4], afl[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                  af[t] = *(const f16x8*)(arow + 8 * t);
                  afl[t] = *(const f16x8*)(arow + 32 * ROW_H + 8 * t);
                }
                float xsr[16];
#pragma unroll
                for (int r = 0; r < 16; ++r) xsr[r] = xss[uc * 32 + mfma_row(r, lane)];
                q4_group_mma1(acc, af, afl, xsr, wq[p], wsb[p]);
              } else {
                const bf16x8 af =
                    *(const bf16x8*)(xs + (lane & 31) * ROW_H + uc * 16 + 8 * (lane >> 5));
                acc = mfma_bf16(af, wbf[p], acc);
              }
            }
            // refill this slot with the unit P places ahead (maybe in the next chunk)
            const int nu = u + P;
            if (nu < UPW) load_unit(p, c0u + wk * UPW + nu);
            else if (c0u + CH < units) load_unit(p, c0u + CH + wk * UPW + (nu - UPW));
          }
        }
      }
    }
  }

  // Reduce the WK partial tiles of each n-tile in LDS, in a fixed order.
  __syncthreads();
  float* red = (float*)smem;  // [WK][WN][32][33]
#pragma unroll
  for (int r = 0; r < 16; ++r) red[((wk * WN + wn) * 32 + mfma_row(r, lane)) * 33 + (lane & 31)] = acc[r];
  __syncthreads();
  for (int e = threadIdx.x; e < 32 * 32 * WN; e += NTHR) {
    const int tn = e >> 10, rr = (e >> 5) & 31, cc = e & 31;
    float s = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < WK; ++w2) s += red[((w2 * WN + tn) * 32 + rr) * 33 + cc];
    red[(tn * 32 + rr) * 33 + cc] = a.rnd_bf16 ? round_bf16(s) : s;
  }
  __syncthreads();
  // final tile element (row r, column c of this work-group's 32*WN columns)
#define TT(r, c) red[(((c) >> 5) * 32 + (r)) * 33 + ((c) & 31)]
  const int n0 = blockIdx.x * WN * 32;
  if (EPI == EPI_STORE || EPI == EPI_RESID) {
    for (int e = threadIdx.x; e < 32 * 32 * WN; e += NTHR) {
      const int r = e / (32 * WN), c = e - r * (32 * WN);
      const int m = m0 + r, n = n0 + c;
      if (m < M && n < N) {
        float v = TT(r, c);
        if (a.bias) v += bf16_bits_to_float(a.bias[n]);
        if (EPI == EPI_STORE) a.y[(int64_t)m * N + n] = v;
        else a.hidden_out[(int64_t)m * N + n] += v;
      }
    }
  } else if (EPI == EPI_SWIGLU) {
    static_assert(EPI != EPI_SWIGLU || WN == 4, "SwiGLU needs [gate 64 | up 64] blocks");
    const int F = N >> 1;
    const int f0 = blockIdx.x * 64;
    for (int r = wave; r < 32; r += NW) {
      const int m = m0 + r;
      if (m >= M) continue;  // wave-uniform
      const float g = TT(r, lane), u = TT(r, 64 + lane);
      const float y = g * (1.f / (1.f + expf(-g))) * u;
      if (a.act_fmt == ACT_F16P) {
        const _Float16 h = (_Float16)y, lo = f16_lo(y, h);
        _Float16* o = (_Float16*)a.act_out + (int64_t)m * F + f16p_index(f0 + lane);
        o[0] = h;
        o[(int64_t)M * F] = lo;
        if (__ballot(f16_overflows(y)) && lane == 0) raise_range(a);
        const float s = wave_sum((float)h + (float)lo);
        if (lane == 0) a.xsum_out[(int64_t)m * (F >> 6) + (f0 >> 6)] = s;
      } else {
        ((uint16_t*)a.act_out)[(int64_t)m * F + f0 + lane] = float_to_bf16_bits(y);
      }
    }
  } else if (EPI == EPI_QKV) {
    static_assert(EPI != EPI_QKV || WN == 4, "QKV epilogue needs one 128-wide head");
    const int head = blockIdx.x;
    const int row0 = a.desc ? a.desc->row0 : 0;
    for (int r = wave; r < 32; r += NW) {
      const int m = m0 + r;
      if (m >= M) continue;  // wave-uniform
      float x0 = TT(r, lane), x1 = TT(r, lane + 64);
      if (a.bias) {
        x0 += bf16_bits_to_float(a.bias[head * 128 + lane]);
        x1 += bf16_bits_to_float(a.bias[head * 128 + 64 + lane]);
      }
      if (a.kv_bf16) qkv_head_store<__bf16>(a, head, m, row0 + m, x0, x1, lane);
      else qkv_head_store<_Float16>(a, head, m, row0 + m, x0, x1, lane);
    }
  }
#undef TT
}

#define DRT_INST(W, WN, WK, P, E) \
  template __global__ void fused_linear_kernel<W, WN, WK, P, E>(const FusedArgs);
DRT_INST(W_Q4, 4, 2, PRO_NORM, EPI_QKV)
DRT_INST(W_Q4, 1, 8, PRO_ACT, EPI_RESID)
DRT_INST(W_Q4, 4, 2, PRO_NORM, EPI_SWIGLU)
DRT_INST(W_Q4, 1, 8, PRO_ACT, EPI_STORE)
DRT_INST(W_Q4, 4, 4, PRO_ACT, EPI_RESID)
DRT_INST(W_BF16, 4, 4, PRO_NORM, EPI_QKV)
DRT_INST(W_BF16, 1, 16, PRO_ACT, EPI_RESID)
DRT_INST(W_BF16, 4, 4, PRO_NORM, EPI_SWIGLU)
DRT_INST(W_BF16, 1, 16, PRO_ACT, EPI_STORE)
DRT_INST(W_BF16, 4, 4, PRO_ACT, EPI_RESID)
#undef DRT_INST

namespace drt {

constexpr size_t FUSED_LDS = 2 * 32 * (1024 + 8) * 2 + 16 * 32 * 4 + 32 * 4 + 32 * 2 * 4;

void fused_linear(const FusedArgs& a, int kind, hipStream_t s) {
  require(a.N % 32 == 0, "fused linear needs N % 32 == 0");
  if (skinny_linear(a, kind, s)) return;
  if (kind == FL_STORE && big_linear_supported(a, kind)) {  // > 32 rows, q4
    big_linear(a, FL_STORE, 1, s);
    return;
  }
  require(a.K % (a.qw ? 64 : 16) == 0, "fused linear needs K % 64 (q4) or K % 16 (bf16)");
  static_assert(FUSED_LDS >= 16 * 32 * 33 * 4, "LDS staging must also hold the reduction");
  const bool q4 = a.qw != nullptr;
  const int m_tiles = (a.M + 31) / 32;
  const double bytes = q4 ? (double)a.N * a.K / 2 + (double)a.N * a.K / 16 + 2.0 * a.M * a.K +
                                2.0 * a.M * a.N
                          : 2.0 * a.N * a.K + 2.0 * a.M * a.K + 2.0 * a.M * a.N;
#define DRT_FL(W, WN, WK, P, E)                                                             \
  {                                                                                         \
    auto fn = fused_linear_kernel<W, WN, WK, P, E>;                                         \
    static size_t granted = 0;                                                              \
    grant_lds((const void*)fn, FUSED_LDS, granted);                                         \
    const dim3 grid((a.N / 32 + WN - 1) / WN, m_tiles);                                     \
    DRT_LAUNCH(Profiler::GEMM, bytes, fn, grid, dim3(64 * WN * WK), FUSED_LDS, s, a);       \
  }
  switch (kind) {
    // q4 kernels run 8 waves where the bf16 ones run 16: the hi and lo A
    // fragments need the registers of 512-thread work-groups
    case FL_QKV:
      require(a.N % 128 == 0, "QKV epilogue needs whole heads");
      if (q4) DRT_FL(W_Q4, 4, 2, PRO_NORM, EPI_QKV) else DRT_FL(W_BF16, 4, 4, PRO_NORM, EPI_QKV)
      break;
    case FL_RESID:
      // decode-sized tiles read A straight from global; large M shares it via LDS
      if (a.M <= 32) {
        if (q4) DRT_FL(W_Q4, 1, 8, PRO_ACT, EPI_RESID) else DRT_FL(W_BF16, 1, 16, PRO_ACT, EPI_RESID)
      } else {
        if (q4) DRT_FL(W_Q4, 4, 4, PRO_ACT, EPI_RESID) else DRT_FL(W_BF16, 4, 4, PRO_ACT, EPI_RESID)
      }
      break;
    case FL_SWIGLU:
      require(a.N % 128 == 0, "SwiGLU epilogue needs 64-column gate/up blocks");
      if (q4) DRT_FL(W_Q4, 4, 2, PRO_NORM, EPI_SWIGLU) else DRT_FL(W_BF16, 4, 4, PRO_NORM, EPI_SWIGLU)
      break;
    case FL_STORE:
      if (q4) DRT_FL(W_Q4, 1, 8, PRO_ACT, EPI_STORE) else DRT_FL(W_BF16, 1, 16, PRO_ACT, EPI_STORE)
      break;
    default:
      fail(INVALID_ARGUMENT, "unknown fused linear kind");
  }
#undef DRT_FL
  DRT_HIP(hipGetLastError());
}

}  // namespace drt
