// Split-K linears for decode-sized activations (M <= 32 rows per row tile, up to
// sk_row_tiles tiles) and q4 or bf16 weights (WK). With bf16 weights the
// activation is ACT_BF16 (one plane), each 64-k unit is four bf16 MFMAs, and the
// summed tile is rounded to bf16 before the epilogue, as the reference's bf16
// matmul output is (backends/mlx_ops.py:122-125) and as fused_linear_kernel does.
//
// A decode step's linears read only 1-4 MB of weights; what bounds them is how
// much each CU must pull (about 64 GB/s per CU) and how many dependent memory
// round trips a work-group makes. So these kernels spread every linear over
// 128-448 work-groups of 4 waves, each reading a K slice of its columns' weights
// and only that slice of the activation, with every load issued up front. The
// K slices of one output block meet in a global workspace: each work-group
// writes its partial tile, bumps the block's arrival counter, and the last to
// arrive adds the partials in slice order (deterministic) and runs the
// epilogue. Nothing waits on another work-group, so no launch order is assumed.
// A forward of more than 32 rows runs its 32-row tiles as the grid's y
// dimension: each tile's work-groups repeat the weight slices (the second read
// mostly from L2) and keep partials, counters and row statistics of their own.
//
// The exchange stays inside one XCD's L2: work-group i runs on XCD i % n_xcc
// (the dispatcher's round-robin), so the grid is laid out to give every slice
// of block b the XCD b % n_xcc. Plain stores, the L2 atomic and plain loads are
// then coherent with each other, with no device-wide fence (an L2 writeback and
// invalidate per work-group costs tens of microseconds). Each work-group checks
// the XCD it runs on and raises `placement_err` if the layout assumption fails,
// which the host turns into an error. The runtime probes the placement once at
// creation; where it does not hold, the kernels run `fenced`: each slice's
// stores are released at device scope before a device-scope arrival atomic,
// and the last work-group acquires before reading the slices.
//
//   skinny_wide_kernel  : 128 columns (4 n-tiles, one per wave), RMSNorm
//                         prologue (row statistics from the producer's
//                         per-32-column partial sums of squares), epilogue on a
//                         whole head (q/k norm, RoPE, Q out, K/V into the cache)
//                         or a [gate 64 | up 64] block (SwiGLU -> down activation).
//   skinny_narrow_kernel: 32 columns, 4 waves split the slice, the activation
//                         (ACT_F16P) read straight from global; epilogue
//                         hidden += tile (+ the new rows' partial sums of
//                         squares for the next RMSNorm) or y = tile (+ bias).
// Reference math: backends/mlx_ops.py:21-35 (rms_norm), :97-130 (q4 linear),
// :133-154 (rope, swiglu); backends/mlx_forward.py:1164-1361 (layer).
#include "fused.h"
#include "gemm_core.h"
#include "launch.h"
#include "linear_dev.h"

#include <cstdlib>
#include <vector>

namespace {

constexpr int SK_RED = 4 * 32 * 33;  // floats of the [4][32][33] reduction tile
constexpr int SK_KS_MAX = 8;         // K slices per output tile (host-enforced)
constexpr int SK_SS_PER_THREAD = 14; // K / 32 <= 8 * 14 = 112 partial sums (d <= 3584)

// LDS of the wide kernel: xs [2][32][64U + 8] halves (hi, lo), xss [U][32],
// rinv [32], red [4][32][33], flag (16 B), then the V tile half [4096] halves.
#define SK_WIDE_V_OFF(U) (((2 * 32 * ((U) * 64 + 8) * 2 + (U) * 32 * 4 + 32 * 4 + SK_RED * 4 + 16) + 15) / 16 * 16)
#define SK_WIDE_LDS(U) (SK_WIDE_V_OFF(U) + 4096 * 2)
// LDS of the narrow kernel: red [4][32][33] floats, flag (16 B), then the A
// staging of the four waves, [4][2 planes][UW][32][144 B]
#define SK_NARROW_STG (SK_RED * 4 + 16)
#define SK_NARROW_LDS(UW) (SK_NARROW_STG + 4 * 2 * (UW) * 32 * 144)

// Kernel arguments the first loads need are fetched in one batch at kernel
// start: one empty asm that takes them all in scalar registers keeps the
// compiler from fetching some only after a wait or behind a branch (a dependent
// round trip each). Pointers pass through the global address space (a generic
// pointer out of the asm would make every access through it a flat access,
// which also counts on lgkmcnt).
#define SK_GLOBAL(T) __attribute__((address_space(1))) T

// Block and K slice of this work-group: with x = i % n_xcc and j = i / n_xcc,
// block x + n_xcc * (j / KS) and slice j % KS, so a block's slices share an XCD.
// Returns false for the padding work-groups past the last block; those get
// block 0 and must leave before their first store. (They run on past their
// loads: an early return would let the compiler sink the loads, and the kernel
// argument fetches they need, behind the branch - one more round trip for
// every work-group.) n_xcc and perr are the pinned a.n_xcc, a.placement_err.
DRT_DEV bool sk_place(int n_xcc, int fenced, int* perr, int n_blocks, int KS, int& blk,
                      int& ks) {
  const int i = blockIdx.x, x = i % n_xcc, j = i / n_xcc;
  blk = x + n_xcc * (j / KS);
  ks = j - (j / KS) * KS;
  if (n_xcc > 1 && !fenced && threadIdx.x == 0 && perr) {
    const int xcc = (int)(__builtin_amdgcn_s_getreg((31 << 11) | 20) & 0xf);  // HW_REG_XCC_ID
    if (xcc != x) __hip_atomic_fetch_or(perr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  const bool live = blk < n_blocks;
  blk = live ? blk : 0;
  return live;
}

// Called after this work-group stored its partial: returns true in the last
// work-group of the block to arrive (which then adds the partials up), false
// elsewhere. The stores complete (in this XCD's L2) before the barrier, and the
// counter is bumped by an L2 atomic after it. Fenced (placement not assumed):
// the stores are released at device scope and the arrival is a device-scope
// acquire-release, so the last work-group sees every slice wherever it ran.
DRT_DEV bool last_to_arrive(int* counter, int arrivals, int* flag, int fenced) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    if (fenced)
      *flag = __hip_atomic_fetch_add(counter, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) ==
              arrivals - 1;
    else
      *flag = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_WORKGROUP) == arrivals - 1;
  }
  __syncthreads();
  return *flag != 0;
}

// The arrival counter back to zero for the next launch (fenced: at device scope,
// where the next launch's arrivals count).
DRT_DEV void reset_counter(int* counter, int fenced) {
  if (fenced) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *counter = 0;
}

// XCD of every work-group of a 1-D launch (the placement probe).
__global__ void xcc_probe_kernel(int* __restrict__ xcc) {
  if (threadIdx.x == 0)
    xcc[blockIdx.x] = (int)(__builtin_amdgcn_s_getreg((31 << 11) | 20) & 0xf);  // HW_REG_XCC_ID
}

// The last work-group's sum of the KS <= KSC partial tiles of a wide block into
// the [4][32][33] LDS tile: 1024 16-byte chunks, 4 per thread; every slice's
// chunks are loaded before any is added (then added in slice order). Slices
// past KS reload the last one and are added times 0: a load under a branch makes
// the compiler wait for it, and for everything issued before it, inside the
// branch.
template <int KSC>
DRT_DEV void sk_wide_sum_slices(const float* pbase, int KS, float* red, bool rnd) {
  f32x4 pv[KSC][4];
#pragma unroll
  for (int k2 = 0; k2 < KSC; ++k2)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      pv[k2][i] = *(const f32x4*)(pbase + (size_t)min(k2, KS - 1) * 4096 + 4 * (threadIdx.x + 256 * i));
  __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the first wait
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k2 = 0; k2 < KSC; ++k2) sum += pv[k2][i] * (k2 < KS ? 1.f : 0.f);
    const int q = threadIdx.x + 256 * i, tn = q >> 8, c4 = q & 255;
    const int ln = c4 & 63, col = ln & 31, r0 = 8 * (c4 >> 6) + 4 * (ln >> 5);
#pragma unroll
    for (int e = 0; e < 4; ++e) red[(tn * 32 + r0 + e) * 33 + col] = rnd ? round_bf16(sum[e]) : sum[e];
  }
}

}  // namespace

// Everything the first loads need is in the leading scalar arguments, which
// arrive in scalar registers at wave start (kernel-argument preloading, 16
// dwords): the sizes packed as dims0 = N | K << 16 and dims1 = M | KS << 8 |
// n_xcc << 16 | fenced << 24. The rest of the arguments (`a`) are fetched
// while the first loads are in flight.
DRT_DEV void sk_dims(uint32_t dims0, uint32_t dims1, int& M, int& N, int& K, int& KS, int& n_xcc,
                     int& fenced) {
  N = (int)(dims0 & 0xffffu);
  K = (int)(dims0 >> 16);
  M = (int)(dims1 & 0xffu);
  KS = (int)((dims1 >> 8) & 0xffu);
  n_xcc = (int)((dims1 >> 16) & 0xffu);
  fenced = (int)(dims1 >> 24);
}

// PRE: the input is pre-scaled ACT_F16P planes (see FusedArgs::pre_out):
// `hidden` points at the planes, `norm_w` at their per-32-column sums and sc_in
// at their scale c per row; they are staged as they are and the output rows are
// multiplied by rinv / c.
template <int WK, int EPI, int U, bool PRE>
__global__ __launch_bounds__(256) void skinny_wide_kernel(
    const uint32_t* __restrict__ qw, const uint32_t* __restrict__ sbp,
    const float* __restrict__ hidden, const uint16_t* __restrict__ norm_w,
    const float* __restrict__ ss_arg, const float* __restrict__ sc_in, int* perr,
    uint32_t dims0, uint32_t dims1, const FusedArgs a) {
  constexpr bool BF = WK == W_BF16;
  static_assert(!PRE || !BF, "pre-scaled planes feed the q4 kernels only");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int M, N, K, KS, n_xcc, fenced;
  sk_dims(dims0, dims1, M, N, K, KS, n_xcc, fenced);
  // 32-row tile of this work-group: rows m0 .. m0 + M - 1 of the forward
  const int mt = blockIdx.y, m0 = 32 * mt, M_all = M;
  M = min(32, M_all - m0);
  const uint16_t* pl_hi = (const uint16_t*)hidden + (int64_t)m0 * K;  // PRE
  const float* pl_xs = (const float*)norm_w + (int64_t)mt * K;        // PRE
  hidden += (int64_t)m0 * K;
  const float* ss_in = ss_arg + (int64_t)mt * K;
  float* part = a.part + (size_t)mt * a.part_floats;
  int* counters = a.counters + (size_t)mt * a.n_counters;
  const int G = K >> 6;
  int grp, ks;
  const bool live = sk_place(n_xcc, fenced, perr, N / 128, KS, grp, ks);
  const int nt = grp * 4 + wave;
  const int u0 = ks * U, kc0 = u0 * 64;
  // absolute position of row 0 (the q|k|v epilogue's rotary tables), read at
  // the start: the tables' loads after the MFMAs depend on it
  const int row0 = EPI == EPI_QKV && a.desc ? a.desc->row0 : 0;
  constexpr int KCN = U * 64;
  constexpr int ROW_H = KCN + 8;  // 16-bit elements per LDS row (+16 B pad)
  extern __shared__ __align__(16) char smem[];
  uint16_t* xs = (uint16_t*)smem;                       // [32][ROW_H] ACT_F16P hi
  uint16_t* xsl = xs + 32 * ROW_H;                      // [32][ROW_H] ACT_F16P lo
  float* xss = (float*)(smem + 2 * 32 * ROW_H * 2);     // [U][32] group sums
  float* rinv = xss + U * 32;                           // [32] (PRE: rinv / c)
  float* red = rinv + 32;                               // [4][32][33]
  int* flag = (int*)(red + SK_RED);
  uint16_t* vbuf = (uint16_t*)(smem + SK_WIDE_V_OFF(U));  // [4096] V tile half (QKV)

  // Loads in the order their data is needed: vector memory loads retire in
  // issue order, so data from L2 issued behind the weights (from HBM) would
  // wait for them. 1. row statistics: thread (group g = tid / 32, row r = tid %
  // 32) loads the producer's partial sums of squares g, g + 8, ... at once.
  // Every load of steps 1-3 is unconditional (rows past M read row M - 1 and are
  // zeroed by their norm factor, partial sums past the last are clamped and
  // masked after the wait): a load under a branch makes the compiler wait for it
  // inside the branch, i.e. for every load issued before it.
  const int np = K >> 5;  // <= 8 * SK_SS_PER_THREAD
  float sv[SK_SS_PER_THREAD];
#pragma unroll
  for (int e = 0; e < SK_SS_PER_THREAD; ++e)
    sv[e] = ss_in[min((int)(threadIdx.x >> 5) + 8 * e, np - 1) * 32 + (threadIdx.x & 31)];
  // PRE: the planes' scale of this thread's row
  const float c_in = PRE ? sc_in[m0 + min((int)(threadIdx.x & 31), M - 1)] : 1.f;
  // 2. the hidden slice (8-wide items: U per thread) and the matching norm weights;
  // PRE: the planes' slice (hi, lo) and the sums of the slice's 32-column halves
  f32x4 hv[U][2];
  u32x4 nw[U];
  float xp[2];
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const int it = threadIdx.x + 256 * j;
    const int r = it / (8 * U), c8 = it - r * (8 * U);
    const int k = kc0 + c8 * 8;
    if (PRE) {
      const uint16_t* src = pl_hi + (int64_t)min(r, M - 1) * K + k;
      hv[j][0] = __builtin_bit_cast(f32x4, *(const u32x4*)src);
      hv[j][1] = __builtin_bit_cast(f32x4, *(const u32x4*)(src + (int64_t)M_all * K));
    } else {
      const f32x4* src = (const f32x4*)(hidden + (int64_t)min(r, M - 1) * K + k);
      hv[j][0] = src[0];
      hv[j][1] = src[1];
      nw[j] = *(const u32x4*)(norm_w + k);
    }
  }
  if (PRE) {  // thread (unit u = tid / 32 clamped, row tid % 32)
    const int u = min((int)(threadIdx.x >> 5), U - 1), r = min((int)(threadIdx.x & 31), M - 1);
    const float* src = pl_xs + ((kc0 >> 5) + 2 * u) * 32 + r;
    xp[0] = src[0];
    xp[1] = src[32];
  }
  __builtin_amdgcn_sched_barrier(0);
  // 3. this wave's weights for the U units (bf16: the unit's four 16-k MFMA
  // fragments), in flight while the row statistics and the norm are computed
  u32x4 wq[U][BF ? 4 : 1];
  uint32_t wsb[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (BF) {
#pragma unroll
      for (int t = 0; t < (BF ? 4 : 1); ++t)
        wq[u][t] = __builtin_nontemporal_load(
            (const u32x4*)bf16_tile_frag((const uint16_t*)qw, nt, K >> 4, 4 * (u0 + u) + t, lane));
      wsb[u] = 0u;
    } else {
      wq[u][0] = __builtin_nontemporal_load(q4_tile_words(qw, nt, G, u0 + u, lane));
      wsb[u] = q4_tile_sb(sbp, nt, G, u0 + u, lane);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  {  // the 8 group sums of each row, added in order
    const int g8 = threadIdx.x >> 5;
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < SK_SS_PER_THREAD; ++e)  // a product, not a select, so that
      q += sv[e] * (g8 + 8 * e < np ? 1.f : 0.f);  // the load is not sunk into a branch
    red[g8 * 32 + (threadIdx.x & 31)] = q;
    // PRE: c of the row through LDS (the V tile's space, used only by the
    // epilogue), written by every thread of the row: a use in a branch would
    // let the compiler sink the load behind the weights
    if (PRE) ((float*)vbuf)[threadIdx.x & 31] = c_in;
  }
  __syncthreads();
  if (PRE) {
    if (threadIdx.x < 32) {
      float ssum = 0.f;
#pragma unroll
      for (int g8 = 0; g8 < 8; ++g8) ssum += red[g8 * 32 + threadIdx.x];
      const float ri = 1.f / sqrtf(ssum / (float)K + a.eps);
      rinv[threadIdx.x] = (int)threadIdx.x < M ? ri / ((float*)vbuf)[threadIdx.x] : 0.f;
      if (a.pre_sc_out && grp == 0 && ks == 0 && live && (int)threadIdx.x < M)
        a.pre_sc_out[m0 + threadIdx.x] = pre_scale_of(ri);
    }
    // 4. the planes into LDS as they are, and the 64-k group sums
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int it = threadIdx.x + 256 * j;
      const int r = it / (8 * U), c8 = it - r * (8 * U);
      *(u32x4*)(xs + r * ROW_H + c8 * 8) = __builtin_bit_cast(u32x4, hv[j][0]);
      *(u32x4*)(xsl + r * ROW_H + c8 * 8) = __builtin_bit_cast(u32x4, hv[j][1]);
    }
    if ((int)threadIdx.x < 32 * U) xss[threadIdx.x] = xp[0] + xp[1];
  } else {
    if (threadIdx.x < 32) {
      float ssum = 0.f;
#pragma unroll
      for (int g8 = 0; g8 < 8; ++g8) ssum += red[g8 * 32 + threadIdx.x];
      rinv[threadIdx.x] = 1.f / sqrtf(ssum / (float)K + a.eps);
    }
    __syncthreads();
  }
  // 4. RMSNorm(h) * w -> ACT_F16P hi / lo (chunk order 0,4,1,5,2,6,3,7) + group sums
  bool over = false;
#pragma unroll
  for (int j = 0; j < (PRE ? 0 : U); ++j) {
    const int it = threadIdx.x + 256 * j;
    const int r = it / (8 * U), c8 = it - r * (8 * U);
    const float inv = r < M ? rinv[r] : 0.f;
    float x[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = (hv[j][e >> 1][(2 * e) & 3] * inv) * bf16_bits_to_float(nw[j][e] & 0xffffu);
      x[2 * e + 1] = (hv[j][e >> 1][(2 * e + 1) & 3] * inv) * bf16_bits_to_float(nw[j][e] >> 16);
    }
    if (BF) {  // ACT_BF16 in natural order, no group sums
      u32x4 pk;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        pk[e] = (uint32_t)float_to_bf16_bits(x[2 * e]) |
                ((uint32_t)float_to_bf16_bits(x[2 * e + 1]) << 16);
      *(u32x4*)(xs + r * ROW_H + c8 * 8) = pk;
      continue;
    }
    _Float16 h[8], lo[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      h[e] = (_Float16)x[e];
      lo[e] = f16_lo(x[e], h[e]);
      over = over || f16_overflows(x[e]);
    }
    u32x4 pk, pl;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      pk[e] = (uint32_t)half_bits(h[e]) | ((uint32_t)half_bits(h[e + 4]) << 16);
      pl[e] = (uint32_t)half_bits(lo[e]) | ((uint32_t)half_bits(lo[e + 4]) << 16);
    }
    *(u32x4*)(xs + r * ROW_H + c8 * 8) = pk;
    *(u32x4*)(xsl + r * ROW_H + c8 * 8) = pl;
    float gs = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) gs += (float)h[e] + (float)lo[e];
    gs = sum8_dpp(gs);  // a 64-k group is 8 consecutive items of one row = 8 lanes
    if ((c8 & 7) == 0) xss[(c8 >> 3) * 32 + r] = gs;
  }
  if (over && live) raise_range(a);
  __syncthreads();
  // 5. this wave's n-tile over the U units
  f32x16 acc = f32x16{};
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (BF) {  // k = 16 t + 8 (lane >> 5) + e of the unit, natural order
      const uint16_t* brow = xs + (lane & 31) * ROW_H + u * 64 + 8 * (lane >> 5);
#pragma unroll
      for (int t = 0; t < (BF ? 4 : 1); ++t)
        acc = mfma_bf16(*(const bf16x8*)(brow + 16 * t), __builtin_bit_cast(bf16x8, wq[u][t]), acc);
      continue;
    }
    const _Float16* arow = (const _Float16*)xs + (lane & 31) * ROW_H + u * 64 + 32 * (lane >> 5);
    f16x8 af[4], afl[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      af[t] = *(const f16x8*)(arow + 8 * t);
      afl[t] = *(const f16x8*)(arow + 32 * ROW_H + 8 * t);
    }
    float xsr[16];
    load_row_sums(xss + u * 32, lane, xsr);
    q4_group_mma1(acc, af, afl, xsr, wq[u][0], wsb[u]);
  }
  if (PRE) {  // the rows' factors rinv / c (0 past M)
    float fr[16];
    load_row_sums(rinv, lane, fr);
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] *= fr[i];
  }
  // the q|k|v epilogue's tables (rotary angles, q/k norm weights, bias), issued
  // before the exchange so that their latency passes during it
  QkvTables qt;
  if (EPI == EPI_QKV) qt = qkv_tables(a, grp, row0 + m0, M);
  if (!live) return;  // work-group-uniform, before any global store
  // 6. K slices meet: the last work-group of the column block adds the partials
  if (KS > 1) {
    // partial tile of this wave in accumulator order: chunk jj*64 + lane holds
    // rows 8jj + 4(lane >> 5) .. +3 of column lane & 31, so each store
    // instruction writes 1 KiB of whole cache lines
    float* pw = part + ((size_t)(grp * KS + ks) * 4 + wave) * 1024 + 4 * lane;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
      *(f32x4*)(pw + 256 * jj) = f32x4{acc[4 * jj], acc[4 * jj + 1], acc[4 * jj + 2], acc[4 * jj + 3]};
    if (!last_to_arrive(&counters[grp], KS, flag, a.fenced)) return;
    const float* pbase = part + (size_t)grp * KS * 4096;
    const bool rnd = BF && a.rnd_bf16;
    if (KS <= 2) sk_wide_sum_slices<2>(pbase, KS, red, rnd);
    else if (KS <= 4) sk_wide_sum_slices<4>(pbase, KS, red, rnd);
    else sk_wide_sum_slices<SK_KS_MAX>(pbase, KS, red, rnd);
  } else {
#pragma unroll
    for (int r = 0; r < 16; ++r)
      red[(wave * 32 + mfma_row(r, lane)) * 33 + (lane & 31)] =
          BF && a.rnd_bf16 ? round_bf16(acc[r]) : acc[r];
  }
  __syncthreads();
#define TT(r, c) red[(((c) >> 5) * 32 + (r)) * 33 + ((c) & 31)]
  if (EPI == EPI_SWIGLU) {
    // thread t: row t >> 3, outputs f0 + 8c .. +7 (c = t & 7) from gate columns
    // 8c.. and up columns 64 + 8c.. of the [gate 64 | up 64] block; one 16-byte
    // store per thread (ACT_F16P chunk order 0,4,1,5,2,6,3,7; hi and lo planes).
    // No group sums: the down projection computes them from the values it reads.
    const int F = N >> 1;
    const int f0 = grp * 64;
    const int m = threadIdx.x >> 3, c = threadIdx.x & 7;
    if (m < M) {
      float y[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float g = TT(m, 8 * c + e), u = TT(m, 64 + 8 * c + e);
        y[e] = g * (1.f / (1.f + expf(-g))) * u;
      }
      uint16_t* dst = (uint16_t*)a.act_out + (int64_t)(m0 + m) * F + f0 + 8 * c;
      u32x4 pk;
      if (a.act_fmt == ACT_F16P) {
        u32x4 pl;
        bool over = false;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const _Float16 h0 = (_Float16)y[e], h1 = (_Float16)y[e + 4];
          pk[e] = (uint32_t)half_bits(h0) | ((uint32_t)half_bits(h1) << 16);
          pl[e] = (uint32_t)half_bits(f16_lo(y[e], h0)) |
                  ((uint32_t)half_bits(f16_lo(y[e + 4], h1)) << 16);
          over = over || f16_overflows(y[e]) || f16_overflows(y[e + 4]);
        }
        *(u32x4*)(dst + (int64_t)M_all * F) = pl;
        if (over) raise_range(a);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          pk[e] = (uint32_t)float_to_bf16_bits(y[2 * e]) |
                  ((uint32_t)float_to_bf16_bits(y[2 * e + 1]) << 16);
      }
      *(u32x4*)dst = pk;
    }
  } else if (EPI == EPI_QKV) {
    auto get = [&](int m, int d) { return red[((d >> 5) * 32 + m) * 33 + (d & 31)]; };
    if (a.kv_bf16) qkv_epilogue<__bf16>(a, qt, grp, m0, row0 + m0, M, get, vbuf);
    else qkv_epilogue<_Float16>(a, qt, grp, m0, row0 + m0, M, get, vbuf);
  }
#undef TT
  // the arrival counter back to zero, after the epilogue: on this target a wait
  // for a load also waits for every store issued before it
  if (KS > 1 && threadIdx.x == 0) reset_counter(&counters[grp], a.fenced);
}

// UW: units per wave held in registers at once (the wave's units are processed
// in chunks of UW, each chunk's loads issued together).
// XIN: the activation's format. 0: ACT_F16P (hi plane, lo plane at + M * K);
// 1: fp32 rows [M][K] and 2: bf16 rows (a per-op call's input), split into the
// hi and lo planes in registers on the way to LDS (no preparation pass).
template <int WK, int EPI, int UW, int XIN>
__global__ __launch_bounds__(256) void skinny_narrow_kernel(
    const uint32_t* __restrict__ qw, const uint32_t* __restrict__ sbp,
    const uint16_t* __restrict__ act, int* perr, uint32_t dims0, uint32_t dims1,
    const FusedArgs a) {
  static_assert(XIN == 0 || WK == W_Q4, "fp32 / bf16 rows feed the q4 kernels only");
  constexpr bool BF = WK == W_BF16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int M, N, K, KS, n_xcc, fenced;
  sk_dims(dims0, dims1, M, N, K, KS, n_xcc, fenced);
  // 32-row tile of this work-group: rows m0 .. m0 + M - 1 of the forward
  const int mt = blockIdx.y, m0 = 32 * mt, M_all = M;
  M = min(32, M_all - m0);
  float* part = a.part + (size_t)mt * a.part_floats;
  int* counters = a.counters + (size_t)mt * a.n_counters;
  const int G = K >> 6;
  const int U = G / KS;
  int nt, ks;
  const bool live = sk_place(n_xcc, fenced, perr, N / 32, KS, nt, ks);
  const int u_lo = ks * U + (U * wave) / 4, u_hi = ks * U + (U * (wave + 1)) / 4;
  extern __shared__ __align__(16) char smem[];
  float* red = (float*)smem;  // [4][32][33]
  int* flag = (int*)(red + SK_RED);

  f32x16 acc = f32x16{};
  // epilogue: thread t owns row t >> 3, columns 4*(t & 7) .. +3 of the tile
  const int m = threadIdx.x >> 3, c0 = 4 * (threadIdx.x & 7);
  const int n = nt * 32 + c0;
  f32x4 h_old = f32x4{0.f, 0.f, 0.f, 0.f};
  uint2 pw = uint2{0u, 0u};
  float pc = 0.f;
  // this wave's A staging: [2 planes][UW][32 rows][144 B] (128 B of a unit's row + pad)
  char* stg = smem + SK_NARROW_STG + wave * (2 * UW * 32 * 144);
  const uint16_t* act_lo = act + (int64_t)M_all * K + (int64_t)m0 * K;  // ACT_F16P lo plane
  const float* x32 = (const float*)act + (int64_t)m0 * K;                // XIN == 1
  act += (int64_t)m0 * K;
  for (int ub = u_lo; ub < u_hi || ub == u_lo; ub += UW) {
    u32x4 wq[UW][BF ? 4 : 1], craw[UW][4], crawl[UW][4], af[UW][4], afl[UW][4];
    f32x4 xr[XIN == 1 ? UW : 1][4][2];  // XIN == 1: the lane's 8 fp32 values
    uint32_t wsb[UW];
    // the activation (from L2) is issued before the weights (from HBM): loads
    // retire in issue order, so the LDS transpose below would otherwise wait
    // for the weights too. Units are clamped to a valid one; a unit beyond the
    // wave's range gets scale and bias 0 (bf16: it is not multiplied), an exact
    // no-op, so every load is used unconditionally.
#pragma unroll
    for (int i = 0; i < UW; ++i) {
      const int u = min(ub + i, max(u_hi, u_lo + 1) - 1);
      // the unit's 32 x 64 activation block as four coalesced loads of 8 rows x
      // 128 B (rows past M read row M - 1: their outputs are never stored)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t off = (int64_t)min(8 * j + (lane >> 3), M - 1) * K + u * 64 + (lane & 7) * 8;
        if (XIN == 1) {
          xr[XIN == 1 ? i : 0][j][0] = *(const f32x4*)(x32 + off);
          xr[XIN == 1 ? i : 0][j][1] = *(const f32x4*)(x32 + off + 4);
        } else {
          craw[i][j] = *(const u32x4*)(act + off);  // XIN == 2: 8 bf16 values
          if (!BF && XIN == 0) crawl[i][j] = *(const u32x4*)(act_lo + off);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < UW; ++i) {
      const int u = min(ub + i, max(u_hi, u_lo + 1) - 1);
      if (BF) {
#pragma unroll
        for (int t = 0; t < (BF ? 4 : 1); ++t)
          wq[i][t] = __builtin_nontemporal_load(
              (const u32x4*)bf16_tile_frag((const uint16_t*)qw, nt, K >> 4, 4 * u + t, lane));
        wsb[i] = 0u;
      } else {
        wq[i][0] = __builtin_nontemporal_load(q4_tile_words(qw, nt, G, u, lane));
        wsb[i] = ub + i < u_hi ? q4_tile_sb(sbp, nt, G, u, lane) : 0u;
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // the epilogue's inputs, issued behind the weights so that their latency
    // (they may come from another XCD's writes or from HBM) passes during the
    // MFMAs and the exchange, and no wait before those is held up by them (with
    // pre-scaled planes out: the next norm's weights and the row's scale;
    // without, the two pre loads read the hidden rows). Unconditional: a load
    // under a branch must be waited for again after it, and on this target a wait
    // also waits for the stores issued before it. (Several unit batches: reloaded
    // each time, from L2.)
    if (EPI == EPI_RESID) {
      const int64_t row = m0 + min(m, M - 1);
      h_old = *(const f32x4*)(a.hidden_out + row * N + n);
      const bool pre = a.pre_out != nullptr;
      pw = *(const uint2*)(pre ? (const void*)(a.pre_norm + n) : (const void*)(a.hidden_out + n));
      pc = *(pre ? a.pre_sc + row : (const float*)a.hidden_out);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (XIN != 0) {
      // fp32 / bf16 rows: the 8 values of each piece as fp16 hi and lo, each
      // 32-bit word holding elements (w, w + 4) (the ACT_F16P chunk order)
#pragma unroll
      for (int i = 0; i < UW; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float v[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            if (XIN == 1) v[e] = xr[XIN == 1 ? i : 0][j][e >> 2][e & 3];
            else v[e] = bf16_bits_to_float(e & 1 ? craw[i][j][e >> 1] >> 16
                                                  : craw[i][j][e >> 1] & 0xffffu);
          }
          u32x4 hp, lp;
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const _Float16 h0 = (_Float16)v[w], h1 = (_Float16)v[w + 4];
            hp[w] = (uint32_t)half_bits(h0) | ((uint32_t)half_bits(h1) << 16);
            lp[w] = (uint32_t)half_bits(f16_lo(v[w], h0)) |
                    ((uint32_t)half_bits(f16_lo(v[w + 4], h1)) << 16);
          }
          craw[i][j] = hp;
          crawl[i][j] = lp;
        }
    }
    // through LDS into the q4 fragment order: lane l takes row l & 31, 16-byte
    // chunks 4(l >> 5) + t, i.e. k = 32(l >> 5) + 8t .. +8 (one wave's LDS
    // operations run in order: no barrier)
    constexpr int PLANE = UW * 32 * 144;
#pragma unroll
    for (int i = 0; i < UW; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        char* d = stg + (i * 32 + 8 * j + (lane >> 3)) * 144 + (lane & 7) * 16;
        *(u32x4*)d = craw[i][j];
        if (!BF) *(u32x4*)(d + PLANE) = crawl[i][j];
      }
    if (BF) {  // bf16: 16-k MFMA chunk t of the unit is 16-byte chunk 2 t + (lane >> 5)
#pragma unroll
      for (int i = 0; i < UW; ++i) {
        if (ub + i >= u_hi) break;  // a clamped repeat of the last unit (wave-uniform)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const bf16x8 ab = *(const bf16x8*)(stg + (i * 32 + (lane & 31)) * 144 +
                                             (2 * t + (lane >> 5)) * 16);
          acc = mfma_bf16(ab, __builtin_bit_cast(bf16x8, wq[i][BF ? t : 0]), acc);
        }
      }
      if (ub + UW >= u_hi) break;
      continue;
    }
#pragma unroll
    for (int i = 0; i < UW; ++i)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const char* sp = stg + (i * 32 + (lane & 31)) * 144 + (4 * (lane >> 5) + t) * 16;
        af[i][t] = *(const u32x4*)sp;
        afl[i][t] = *(const u32x4*)(sp + PLANE);
      }
    float xsr[UW][16];
    row_sums_lane<UW>(af, afl, red + wave * 32 * 33, lane, xsr);
#pragma unroll
    for (int i = 0; i < UW; ++i) {
      f16x8 ah[4], alh[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        ah[t] = __builtin_bit_cast(f16x8, af[i][t]);
        alh[t] = __builtin_bit_cast(f16x8, afl[i][t]);
      }
      q4_group_mma1(acc, ah, alh, xsr[i], wq[i][0], wsb[i]);
    }
    if (ub + UW >= u_hi) break;
  }
  if (!live) return;  // work-group-uniform, before any barrier or store
  // the four waves' K ranges, in order; thread t owns row t >> 3, columns
  // 4*(t & 7) .. +3 of the tile (one 16-byte chunk everywhere below)
#pragma unroll
  for (int r = 0; r < 16; ++r) red[(wave * 32 + mfma_row(r, lane)) * 33 + (lane & 31)] = acc[r];
  __syncthreads();
  // every store of the epilogue comes after its last load (see above)
  f32x4 v;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    v[e] = red[m * 33 + c0 + e] + red[(32 + m) * 33 + c0 + e] + red[(64 + m) * 33 + c0 + e] +
           red[(96 + m) * 33 + c0 + e];
  if (KS > 1) {
    *(f32x4*)(part + (size_t)(nt * KS + ks) * 1024 + m * 32 + c0) = v;
    if (!last_to_arrive(&counters[nt], KS, flag, a.fenced)) return;
    const float* pp = part + (size_t)nt * KS * 1024 + m * 32 + c0;
    f32x4 pv[SK_KS_MAX];
#pragma unroll
    for (int k2 = 0; k2 < SK_KS_MAX; ++k2) pv[k2] = *(const f32x4*)(pp + (size_t)min(k2, KS - 1) * 1024);
    v = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k2 = 0; k2 < SK_KS_MAX; ++k2) v += pv[k2] * (k2 < KS ? 1.f : 0.f);  // unconditional loads
  }
  if (BF && a.rnd_bf16) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = round_bf16(v[e]);
  }
  if (a.bias) {
    const uint2 bb = *(const uint2*)(a.bias + n);
    v[0] += bf16_bits_to_float(bb.x & 0xffffu);
    v[1] += bf16_bits_to_float(bb.x >> 16);
    v[2] += bf16_bits_to_float(bb.y & 0xffffu);
    v[3] += bf16_bits_to_float(bb.y >> 16);
  }
  if (EPI == EPI_RESID) {
    const f32x4 h = m < M ? h_old + v : f32x4{0.f, 0.f, 0.f, 0.f};
    const float q = sum8_dpp(h[0] * h[0] + h[1] * h[1] + h[2] * h[2] + h[3] * h[3]);
    // pre-scaled planes: the next norm's input w * h * c as hi / lo fp16 (rows
    // past M: zeros, not stored), and the sum of the 32 columns' hi + lo per row.
    // Computed whether or not they are stored, so that every load is used (and
    // waited for) before the first store.
    uint2 wh, wl;
    float xsum = 0.f;
    bool over = false;
    {
      const float wv[4] = {bf16_bits_to_float(pw.x & 0xffffu), bf16_bits_to_float(pw.x >> 16),
                           bf16_bits_to_float(pw.y & 0xffffu), bf16_bits_to_float(pw.y >> 16)};
      _Float16 hh[4], ll[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = (h[e] * pc) * wv[e];
        hh[e] = (_Float16)x;
        ll[e] = f16_lo(x, hh[e]);
        over = over || f16_overflows(x);
        xsum += (float)hh[e] + (float)ll[e];
      }
      xsum = sum8_dpp(xsum);
      // ACT_F16P chunk order: word w of an 8-column chunk holds columns (w, w + 4);
      // the chunk's columns 0-3 are this (even) thread's, 4-7 its odd neighbour's.
      // The even thread stores words 0-1, the odd one words 2-3.
      const bool odd = threadIdx.x & 1;
      const uint32_t sh = odd ? pack_half2(hh[0], hh[1]) : pack_half2(hh[2], hh[3]);
      const uint32_t sl = odd ? pack_half2(ll[0], ll[1]) : pack_half2(ll[2], ll[3]);
      const uint32_t rh = (uint32_t)__shfl_xor((int)sh, 1), rl = (uint32_t)__shfl_xor((int)sl, 1);
      if (odd) {
        wh = uint2{(rh & 0xffffu) | ((uint32_t)half_bits(hh[2]) << 16),
                   (rh >> 16) | ((uint32_t)half_bits(hh[3]) << 16)};
        wl = uint2{(rl & 0xffffu) | ((uint32_t)half_bits(ll[2]) << 16),
                   (rl >> 16) | ((uint32_t)half_bits(ll[3]) << 16)};
      } else {
        wh = uint2{(uint32_t)half_bits(hh[0]) | (rh << 16),
                   (uint32_t)half_bits(hh[1]) | (rh & 0xffff0000u)};
        wl = uint2{(uint32_t)half_bits(ll[0]) | (rl << 16),
                   (uint32_t)half_bits(ll[1]) | (rl & 0xffff0000u)};
      }
    }
    // the stores
    if (m < M) *(f32x4*)(a.hidden_out + (int64_t)(m0 + m) * N + n) = h;
    if (a.ss_out && (threadIdx.x & 7) == 0) a.ss_out[(int64_t)mt * N + nt * 32 + m] = q;
    if (a.pre_out) {
      if ((threadIdx.x & 7) == 0) a.pre_xs_out[(int64_t)mt * N + nt * 32 + m] = xsum;
      if (m < M) {
        uint16_t* dst = (uint16_t*)a.pre_out + (int64_t)(m0 + m) * N + n;
        *(uint2*)dst = wh;
        *(uint2*)(dst + (int64_t)M_all * N) = wl;
        if (over) raise_range(a);
      }
    }
  } else if (m < M) {
    *(f32x4*)(a.y + (int64_t)(m0 + m) * N + n) = v;
  }
  if (KS > 1 && threadIdx.x == 0) reset_counter(&counters[nt], a.fenced);
}

// gate|up + SwiGLU of <= 32 rows per row tile over the whole K, without
// split-K (q4 weights, pre-scaled norm input, K = 64 G with G in {8, 16}).
// The fused weight interleaves [gate 64 | up 64] per 128 columns, so n-tiles
// 4b + i (gate) and 4b + 2 + i (up) give SwiGLU outputs 64b + 32i .. + 31:
// work-group (p = 2b + i, 16-row half h of a row tile) owns that pair for 16
// rows. Its activation slice (16 rows x K, hi and lo planes) goes into LDS by
// direct-to-LDS loads; wave w of 8 takes the 64-k units G/8 w .. + G/8 - 1 of
// both tiles (one read of the A fragments feeds the gate and the up MFMAs, the
// 16 rows' hi and lo planes stacked as the MFMA's 32 rows); the waves' tiles are
// added in LDS in wave order and SwiGLU runs on the sums. No partial tiles,
// arrival counters or last work-group, whose round trips cost more than every
// work-group staging all of K; 16-row halves halve that staging and keep two
// work-groups per CU. Leading arguments as in skinny_wide_kernel (planes, their
// per-32-column sums, sums of squares, the planes' scale c per row).
constexpr int GU_RH = 16;  // rows per work-group
constexpr int GU_RS = 36;  // floats per row of a wave's tile in LDS (16-byte rows, padded)
// bytes of LDS shared by the activation (before the MFMAs) and the waves' tiles (after)
constexpr int gu_region_bytes(int G) {
  return 2 * GU_RH * (G * 64 + 8) * 2 > 8 * 2 * GU_RH * GU_RS * 4 ? 2 * GU_RH * (G * 64 + 8) * 2
                                                                 : 8 * 2 * GU_RH * GU_RS * 4;
}
template <int G>
__global__ __launch_bounds__(512) void skinny_gu_kernel(
    const uint32_t* __restrict__ qw, const uint32_t* __restrict__ sbp,
    const uint16_t* __restrict__ planes, const float* __restrict__ xs_part,
    const float* __restrict__ ss_arg, const float* __restrict__ sc_in, int* perr,
    uint32_t dims0, uint32_t dims1, const FusedArgs a) {
  static_assert(G == 8 || G == 16, "K = 512 or 1024");
  constexpr int K = G * 64, ROW = K + 8, CPR = G / 8, UPW = G / 8, RH = GU_RH;
  constexpr int RS = GU_RS;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int M, N, Kd, KS, n_xcc, fenced;
  sk_dims(dims0, dims1, M, N, Kd, KS, n_xcc, fenced);
  (void)Kd, (void)KS, (void)n_xcc, (void)fenced, (void)perr;
  // rows m0 .. m0 + M - 1 of the forward: half hr of 32-row tile mt
  const int mt = blockIdx.y >> 1, hr = blockIdx.y & 1, tr0 = RH * hr;
  const int m0 = 32 * mt + tr0, M_all = M;
  M = min(RH, M_all - m0);
  if (M <= 0) return;  // work-group-uniform: a half with no rows
  const int blk = blockIdx.x >> 1, half = blockIdx.x & 1;
  const int nt_g = 4 * blk + half, nt_u = nt_g + 2;
  extern __shared__ __align__(16) char smem[];
  uint16_t* act = (uint16_t*)smem;                   // [2 planes][RH][ROW] halves
  float* xss = (float*)(smem + gu_region_bytes(G));  // [G][32] group sums
  float* rfac = xss + G * 32;                        // [32] rinv / c
  float* red = rfac + 32;                            // [16][32] sums of squares
  float* cl = red + 16 * 32;                         // [32] c
  float* red2 = (float*)smem;                        // [8 waves][2 tiles][RH][RS] after the MFMAs

  // 1. the small L2-resident loads: thread t takes row t % 32 (clamped to the
  // work-group's rows), partial sums of squares t / 32 and t / 32 + 16, the two
  // 32-column sums of group t / 32, and c (unconditional, masked after the wait)
  const int np = K >> 5;  // 32-column partial sums per row (<= 32)
  const int r32 = threadIdx.x & 31, q16 = threadIdx.x >> 5;
  const float* ss_in = ss_arg + (int64_t)mt * K;
  const float* xsp = xs_part + (int64_t)mt * K;
  const int rr = min(r32, M - 1), gx = min(q16, G - 1);
  const float sv0 = ss_in[min(q16, np - 1) * 32 + tr0 + rr];
  const float sv1 = ss_in[min(q16 + 16, np - 1) * 32 + tr0 + rr];
  const float xp0 = xsp[(2 * gx) * 32 + tr0 + rr], xp1 = xsp[(2 * gx + 1) * 32 + tr0 + rr];
  const float c_in = sc_in[m0 + rr];
  // 2. this wave's weights (both tiles; issued before the activation so that
  // their HBM latency starts first)
  u32x4 wg[UPW], wu[UPW];
  uint32_t sg[UPW], su[UPW];
#pragma unroll
  for (int j = 0; j < UPW; ++j) {
    const int g = wave * UPW + j;
    wg[j] = __builtin_nontemporal_load(q4_tile_words(qw, nt_g, G, g, lane));
    wu[j] = __builtin_nontemporal_load(q4_tile_words(qw, nt_u, G, g, lane));
    sg[j] = q4_tile_sb(sbp, nt_g, G, g, lane);
    su[j] = q4_tile_sb(sbp, nt_u, G, g, lane);
  }
  // 3. the activation into LDS: 1 KiB chunks (plane, row, piece), 16 B a lane;
  // rows past M repeat row M - 1 (their results are never stored)
#pragma unroll
  for (int i = 0; i < 2 * RH * CPR / 8; ++i) {
    const int ch = wave + 8 * i, pl = ch / (RH * CPR), r = (ch / CPR) % RH, q = ch % CPR;
    const uint16_t* src = planes + ((int64_t)pl * M_all + m0 + min(r, M - 1)) * K + q * 512 + lane * 8;
    __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)(
                                         act + (pl * RH + r) * ROW + q * 512),
                                     16, 0, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
  red[q16 * 32 + r32] = sv0 * (q16 < np ? 1.f : 0.f) + sv1 * (q16 + 16 < np ? 1.f : 0.f);
  if ((int)threadIdx.x < 32 * G) xss[threadIdx.x] = xp0 + xp1;
  if (threadIdx.x < 32) cl[threadIdx.x] = c_in;
  __builtin_amdgcn_s_waitcnt(0);  // this wave's activation chunks landed
  __syncthreads();                // ... and every other wave's
  if (threadIdx.x < 32) {
    float ssum = 0.f;
#pragma unroll
    for (int g = 0; g < 16; ++g) ssum += red[g * 32 + threadIdx.x];
    const float ri = 1.f / sqrtf(ssum / (float)K + a.eps);
    rfac[threadIdx.x] = (int)threadIdx.x < M ? ri / cl[threadIdx.x] : 0.f;
    if (a.pre_sc_out && blockIdx.x == 0 && (int)threadIdx.x < M)
      a.pre_sc_out[m0 + threadIdx.x] = pre_scale_of(ri);
  }
  // 4. this wave's units, each A fragment read once for both tiles: LDS rows
  // 0-15 are the hi plane and 16-31 the lo plane, the MFMA's 32 rows
  static_assert(RH == 16, "hi and lo planes of 16 rows fill the MFMA's 32 rows");
  float acc_g[8] = {}, acc_u[8] = {};
  const _Float16* arow = (const _Float16*)act + (lane & 31) * ROW + 32 * (lane >> 5);
#pragma unroll
  for (int j = 0; j < UPW; ++j) {
    const int g = wave * UPW + j;
    f16x8 af[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) af[t] = *(const f16x8*)(arow + g * 64 + 8 * t);
    float xsr[16];
    load_row_sums(xss + g * 32, lane, xsr);
    q4_group_mma_hl(acc_g, af, xsr, wg[j], sg[j]);
    q4_group_mma_hl(acc_u, af, xsr, wu[j], su[j]);
  }
  __syncthreads();  // every wave is done with the activation; rfac is written
  // accumulator i < 8 holds row mfma_row(i, lane) < 16
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int row = mfma_row(r, lane);
    red2[((wave * 2 + 0) * RH + row) * RS + (lane & 31)] = acc_g[r];
    red2[((wave * 2 + 1) * RH + row) * RS + (lane & 31)] = acc_u[r];
  }
  __syncthreads();
  // 5. SwiGLU: thread t < 128 takes row t / 8, outputs 4 (t % 8) .. + 3 of the
  // pair, the 8 waves' tiles added in wave order and scaled by the row's
  // factor; an 8-column ACT_F16P chunk (order 0,4,1,5,2,6,3,7) is two threads'
  // halves, paired by a lane exchange (the even thread stores words 0-1, the
  // odd one words 2-3; rows past M compute and exchange, then store nothing)
  if (threadIdx.x >= 8 * RH) return;
  const int m = threadIdx.x >> 3, q = threadIdx.x & 7;
  f32x4 gs = *(const f32x4*)(red2 + (0 * RH + m) * RS + 4 * q);
  f32x4 us = *(const f32x4*)(red2 + (1 * RH + m) * RS + 4 * q);
#pragma unroll
  for (int w = 1; w < 8; ++w) {
    gs += *(const f32x4*)(red2 + ((w * 2 + 0) * RH + m) * RS + 4 * q);
    us += *(const f32x4*)(red2 + ((w * 2 + 1) * RH + m) * RS + 4 * q);
  }
  const float f = rfac[m];
  _Float16 hh[4], ll[4];
  bool over = false;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float gv = gs[e] * f, uv = us[e] * f;
    const float y = gv * (1.f / (1.f + expf(-gv))) * uv;
    hh[e] = (_Float16)y;
    ll[e] = f16_lo(y, hh[e]);
    over = over || f16_overflows(y);
  }
  const bool odd = q & 1;
  const uint32_t sh = odd ? pack_half2(hh[0], hh[1]) : pack_half2(hh[2], hh[3]);
  const uint32_t sl = odd ? pack_half2(ll[0], ll[1]) : pack_half2(ll[2], ll[3]);
  const uint32_t rh = (uint32_t)__shfl_xor((int)sh, 1), rl = (uint32_t)__shfl_xor((int)sl, 1);
  uint2 wh, wl;
  if (odd) {
    wh = uint2{(rh & 0xffffu) | ((uint32_t)half_bits(hh[2]) << 16),
               (rh >> 16) | ((uint32_t)half_bits(hh[3]) << 16)};
    wl = uint2{(rl & 0xffffu) | ((uint32_t)half_bits(ll[2]) << 16),
               (rl >> 16) | ((uint32_t)half_bits(ll[3]) << 16)};
  } else {
    wh = uint2{(uint32_t)half_bits(hh[0]) | (rh << 16), (uint32_t)half_bits(hh[1]) | (rh & 0xffff0000u)};
    wl = uint2{(uint32_t)half_bits(ll[0]) | (rl << 16), (uint32_t)half_bits(ll[1]) | (rl & 0xffff0000u)};
  }
  if (m >= M) return;
  const int F = N >> 1;
  uint16_t* dst = (uint16_t*)a.act_out + (int64_t)(m0 + m) * F + 64 * blk + 32 * half + 4 * q;
  *(uint2*)dst = wh;
  *(uint2*)(dst + (int64_t)M_all * F) = wl;
  if (over) raise_range(a);
}
#define SK_GU_LDS(G) (gu_region_bytes(G) + ((G) * 32 + 32 + 16 * 32 + 32) * 4)
template __global__ void skinny_gu_kernel<8>(const uint32_t*, const uint32_t*, const uint16_t*,
                                             const float*, const float*, const float*, int*,
                                             uint32_t, uint32_t, const FusedArgs);
template __global__ void skinny_gu_kernel<16>(const uint32_t*, const uint32_t*, const uint16_t*,
                                              const float*, const float*, const float*, int*,
                                              uint32_t, uint32_t, const FusedArgs);

#define DRT_WIDE(W, E, U, P)                                                               \
  template __global__ void skinny_wide_kernel<W, E, U, P>(const uint32_t*, const uint32_t*,   \
                                                          const float*, const uint16_t*,      \
                                                          const float*, const float*, int*,   \
                                                          uint32_t, uint32_t, const FusedArgs);
#define DRT_WIDE_U(W, E, P) \
  DRT_WIDE(W, E, 1, P) DRT_WIDE(W, E, 2, P) DRT_WIDE(W, E, 4, P) DRT_WIDE(W, E, 8, P)
DRT_WIDE_U(W_Q4, EPI_QKV, true) DRT_WIDE_U(W_Q4, EPI_SWIGLU, true)
DRT_WIDE_U(W_Q4, EPI_QKV, false) DRT_WIDE_U(W_Q4, EPI_SWIGLU, false)
DRT_WIDE_U(W_BF16, EPI_QKV, false) DRT_WIDE_U(W_BF16, EPI_SWIGLU, false)
#undef DRT_WIDE_U
#undef DRT_WIDE
#define DRT_NARROW(W, E, UW) DRT_NARROW_X(W, E, UW, 0)
#define DRT_NARROW_X(W, E, UW, X)                                                             \
  template __global__ void skinny_narrow_kernel<W, E, UW, X>(const uint32_t*, const uint32_t*, \
                                                             const uint16_t*, int*, uint32_t,   \
                                                             uint32_t, const FusedArgs);
DRT_NARROW(W_Q4, EPI_RESID, 1) DRT_NARROW(W_Q4, EPI_RESID, 2)
DRT_NARROW(W_Q4, EPI_STORE, 1) DRT_NARROW(W_Q4, EPI_STORE, 2)
DRT_NARROW(W_BF16, EPI_RESID, 1) DRT_NARROW(W_BF16, EPI_RESID, 2)
DRT_NARROW(W_BF16, EPI_STORE, 1) DRT_NARROW(W_BF16, EPI_STORE, 2)
DRT_NARROW_X(W_Q4, EPI_STORE, 1, 1) DRT_NARROW_X(W_Q4, EPI_STORE, 2, 1)
DRT_NARROW_X(W_Q4, EPI_STORE, 1, 2) DRT_NARROW_X(W_Q4, EPI_STORE, 2, 2)
#undef DRT_NARROW_X
#undef DRT_NARROW

namespace drt {
namespace {


// Wide: units per work-group U (instantiated values) with G % U == 0, the largest
// U whose split still gives >= 128 work-groups; else the smallest U available.
// (U <= 8: the hi and lo activation of more units would not fit the registers.)
int wide_units(int N, int K) {
  const int G = K / 64, NG = N / 128;
  int best = 0;
  for (int u : {8, 4, 2, 1}) {
    if (G % u) continue;
    if (best == 0) best = u;
    if (NG * (G / u) >= 128) return u;
    best = u;
  }
  return best;
}

// Narrow: K slices KS (a divisor of G) - the fewest giving >= 256 work-groups.
int narrow_slices(int N, int K) {
  const int G = K / 64, NT = N / 32;
  int ks = 1;
  for (int d = 1; d <= G; ++d) {
    if (G % d) continue;
    ks = d;
    if (NT * d >= 256) break;
  }
  return ks;
}

}  // namespace

// Whether work-group i of a launch runs on XCD i % n_xcc (the layout the
// split-K exchange assumes), from one probe launch of 4 * 64 work-groups.
bool probe_round_robin(int n_xcc, int* scratch_dev, hipStream_t s) {
  if (n_xcc <= 1) return true;
  constexpr int WGS = 256;
  hipLaunchKernelGGL(xcc_probe_kernel, dim3(WGS), dim3(64), 0, s, scratch_dev);
  DRT_HIP(hipGetLastError());
  std::vector<int> xcc(WGS);
  DRT_HIP(hipMemcpyAsync(xcc.data(), scratch_dev, WGS * sizeof(int), hipMemcpyDeviceToHost, s));
  DRT_HIP(hipStreamSynchronize(s));
  for (int i = 0; i < WGS; ++i)
    if (xcc[i] != i % n_xcc) return false;
  return true;
}

size_t skinny_part_floats(int N, int K) {
  if (K % 64 || N % 32) return 0;
  size_t wide = 0;
  if (N % 128 == 0) {
    const int u = wide_units(N, K);
    wide = u ? (size_t)(N / 128) * (K / 64 / u) * 4096 : 0;
  }
  const size_t narrow = (size_t)(N / 32) * narrow_slices(N, K) * 1024;
  return std::max(wide, narrow);
}

int skinny_counters(int N) { return N / 32; }

bool skinny_supported(int kind, int N, int K) {
  if (K % 64 || N % 32 || N >= 65536 || K >= 65536) return false;
  if (kind == FL_QKV || kind == FL_SWIGLU) {
    const int U = wide_units(N, K);
    return N % 128 == 0 && K / 32 <= 8 * SK_SS_PER_THREAD && U && K / 64 / U <= SK_KS_MAX;
  }
  return narrow_slices(N, K) <= SK_KS_MAX;
}

namespace {
uint32_t sk_dims1(const FusedArgs& a, int KS) {
  return (uint32_t)a.M | ((uint32_t)KS << 8) | ((uint32_t)a.n_xcc << 16) |
         ((uint32_t)(a.fenced ? 1 : 0) << 24);
}
}  // namespace

static bool skinny_launch(const FusedArgs& a, int kind, hipStream_t s);

bool skinny_linear(const FusedArgs& a, int kind, hipStream_t s) {
  // pre-scaled planes in or out have no other kernel: refusing them is an error
  const bool pre = a.pre_sc_in || a.pre_out;
  if (pre) {
    require(a.qw && (kind == FL_RESID ? a.pre_xs_out && a.pre_norm && a.pre_sc
                                      : a.act && a.act_xsum && a.x_in == 0),
            "pre-scaled planes: q4 weights and every plane argument required");
  }
  const bool ok = skinny_launch(a, kind, s);
  require(ok || !pre, "pre-scaled planes: the split-K kernels refused the linear");
  return ok;
}

static bool skinny_launch(const FusedArgs& a, int kind, hipStream_t s) {
  const int MT = (a.M + 31) / 32;
  if ((!a.qw && !a.wb) || a.M < 1 || MT > a.sk_row_tiles || !a.part ||
      !a.counters || a.K % 64 || a.N % 32 || a.n_xcc < 1)
    return false;
  const bool bf = a.qw == nullptr;
  const uint32_t* wq = bf ? (const uint32_t*)a.wb : a.qw;
  // the packed sizes of the kernels' leading arguments (see sk_dims)
  require(a.N < 65536 && a.K < 65536 && a.M < 256 && a.n_xcc < 256,
          "split-K linear sizes exceed the packed argument fields");
  const uint32_t dims0 = (uint32_t)a.N | ((uint32_t)a.K << 16);
  const int G = a.K / 64;
  const double bytes = (bf ? 2.0 * a.N * a.K : (double)a.N * a.K / 2 + (double)a.N * a.K / 16) +
                       2.0 * a.M * a.K + 2.0 * a.M * a.N;
  if (kind == FL_SWIGLU && a.pre_sc_in && !bf && a.x_in == 0 && a.ss_in && a.N % 128 == 0 &&
      (a.K == 512 || a.K == 1024)) {
    // gate|up over the whole K (no split-K): 64-column work-groups of 8 waves
    const dim3 grid((unsigned)(a.N / 64), 2 * MT);  // 16-row halves of the row tiles
#define DRT_GU(GG)                                                                         \
  {                                                                                        \
    auto fn = skinny_gu_kernel<GG>;                                                        \
    static size_t granted = 0;                                                             \
    grant_lds((const void*)fn, SK_GU_LDS(GG), granted);                                    \
    DRT_LAUNCH(Profiler::GEMM, bytes, fn, grid, dim3(512), SK_GU_LDS(GG), s, wq, a.sb,     \
               (const uint16_t*)a.act, a.act_xsum, a.ss_in, a.pre_sc_in, a.placement_err,  \
               dims0, sk_dims1(a, 1), a);                                                  \
  }
    if (a.K == 1024) DRT_GU(16) else DRT_GU(8)
#undef DRT_GU
    DRT_HIP(hipGetLastError());
    return true;
  }
  if (kind == FL_QKV || kind == FL_SWIGLU) {
    if (a.x_in != 0 || !a.ss_in || a.N % 128 || a.K / 32 > 8 * SK_SS_PER_THREAD) return false;
    const bool pre = a.pre_sc_in != nullptr;  // q4 (checked by the caller)
    // PRE: the planes and their sums take the places of the rows and the norm weight
    const float* x0 = pre ? (const float*)a.act : a.hidden;
    const uint16_t* x1 = pre ? (const uint16_t*)a.act_xsum : a.norm_w;
    const int U = wide_units(a.N, a.K);
    if (!U) return false;
    const int KS = G / U, NG = a.N / 128;
    if (KS > SK_KS_MAX || (size_t)NG * KS * 4096 > a.part_floats || NG > a.n_counters)
      return false;  // (padding work-groups past the last block exit before any access)
    const size_t lds = SK_WIDE_LDS(U);
    const dim3 grid((unsigned)((NG + a.n_xcc - 1) / a.n_xcc * a.n_xcc * KS), MT);
#define DRT_SW1(W, E, UU, P)                                                         \
  {                                                                                  \
    auto fn = skinny_wide_kernel<W, E, UU, P>;                                       \
    static size_t granted = 0;                                                       \
    grant_lds((const void*)fn, lds, granted);                                        \
    DRT_LAUNCH(Profiler::GEMM, bytes, fn, grid, dim3(256), lds, s, wq, a.sb, x0, x1,   \
               a.ss_in, a.pre_sc_in, a.placement_err, dims0, sk_dims1(a, KS), a);    \
  }
#define DRT_SW(E, UU)                          \
  {                                            \
    if (bf) DRT_SW1(W_BF16, E, UU, false)      \
    else if (pre) DRT_SW1(W_Q4, E, UU, true)   \
    else DRT_SW1(W_Q4, E, UU, false)           \
  }
#define DRT_SW_U(E)                                  \
  switch (U) {                                       \
    case 1: DRT_SW(E, 1) break;                      \
    case 2: DRT_SW(E, 2) break;                      \
    case 4: DRT_SW(E, 4) break;                      \
    default: DRT_SW(E, 8) break;                     \
  }
    if (kind == FL_QKV) {
      DRT_SW_U(EPI_QKV)
    } else {
      DRT_SW_U(EPI_SWIGLU)
    }
#undef DRT_SW_U
#undef DRT_SW
#undef DRT_SW1
  } else if (kind == FL_RESID || kind == FL_STORE) {
    const int KS = narrow_slices(a.N, a.K), NT = a.N / 32;
    if (KS > SK_KS_MAX || (size_t)NT * KS * 1024 > a.part_floats || NT > a.n_counters)
      return false;
    const int per_wave = (G / KS + 3) / 4;
    const dim3 grid((unsigned)((NT + a.n_xcc - 1) / a.n_xcc * a.n_xcc * KS), MT);
#define DRT_SN1(W, E, UW) DRT_SN1X(W, E, UW, 0)
#define DRT_SN1X(W, E, UW, X)                                                      \
  {                                                                                \
    auto fn = skinny_narrow_kernel<W, E, UW, X>;                                   \
    static size_t granted = 0;                                                     \
    grant_lds((const void*)fn, SK_NARROW_LDS(UW), granted);                        \
    DRT_LAUNCH(Profiler::GEMM, bytes, fn, grid, dim3(256), SK_NARROW_LDS(UW), s, wq, a.sb, \
               (const uint16_t*)a.act, a.placement_err, dims0, sk_dims1(a, KS), a);      \
  }
#define DRT_SN(E, UW)                  \
  {                                    \
    if (bf) DRT_SN1(W_BF16, E, UW)     \
    else DRT_SN1(W_Q4, E, UW)          \
  }
    // (more than two units per wave: loops of two, the hi and lo fragments of
    // a larger batch would not fit the registers). Two row tiles double the
    // work-groups: one unit at a time keeps two of them per CU (the LDS of
    // two-unit staging holds one), so they run in one round instead of two.
    const bool one_unit = per_wave <= 1 || MT > 1;
    if (a.x_in != 0) {
      if (kind != FL_STORE || bf) return false;
      if (a.x_in == 1) {
        if (one_unit) DRT_SN1X(W_Q4, EPI_STORE, 1, 1) else DRT_SN1X(W_Q4, EPI_STORE, 2, 1)
      } else {
        if (one_unit) DRT_SN1X(W_Q4, EPI_STORE, 1, 2) else DRT_SN1X(W_Q4, EPI_STORE, 2, 2)
      }
    } else if (kind == FL_RESID) {
      if (one_unit) DRT_SN(EPI_RESID, 1) else DRT_SN(EPI_RESID, 2)
    } else {
      if (one_unit) DRT_SN(EPI_STORE, 1) else DRT_SN(EPI_STORE, 2)
    }
#undef DRT_SN
#undef DRT_SN1X
#undef DRT_SN1
  } else {
    return false;
  }
  DRT_HIP(hipGetLastError());
  return true;
}

}  // namespace drt
