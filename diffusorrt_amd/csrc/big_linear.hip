// Large-M q4 linear for gfx950: the forwards of more than 32 rows (Dream's
// full canvas, BD3 prefix commits). At these sizes the contraction is MFMA
// bound, so the weights are dequantized once per work-group into fp16 MFMA
// operands (w = s * q + b, one fp16 rounding; backends/mlx_ops.py:97-130 for the
// linear, :43-60 for the MLX q4 g64 packing) instead of the per-group scaled
// accumulators of the weight-streaming kernels, whose two FMAs per output and
// group would cost as much VALU time as the MFMAs.
//
// Work-group tile: 128 rows x 256 columns, 4 waves side by side in N; a wave
// owns 128 x 64 (4 x 2 MFMA 32x32x16 tiles, 128 fp32 accumulators per lane).
//   A (the ACT_F16P activation: hi and lo planes of [M][K]) is streamed per
//     64-k group straight into LDS (global_load_lds, no registers held),
//     double buffered: 2 planes x 128 rows x 128 B per group. Rows are stored
//     unpadded with the 16-byte chunks of row r permuted (chunk c at position
//     c ^ (r & 7) ^ ((r >> 3) & 1)), so the MFMA fragment reads of 8 consecutive
//     rows hit 8 different 16-byte bank groups of a 128-byte row, and those of
//     16 consecutive rows 16 different ones of two rows (256 bytes): no bank
//     conflict whether the LDS serves 8 or 16 lanes of a 16-byte read per
//     cycle. Each MFMA step multiplies hi and lo by the same B.
//   B (q4 tile layout: per 32-column n-tile and 64-k group, 1 KiB of words and
//     32 scale|bias pairs) goes straight from global memory to registers and is
//     dequantized there, one k step at a time: 2 n-tiles per wave per group.
// Group g + 1's loads are issued right after the barrier that proves group g
// in LDS, so they stream during g's MFMAs; two work-groups per CU (<= 256
// registers per lane) hide each other's waits.
// Split-K over blockIdx.z (KS slices) writes fp32 partial slices y + ks * M * N
// that a reduce pass sums (residual_norm_kernel).
// Split last round (tail.kt >= 2, one-dimensional grid): when the tiles fill the
// device's work-group slots (two per CU) once with a few left over, the first
// tail.full tiles run whole and each of the remaining ones is split into tail.kt
// K ranges on as many work-groups of one XCD, so the last round takes a fraction
// of a tile instead of leaving most CUs idle. The slices meet as in the split-K
// decode linears: each writes its partial tile, counts its arrival in that XCD's
// L2, and the last to arrive adds the slices in slice order and runs the epilogue.
// Epilogues run on 32-row pieces of the tile staged through LDS:
//   EPI_STORE : y (+ bias on slice 0)
//   EPI_SWIGLU: [gate 64 | up 64] column blocks -> silu(g) * u -> ACT_F16P
//   EPI_QKV   : (+ bias), q/k RMSNorm, RoPE, Q out / K,V into the tiled cache
//   EPI_LMSTAT: the LM head's softmax statistics per (row, 64-column block),
//               the logits themselves only on request
#include "fused.h"
#include "gemm_core.h"
#include "launch.h"

#include "linear_dev.h"
#include "lmstat.h"

namespace {

constexpr int BG_WM = 128;                     // rows per work-group
constexpr int BG_WN = 256;                     // columns per work-group (4 waves x 64)
constexpr int BG_PLANE_BYTES = BG_WM * 128;    // one plane of one group: 128 rows x 64 halves
constexpr int BG_BUF_BYTES = 2 * BG_PLANE_BYTES;  // hi + lo planes of one group
constexpr int BG_EROW = BG_WN + 4;             // floats per LDS row of an epilogue piece
constexpr int BG_V_OFF = (32 * BG_EROW * 4 + 15) / 16 * 16;  // V tile half, after the piece
constexpr int BG_LDS = 2 * BG_BUF_BYTES;       // two group buffers (the epilogue reuses them)
static_assert(BG_V_OFF + 4096 * 2 <= BG_LDS, "epilogue piece + V tile must fit the A buffers");

template <int S> struct Slot { static constexpr int value = S; };

typedef _Float16 h2v __attribute__((ext_vector_type(2)));

// fp16 B fragment of k step t of one 64-k group of one 32-column n-tile: word t
// of the lane holds the 8 k of the step in the ACT_F16P order (0,4,1,5,2,6,3,7);
// nibble pairs become (1024 + q) halves by bit placement, then q * s + b in one fma.
DRT_DEV f16x8 dequant_q4_step(uint32_t wt, uint32_t sbv) {
  const _Float16 s = (_Float16)bf16_bits_to_float(sbv & 0xffffu);
  const _Float16 z = (_Float16)bf16_bits_to_float(sbv >> 16);
  const h2v s2 = {s, s}, z2 = {z, z};
  const h2v k2 = {(_Float16)-1024.f, (_Float16)-1024.f};
  u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const h2v h = __builtin_bit_cast(h2v, ((wt >> (4 * e)) & 0x000F000Fu) | 0x64006400u);
    o[e] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(h + k2, s2, z2));
  }
  return __builtin_bit_cast(f16x8, o);
}

// dequant_q4_step with the group's scale and bias already in fp16 pairs and
// the nibble mask in a register (one v_and_or_b32 per nibble pair)
DRT_DEV f16x8 dequant_q4_step_sz(uint32_t wt, h2v s2, h2v z2, uint32_t mask) {
  const h2v k2 = {(_Float16)-1024.f, (_Float16)-1024.f};
  u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const h2v h = __builtin_bit_cast(h2v, ((wt >> (4 * e)) & mask) | 0x64006400u);
    o[e] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(h + k2, s2, z2));
  }
  return __builtin_bit_cast(f16x8, o);
}

// LDS fragment read the compiler does not see: a plain read after a
// direct-to-LDS load makes it wait for every global load in flight first
// (it cannot tell the group being read from the one being filled).
DRT_DEV void lds_read16(f16x8& v, uint32_t addr) {
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
}
// ... at a constant byte offset from addr (the instruction's offset field)
template <int OFF>
DRT_DEV void lds_read16o(f16x8& v, uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds_read offset field");
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
}

}  // namespace

struct BgTail {
  int full = 0;            // whole tiles (the first work-groups, dealt in XCD runs)
  int kt = 0;              // K slices per remaining tile (0: the three-dimensional grid)
  float* part = nullptr;   // [remaining tiles][kt][128 * 256] partial tiles
  int* count = nullptr;    // [remaining tiles] arrival counters, zero on entry and exit
};
constexpr int BG_TAIL_KT_MAX = 8;

template <int EPI>
__global__ __launch_bounds__(256, 2) void big_q4_kernel(const FusedArgs a, int KS, const BgTail tail) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: LDS bases in SGPRs
  const int M = a.M, N = a.N, K = a.K, G = K >> 6;
  // Tiles t = y + MT (x + NX z) (row tile y fastest), dealt to the XCDs in
  // contiguous runs: work-group b runs on XCD b % 8 and takes tile
  // (b % 8) * T8 / 8 + b / 8 (the last T - T8 tiles as they come), so an XCD's
  // L2 holds whole columns of row tiles: each weight tile is fetched by one XCD,
  // and a K slice of a split-K grid whose tiles fill an XCD's run stays on it.
  const int MT = (M + BG_WM - 1) / BG_WM, NX = (N + BG_WN - 1) / BG_WN;
  auto xcd_run = [](int b, int T) {
    const int T8 = T & ~7;
    return b < T8 ? (b & 7) * (T8 >> 3) + (b >> 3) : b;
  };
  int tile_x, tile_y, ks, tail_idx = -1;
  {
    const int T = (int)(gridDim.x * gridDim.y * gridDim.z);
    const int t = xcd_run((int)(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z)), T);
    tile_y = t % MT;
    tile_x = (t / MT) % NX;
    ks = t / (MT * NX);
  }
  if (EPI == EPI_SWIGLU && tail.kt) {
    // work-group b: tile b (the first full tiles in XCD runs), or K slice of a
    // remaining tile; the slices of one remaining tile share b % 8, i.e. one
    // XCD (full % 8 == 0)
    const int b = blockIdx.x;
    int t = xcd_run(b, tail.full);
    ks = 0;
    KS = 1;
    if (b >= tail.full) {
      const int j = b - tail.full, q = j >> 3;
      tail_idx = (j & 7) + 8 * (q / tail.kt);
      ks = q % tail.kt;
      KS = tail.kt;
      t = tail.full + tail_idx;
      // the slices meet through this XCD's L2: a work-group found elsewhere
      // raises the placement error (the host then fails the forward)
      if (threadIdx.x == 0 && a.placement_err) {
        const int xcc = (int)(__builtin_amdgcn_s_getreg((31 << 11) | 20) & 0xf);  // HW_REG_XCC_ID
        if (xcc != (b & 7))
          __hip_atomic_fetch_or(a.placement_err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    tile_y = t % MT;
    tile_x = t / MT;
  }
  const int n0 = tile_x * BG_WN, m0 = tile_y * BG_WM;
  const int g_lo = (int)((int64_t)G * ks / KS), g_hi = (int)((int64_t)G * (ks + 1) / KS);
  const int n_g = g_hi - g_lo;
  const int NT = N >> 5;
  // this wave's two n-tiles, clamped so that loads stay in bounds (columns
  // beyond N are computed from the last n-tile and never stored)
  const int nt0 = min((n0 >> 5) + 2 * wave, NT - 1);
  const int nt1 = min((n0 >> 5) + 2 * wave + 1, NT - 1);
  extern __shared__ __align__(16) char smem[];
  const _Float16* act = (const _Float16*)a.act;

  u32x4 wq[2][2];
  uint32_t wsb[2][2];
  // A of group g into buffer buf: plane pl, 8-row block blk = wave + 4i is one
  // wave instruction (lane l: row blk*8 + (l >> 3), LDS position l & 7, which
  // holds the row's chunk (l & 7) ^ (l >> 3) ^ (blk & 1), blk & 1 being
  // wave & 1); rows past M re-read row M - 1,
  // whose copies feed only outputs that are never stored. Addresses are a
  // uniform base per group plus 32-bit lane offsets (activation < 4 GiB),
  // recomputed at each issue (24-bit multiplies, from lane values made opaque
  // there) instead of staying live across the loop.
  const int row_l = m0 + wave * 8 + (lane >> 3);
  const uint32_t col_l = (uint32_t)(((lane & 7) ^ (lane >> 3) ^ (wave & 1)) * 16);
  const uint32_t K2 = (uint32_t)K * 2u;
  const char* act_b = (const char*)act;
  auto issue = [&](int g, int buf, auto slot) {
    constexpr int S = decltype(slot)::value;
    const char* ag = act_b + (size_t)g * 128;
    int rl = row_l;
    uint32_t cl = col_l;
    asm volatile("" : "+v"(rl), "+v"(cl));
#pragma unroll
    for (int pl = 0; pl < 2; ++pl)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t m = (uint32_t)(min(rl + 32 * i, M - 1) + pl * M);
        char* dst = smem + buf * BG_BUF_BYTES + pl * BG_PLANE_BYTES + (wave + 4 * i) * 1024;
        __builtin_amdgcn_global_load_lds(
            (__attribute__((address_space(1))) void*)(ag + (__umul24(m, K2) + cl)),
            (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
      }
    wq[S][0] = *q4_tile_words(a.qw, nt0, G, g, lane);
    wq[S][1] = *q4_tile_words(a.qw, nt1, G, g, lane);
    wsb[S][0] = q4_tile_sb(a.sb, nt0, G, g, lane);
    wsb[S][1] = q4_tile_sb(a.sb, nt1, G, g, lane);
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i][0] = acc[i][1] = f32x16{};

  // this lane's fragment row within each 32-row m-tile is lane & 31; its k
  // chunk at step t is 4 * (lane >> 5) + t, stored at position
  // chunk ^ (row & 7) ^ ((row >> 3) & 1) (row & 15 == lane & 15)
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem + (lane & 31) * 128;
  // one k step's operands (A hi and lo fragments, the two dequantised B
  // fragments); steps alternate between two sets, the next step's read and
  // dequantised while the current step's MFMAs run
  struct Ops {
    f16x8 h[4], l[4], b[2];
  };
  uint32_t nib_mask = 0x000F000Fu;
  asm volatile("" : "+v"(nib_mask));  // in a register: v_and_or_b32 takes one constant
  h2v gs2[2], gz2[2];                // the current group's scale and bias pairs
  auto group_scales = [&](auto slot) {
    constexpr int S = decltype(slot)::value;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const _Float16 sc = (_Float16)bf16_bits_to_float(wsb[S][j] & 0xffffu);
      const _Float16 zb = (_Float16)bf16_bits_to_float(wsb[S][j] >> 16);
      gs2[j] = h2v{sc, sc};
      gz2[j] = h2v{zb, zb};
    }
  };
  auto load_ops = [&](Ops& o, int buf, int t, auto slot) {
    constexpr int S = decltype(slot)::value;
    // m-tile i of the hi plane at + 4096 i, of the lo plane at + BG_PLANE_BYTES + 4096 i
    const uint32_t ab =
        lds0 + buf * BG_BUF_BYTES +
        (uint32_t)(((4 * (lane >> 5) + t) ^ (lane & 7) ^ ((lane >> 3) & 1)) * 16);
    lds_read16o<0>(o.h[0], ab);
    lds_read16o<BG_PLANE_BYTES>(o.l[0], ab);
    lds_read16o<4096>(o.h[1], ab);
    lds_read16o<BG_PLANE_BYTES + 4096>(o.l[1], ab);
    lds_read16o<8192>(o.h[2], ab);
    lds_read16o<BG_PLANE_BYTES + 8192>(o.l[2], ab);
    lds_read16o<12288>(o.h[3], ab);
    lds_read16o<BG_PLANE_BYTES + 12288>(o.l[3], ab);
#pragma unroll
    for (int j = 0; j < 2; ++j) o.b[j] = dequant_q4_step_sz(wq[S][j][t], gs2[j], gz2[j], nib_mask);
  };
  auto lds_wait = [](Ops& o) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(o.h[0]), "+v"(o.h[1]), "+v"(o.h[2]), "+v"(o.h[3]), "+v"(o.l[0]),
                   "+v"(o.l[1]), "+v"(o.l[2]), "+v"(o.l[3]));
  };
  Ops X, Y;
  if (n_g > 0) {
    issue(g_lo, 0, Slot<0>{});
    if (n_g > 1) issue(g_lo + 1, 1, Slot<1>{});
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();                     // group g_lo is in LDS in every wave
    group_scales(Slot<0>{});
    load_ops(X, 0, 0, Slot<0>{});
    lds_wait(X);
  }
  // k step t of group gi (buffer and B slot S = gi & 1) on `cur`, the next
  // step's operands into `nxt`; at the last step, once group gi + 1 is in LDS
  // in every wave (and every wave is done with buffer S), group gi + 2 is
  // issued into buffer and slot S
  auto kstep = [&](Ops& cur, Ops& nxt, int gi, int t, auto slot) {
    constexpr int S = decltype(slot)::value;
    bool more = true;
    if (t < 3) {
      load_ops(nxt, S, t + 1, Slot<S>{});
    } else if (gi + 1 < n_g) {
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      __syncthreads();
      if (gi + 2 < n_g) issue(g_lo + gi + 2, S, Slot<S>{});
      group_scales(Slot<S ^ 1>{});
      load_ops(nxt, S ^ 1, 0, Slot<S ^ 1>{});
    } else {
      more = false;
    }
    // the hi products of the step, then the lo ones (a tile's two MFMAs eight apart)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[i][0] = mfma_f16(cur.h[i], cur.b[0], acc[i][0]);
      acc[i][1] = mfma_f16(cur.h[i], cur.b[1], acc[i][1]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[i][0] = mfma_f16(cur.l[i], cur.b[0], acc[i][0]);
      acc[i][1] = mfma_f16(cur.l[i], cur.b[1], acc[i][1]);
    }
    if (more) lds_wait(nxt);
  };
  auto group = [&](int gi, auto slot) {
    kstep(X, Y, gi, 0, slot);
    kstep(Y, X, gi, 1, slot);
    kstep(X, Y, gi, 2, slot);
    kstep(Y, X, gi, 3, slot);
  };
  for (int gb = 0; gb < n_g; gb += 2) {
    group(gb, Slot<0>{});
    if (gb + 1 < n_g) group(gb + 1, Slot<1>{});
  }
  if (EPI == EPI_SWIGLU && tail_idx >= 0) {  // (the split last round is used for gate|up)
    // a K slice of a remaining tile: store it as 16-byte chunks (chunk c = four
    // consecutive accumulators of thread t at (c * 256 + t) * 4), and let the
    // last slice to arrive add them all in slice order, two chunks of every
    // slice in flight at a time
    constexpr int TILE = BG_WM * BG_WN;
    float* pt = tail.part + (size_t)tail_idx * tail.kt * TILE;
    f32x4* mine = (f32x4*)(pt + (size_t)ks * TILE) + threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          mine[((i * 2 + j) * 4 + q) * 256] =
              f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
    __shared__ int last_flag;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // every store of the work-group is in this XCD's L2
    if (threadIdx.x == 0)
      last_flag = __hip_atomic_fetch_add(&tail.count[tail_idx], 1, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_WORKGROUP) == tail.kt - 1;
    __syncthreads();
    if (!last_flag) return;
    const f32x4* pv = (const f32x4*)pt + threadIdx.x;
#pragma unroll
    for (int c0 = 0; c0 < 32; c0 += 2) {
      f32x4 v[2][BG_TAIL_KT_MAX];
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
#pragma unroll
        for (int k = 0; k < BG_TAIL_KT_MAX; ++k)  // every slice's chunk loaded first
          v[cc][k] = pv[(size_t)min(k, tail.kt - 1) * (TILE / 4) + (c0 + cc) * 256];
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        const int c = c0 + cc, i = c >> 3, j = (c >> 2) & 1, q = c & 3;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float sum = 0.f;
#pragma unroll
          for (int k = 0; k < BG_TAIL_KT_MAX; ++k)
            if (k < tail.kt) sum += k == ks ? acc[i][j][4 * q + e] : v[cc][k][e];
          acc[i][j][4 * q + e] = sum;
        }
      }
    }
    if (threadIdx.x == 0) tail.count[tail_idx] = 0;
  }
  __syncthreads();  // every wave's last fragment reads are done: the epilogue reuses the LDS

  // Epilogue in 32-row pieces (MFMA m-tile p of every wave) through LDS.
  float* e = (float*)smem;  // [32][BG_EROW]
  uint16_t* vbuf = (uint16_t*)(smem + BG_V_OFF);
  const int row0 = a.desc ? a.desc->row0 : 0;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int mp = m0 + 32 * p;  // forward row of local row 0
    if (mp >= M) break;          // uniform
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        e[mfma_row(r, lane) * BG_EROW + wave * 64 + j * 32 + (lane & 31)] = acc[p][j][r];
    __syncthreads();
    if (EPI == EPI_STORE) {
      float* y = a.y + (int64_t)ks * M * N;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int c = threadIdx.x + 256 * i;
        const int r = c >> 6, n = n0 + (c & 63) * 4;
        if (mp + r < M && n < N) {
          f32x4 v = *(const f32x4*)(e + r * BG_EROW + (c & 63) * 4);
          if (a.bias && ks == 0) {
#pragma unroll
            for (int k = 0; k < 4; ++k) v[k] += bf16_bits_to_float(a.bias[n + k]);
          }
          *(f32x4*)(y + (int64_t)(mp + r) * N + n) = v;
        }
      }
    } else if (EPI == EPI_SWIGLU) {
      // output chunk q: block q >> 3 of [gate 64 | up 64], 8 outputs at (q & 7) * 8;
      // ACT_F16P hi plane, then the lo plane at + M * F
      const int F = N >> 1;
      bool over = false;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int c = threadIdx.x + 256 * i;
        const int r = c >> 4, q = c & 15, blk = q >> 3, c8 = (q & 7) * 8;
        if (mp + r < M && n0 + blk * 128 < N) {
          _Float16 h[8], lo[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const float g = e[r * BG_EROW + blk * 128 + c8 + k];
            const float u = e[r * BG_EROW + blk * 128 + 64 + c8 + k];
            const float y = g * (1.f / (1.f + expf(-g))) * u;
            const _Float16 hk = (_Float16)y;
            h[f16p_index(k)] = hk;
            lo[f16p_index(k)] = f16_lo(y, hk);
            over = over || f16_overflows(y);
          }
          _Float16* dst = (_Float16*)a.act_out + (int64_t)(mp + r) * F + (n0 >> 1) + blk * 64 + c8;
          *(u32x4*)dst = __builtin_bit_cast(u32x4, h);
          *(u32x4*)(dst + (int64_t)M * F) = __builtin_bit_cast(u32x4, lo);
        }
      }
      if (over) raise_range(a);
    } else if (EPI == EPI_LMSTAT) {
      // lane: row lane & 31 of the piece, the 32 columns half of its wave's 64
      // (the rows of 8 consecutive lanes sit in 8 different 16-byte bank groups)
      const int r = lane & 31, half = lane >> 5;
      const int col0 = n0 + wave * 64 + half * 32, row = mp + r;
      const bool valid = row < M && n0 + wave * 64 < N;  // (N % 64 == 0)
      const float temperature = a.desc ? a.desc->temperature : a.lm_temp;
      const uint64_t seed = a.desc ? a.desc->seed : a.lm_seed;
      const int step = a.desc ? a.desc->step : a.lm_step;
      const int excl = a.desc ? a.desc->exclude_col : a.lm_excl;
      float v[32];
      const float* src = e + r * BG_EROW + wave * 64 + half * 32;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const f32x4 t4 = *(const f32x4*)(src + 4 * q);
#pragma unroll
        for (int k = 0; k < 4; ++k) v[4 * q + k] = t4[k];
      }
      if (a.lm_logits && valid) {
        f32x4* lp = (f32x4*)(a.lm_logits + (int64_t)row * N + col0);
#pragma unroll
        for (int q = 0; q < 8; ++q) lp[q] = f32x4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
      }
#pragma unroll
      for (int c = 0; c < 32; ++c) v[c] = col0 + c == excl ? -INFINITY : v[c];
      const bool samp = temperature > 0.f && row < M;
      const uint64_t rk = samp ? sampling_row_key(seed, step, a.lm_pos[row]) : 0ull;
      const LmRun32 mine = lm_run32(v, col0, samp, temperature, rk);
      LmRun32 other;
      other.mx = __shfl_xor(mine.mx, 32, 64);
      other.arg = __shfl_xor(mine.arg, 32, 64);
      other.se = __shfl_xor(mine.se, 32, 64);
      other.skey = __shfl_xor(mine.skey, 32, 64);
      other.sarg = __shfl_xor(mine.sarg, 32, 64);
      other.sl = __shfl_xor(mine.sl, 32, 64);
      if (half == 0 && valid)
        ((LmStat*)a.lm_stats)[(int64_t)row * (N >> 6) + (n0 >> 6) + wave] = lm_join64(mine, other);
    } else if (EPI == EPI_QKV) {
      const int rows = min(32, M - mp);
#pragma unroll
      for (int hl = 0; hl < 2; ++hl) {
        const int head = (n0 >> 7) + hl;
        if (head * 128 >= N) break;  // uniform
        if (hl) __syncthreads();     // the V tile buffer of head 0 has been copied out
        auto get = [&](int m, int d) { return e[m * BG_EROW + hl * 128 + d]; };
        const QkvTables qt = qkv_tables(a, head, row0 + mp, rows);
        if (a.kv_bf16) qkv_epilogue<__bf16>(a, qt, head, mp, row0 + mp, rows, get, vbuf);
        else qkv_epilogue<_Float16>(a, qt, head, mp, row0 + mp, rows, get, vbuf);
      }
    }
    __syncthreads();  // the piece's LDS is read before the next piece is written
  }
}

template __global__ void big_q4_kernel<EPI_STORE>(const FusedArgs, int, const BgTail);
template __global__ void big_q4_kernel<EPI_SWIGLU>(const FusedArgs, int, const BgTail);
template __global__ void big_q4_kernel<EPI_QKV>(const FusedArgs, int, const BgTail);
template __global__ void big_q4_kernel<EPI_LMSTAT>(const FusedArgs, int, const BgTail);

// The QKV epilogue of a split-K q|k|v projection: work-group (head, 32-row
// block) sums the KS fp32 partial slices of its head's 128 columns (bias
// excluded, added by the epilogue) into LDS - every slice's loads issued before
// the first add - and runs the same per-head epilogue from there.
template <typename T>
__global__ __launch_bounds__(256) void big_qkv_epilogue_kernel(const FusedArgs a,
                                                               const float* __restrict__ part,
                                                               int KS) {
  __shared__ __align__(16) float tile[32][132];
  __shared__ __align__(16) uint16_t vbuf[4096];
  const int M = a.M, N = a.N;
  const int head = blockIdx.x, mp = blockIdx.y * 32;
  const int rows = min(32, M - mp);
  const int row0 = a.desc ? a.desc->row0 : 0;
  // 32 rows x 32 float4 per slice: thread t takes rows t >> 5 + 8j, float4 t & 31
  constexpr int KMAX = drt::BG_QKV_MAX_KS;
  const QkvTables qt = qkv_tables(a, head, row0 + mp, rows);
  f32x4 v[KMAX][4];
#pragma unroll
  for (int k = 0; k < KMAX; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = min((threadIdx.x >> 5) + 8 * j, rows - 1);
      v[k][j] = *(const f32x4*)(part + (int64_t)min(k, KS - 1) * M * N + (int64_t)(mp + m) * N +
                                head * 128 + (threadIdx.x & 31) * 4);
    }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f32x4 sum = v[0][j];
#pragma unroll
    for (int k = 1; k < KMAX; ++k)
      if (k < KS) sum += v[k][j];
    *(f32x4*)&tile[(threadIdx.x >> 5) + 8 * j][(threadIdx.x & 31) * 4] = sum;
  }
  __syncthreads();
  auto get = [&](int m, int d) { return tile[m][d]; };
  qkv_epilogue<T>(a, qt, head, mp, row0 + mp, rows, get, vbuf);
}

// y = sum of the KS slices (slice order) + bias, 4 floats per thread.
__global__ __launch_bounds__(256) void sum_slices_kernel(const float* __restrict__ part, int KS,
                                                         int64_t n, const uint16_t* __restrict__ bias,
                                                         int N, float* __restrict__ y) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= n) return;
  f32x4 v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) v[k] = *(const f32x4*)(part + (int64_t)min(k, KS - 1) * n + i);
  f32x4 sum = v[0];
#pragma unroll
  for (int k = 1; k < 8; ++k)
    if (k < KS) sum += v[k];
  if (bias) {
#pragma unroll
    for (int e = 0; e < 4; ++e) sum[e] += bf16_bits_to_float(bias[(i + e) % N]);
  }
  *(f32x4*)(y + i) = sum;
}

template __global__ void big_qkv_epilogue_kernel<_Float16>(const FusedArgs, const float*, int);
template __global__ void big_qkv_epilogue_kernel<__bf16>(const FusedArgs, const float*, int);

namespace drt {

// K slices for a large-M q4 linear of M x N x K: enough work-groups for two per
// CU (the kernel's register budget), at most max_ks slices and at least 8 groups
// of 64 k per slice.
int big_linear_splits(int M, int N, int K, int max_ks) {
  const int tiles = ((M + BG_WM - 1) / BG_WM) * ((N + BG_WN - 1) / BG_WN);
  if (tiles >= 384) return 1;
  // the most slices that keep the grid within one round of two work-groups per
  // CU (512 slots on 256 CUs: a CU holding two work-groups while others hold one
  // sets the time), each slice at least 6 groups of 64 k
  int ks = std::min(max_ks, std::max(1, 512 / tiles));
  ks = std::min(ks, std::max(1, (K / 64) / 6));
  return std::max(1, ks);
}

bool big_linear_supported(const FusedArgs& a, int kind) {
  if (!a.qw || !a.sb || a.M <= 32 || a.N % 32 != 0 || a.K % 64 != 0) return false;
  if ((kind == FL_QKV || kind == FL_SWIGLU) && a.N % 128 != 0) return false;
  if (kind == FL_SWIGLU && a.act_fmt != ACT_F16P) return false;
  if (kind == FL_LMSTAT) return a.N % 64 == 0 && a.lm_stats != nullptr;
  return kind == FL_QKV || kind == FL_SWIGLU || kind == FL_STORE;
}

size_t big_tail_part_floats(int M, int N, int K, int n_cu) {
  const int tx = (N + BG_WN - 1) / BG_WN, T = tx * ((M + BG_WM - 1) / BG_WM), S = 2 * n_cu;
  if (n_cu < 1 || T <= S) return 0;
  const int full = T / S * S, rest = T - full;
  const int kt = std::min(BG_TAIL_KT_MAX, std::min(S / std::max(rest, 1), K / 64));
  if (rest % 8 || kt < 2) return 0;
  return (size_t)rest * kt * BG_WM * BG_WN;
}

void big_linear(const FusedArgs& a, int kind, int KS, hipStream_t s, float* tail_part,
                size_t tail_part_floats, int* tail_count, int n_tail_count) {
  require(big_linear_supported(a, kind), "large-M linear: unsupported shape or kind");
  require(KS >= 1 && KS <= a.K / 64 && (KS == 1 || kind == FL_STORE),
          "large-M linear: split-K only for plain stores");
  dim3 grid((a.N + BG_WN - 1) / BG_WN, (a.M + BG_WM - 1) / BG_WM, KS);
  BgTail tail;
  if (kind == FL_SWIGLU && KS == 1 && tail_part && tail_count && !a.fenced && a.n_xcc == 8) {
    // the tiles past the last whole round of two work-groups per CU, split by K
    int dev = 0, n_cu = 0;
    DRT_HIP(hipGetDevice(&dev));
    DRT_HIP(hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev));
    const size_t need = big_tail_part_floats(a.M, a.N, a.K, n_cu);
    const int T = (int)(grid.x * grid.y), S = 2 * n_cu;
    if (need && need <= tail_part_floats && T - T / S * S <= n_tail_count) {
      tail.full = T / S * S;
      tail.kt = std::min(BG_TAIL_KT_MAX, std::min(S / (T - tail.full), a.K / 64));
      tail.part = tail_part;
      tail.count = tail_count;
      grid = dim3((unsigned)(tail.full + (T - tail.full) * tail.kt), 1, 1);
    }
  }
  const double bytes = (double)a.N * a.K / 2 + (double)a.N * a.K / 16 + 2.0 * a.M * a.K +
                       (kind == FL_STORE ? 4.0 * KS : 2.0) * a.M * a.N;
#define DRT_BG(E)                                                                        \
  {                                                                                      \
    auto fn = big_q4_kernel<E>;                                                          \
    static size_t granted = 0;                                                           \
    grant_lds((const void*)fn, BG_LDS, granted);                                         \
    DRT_LAUNCH(Profiler::GEMM, bytes, fn, grid, dim3(256), BG_LDS, s, a, KS, tail);      \
  }
  if (kind == FL_QKV) DRT_BG(EPI_QKV)
  else if (kind == FL_SWIGLU) DRT_BG(EPI_SWIGLU)
  else if (kind == FL_LMSTAT) DRT_BG(EPI_LMSTAT)
  else DRT_BG(EPI_STORE)
#undef DRT_BG
  DRT_HIP(hipGetLastError());
}

void sum_slices(const float* part, int KS, int64_t n, const uint16_t* bias, int N, float* y,
                hipStream_t s) {
  require(KS >= 1 && KS <= 8 && n % 4 == 0 && N % 4 == 0, "sum_slices: 1..8 slices of n % 4 == 0");
  const int64_t blocks = (n / 4 + 255) / 256;
  hipLaunchKernelGGL(sum_slices_kernel, dim3((unsigned)blocks), dim3(256), 0, s, part, KS, n,
                     bias, N, y);
  DRT_HIP(hipGetLastError());
}

void big_qkv(const FusedArgs& a, float* part, size_t part_floats, hipStream_t s) {
  const int ks = big_linear_splits(a.M, a.N, a.K, BG_QKV_MAX_KS);
  if (ks == 1 || ks > BG_QKV_MAX_KS || !part || (size_t)ks * a.M * a.N > part_floats) {
    big_linear(a, FL_QKV, 1, s);
    return;
  }
  FusedArgs g = a;
  g.bias = nullptr;  // the epilogue adds it
  g.y = part;
  big_linear(g, FL_STORE, ks, s);
  qkv_epilogue_slices(a, part, ks, s);
}

void qkv_epilogue_slices(const FusedArgs& a, const float* part, int ks, hipStream_t s) {
  require(ks >= 1 && ks <= BG_QKV_MAX_KS && a.N % 128 == 0, "q|k|v epilogue: 1..8 slices");
  const dim3 grid(a.N / 128, (a.M + 31) / 32);
  if (a.kv_bf16)
    hipLaunchKernelGGL(big_qkv_epilogue_kernel<__bf16>, grid, dim3(256), 0, s, a, part, ks);
  else
    hipLaunchKernelGGL(big_qkv_epilogue_kernel<_Float16>, grid, dim3(256), 0, s, a, part, ks);
  DRT_HIP(hipGetLastError());
}

}  // namespace drt
