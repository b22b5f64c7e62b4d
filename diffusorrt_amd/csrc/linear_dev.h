// Device helpers shared by the linear kernels (fused_linear.hip, skinny_linear.hip).
#pragma once
#include "fused.h"

namespace {

// One 64-wide k group of one q4 n-tile with an ACT_F16P activation: a / al are
// the hi / lo fragments of this lane's row, xsr the group sums (hi + lo) of the
// 16 rows this lane holds in the MFMA result. The B operand is the exact fp16
// integer q (q4_pair_to_f16), so c = sum x q stays small (no large offset for
// the fp32 accumulation to lose bits against) and y += s * c + b * sum x.
DRT_DEV void q4_group_mma1(f32x16& acc, const f16x8 (&a)[4], const f16x8 (&al)[4],
                           const float (&xsr)[16], const u32x4 w, const uint32_t sbv) {
  f32x16 c = f32x16{};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t wt = w[t];
    u32x4 bw;
    bw[0] = q4_pair_to_f16((wt >> 0) & 0x000F000Fu);
    bw[1] = q4_pair_to_f16((wt >> 4) & 0x000F000Fu);
    bw[2] = q4_pair_to_f16((wt >> 8) & 0x000F000Fu);
    bw[3] = q4_pair_to_f16((wt >> 12) & 0x000F000Fu);
    const f16x8 b = __builtin_bit_cast(f16x8, bw);
    c = mfma_f16(a[t], b, c);
    c = mfma_f16(al[t], b, c);
  }
  const float s = bf16_bits_to_float(sbv & 0xffffu);
  const float b = bf16_bits_to_float(sbv >> 16);
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = fmaf(s, c[r], fmaf(b, xsr[r], acc[r]));
}

// q4_group_mma1 for at most 16 rows, their hi and lo halves stacked as the 32
// rows of one MFMA: a holds this lane's fragment of row lane & 31, which is hi
// row lane & 15 for lanes with bit 4 clear and its lo row otherwise, so result
// rows r and r + 16 (accumulators i and i + 8) are the hi and lo products of
// row r and half the MFMAs do the work. acc[i] (i < 8) is row mfma_row(i, lane);
// xsr the group sums (hi + lo) in accumulator order.
DRT_DEV void q4_group_mma_hl(float (&acc)[8], const f16x8 (&a)[4], const float (&xsr)[16],
                             const u32x4 w, const uint32_t sbv) {
  f32x16 c = f32x16{};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t wt = w[t];
    u32x4 bw;
    bw[0] = q4_pair_to_f16((wt >> 0) & 0x000F000Fu);
    bw[1] = q4_pair_to_f16((wt >> 4) & 0x000F000Fu);
    bw[2] = q4_pair_to_f16((wt >> 8) & 0x000F000Fu);
    bw[3] = q4_pair_to_f16((wt >> 12) & 0x000F000Fu);
    c = mfma_f16(a[t], __builtin_bit_cast(f16x8, bw), c);
  }
  const float s = bf16_bits_to_float(sbv & 0xffffu);
  const float b = bf16_bits_to_float(sbv >> 16);
#pragma unroll
  for (int r = 0; r < 8; ++r) acc[r] = fmaf(s, c[r] + c[r + 8], fmaf(b, xsr[r], acc[r]));
}

// v[l] + v[l ^ 32] on every lane (gfx950 v_permlane32_swap, no LDS trip); both
// lanes of a pair add the same two operands in the same order.
DRT_DEV float sum_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The 16 row sums a lane needs in accumulator order (rows 8j + 4(lane >> 5) + i
// for r = 4j + i) from a [32] array of row sums in LDS: four 16-byte reads.
DRT_DEV void load_row_sums(const float* rs, int lane, float (&xsr)[16]) {
  const f32x4* p = (const f32x4*)rs + (lane >> 5);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const f32x4 v = p[2 * j];
#pragma unroll
    for (int i = 0; i < 4; ++i) xsr[4 * j + i] = v[i];
  }
}

// Group sums (hi + lo) of the A fragments of UW units (lane l holds 32 of the 64
// values of row l & 31 for each unit): the lane's half-sums, the two halves
// added across lanes, staged through this wave's LDS scratch (UW x 32 floats)
// and read back in accumulator order. The wave's LDS operations run in order,
// so no barrier is needed; the scratch may be rewritten by the next call.
template <int UW>
DRT_DEV void row_sums_lane(const u32x4 (&a)[UW][4], const u32x4 (&al)[UW][4], float* scratch,
                           int lane, float (&xsr)[UW][16]) {
#pragma unroll
  for (int i = 0; i < UW; ++i) {
    float v = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const f16x8 h = __builtin_bit_cast(f16x8, a[i][t]);
      const f16x8 l = __builtin_bit_cast(f16x8, al[i][t]);
#pragma unroll
      for (int e = 0; e < 8; ++e) v += (float)h[e] + (float)l[e];
    }
    v = sum_xor32(v);
    if (lane < 32) scratch[i * 32 + lane] = v;
  }
#pragma unroll
  for (int i = 0; i < UW; ++i) load_row_sums(scratch + i * 32, lane, xsr[i]);
}

// q4_group_mma1 for one unit whose A fragments (hi, lo) came straight from
// global memory (row sums through this wave's LDS scratch of 32 floats).
DRT_DEV void q4_group_mma1_lane(f32x16& acc, const u32x4 (&a)[4], const u32x4 (&al)[4],
                                const u32x4 w, const uint32_t sbv, int lane, float* scratch) {
  const u32x4(&a1)[1][4] = reinterpret_cast<const u32x4(&)[1][4]>(a);
  const u32x4(&al1)[1][4] = reinterpret_cast<const u32x4(&)[1][4]>(al);
  float xsr[1][16];
  row_sums_lane<1>(a1, al1, scratch, lane, xsr);
  f16x8 ah[4], alh[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    ah[t] = __builtin_bit_cast(f16x8, a[t]);
    alh[t] = __builtin_bit_cast(f16x8, al[t]);
  }
  q4_group_mma1(acc, ah, alh, xsr[0], w, sbv);
}

// Records a value beyond the fp16 range in the runtime's error word.
DRT_DEV void raise_range(const FusedArgs& a) {
  if (a.placement_err)
    __hip_atomic_fetch_or(a.placement_err, DRT_ERR_F16_RANGE, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_AGENT);
}

// A value the operand type T cannot hold (fp16 only: bf16 has fp32's range).
template <typename T> DRT_DEV bool out_of_range(float x) {
  if constexpr (std::is_same<T, _Float16>::value) return f16_overflows(x);
  else return false;
}

template <typename T> DRT_DEV T cvt_to(float f);
template <> DRT_DEV _Float16 cvt_to<_Float16>(float f) { return (_Float16)f; }
template <> DRT_DEV __bf16 cvt_to<__bf16>(float f) {
  return __builtin_bit_cast(__bf16, float_to_bf16_bits(f));
}

// Epilogue of one head: x0/x1 are this lane's elements l and l + 64 of row m.
template <typename T>
DRT_DEV void qkv_head_store(const FusedArgs& a, int head, int m, int pos, float x0, float x1,
                            int lane) {
  const int Hq = a.Hq, Hkv = a.Hkv;
  const bool is_q = head < Hq, is_k = !is_q && head < Hq + Hkv;
  if (is_q || is_k) {
    const uint16_t* nw = is_q ? a.q_norm : a.k_norm;
    if (nw) {
      const float ms = wave_sum(x0 * x0 + x1 * x1) / 128.f;
      const float inv = 1.f / sqrtf(ms + a.eps);
      x0 = (x0 * inv) * bf16_bits_to_float(nw[lane]);
      x1 = (x1 * inv) * bf16_bits_to_float(nw[lane + 64]);
    }
    const float c = a.rope_cos[(int64_t)pos * 64 + lane];
    const float s = a.rope_sin[(int64_t)pos * 64 + lane];
    const float r0 = x0 * c - x1 * s;
    const float r1 = x1 * c + x0 * s;
    x0 = r0;
    x1 = r1;
  }
  if (out_of_range<T>(x0) || out_of_range<T>(x1)) raise_range(a);
  if (is_q) {
    // Q as hi / lo planes: lo at + M * Hq * 128 elements
    T* qo = (T*)a.q_out + ((int64_t)m * Hq + head) * 128;
    T* ql = qo + (int64_t)a.M * Hq * 128;
    const T h0 = cvt_to<T>(x0), h1 = cvt_to<T>(x1);
    qo[lane] = h0;
    qo[lane + 64] = h1;
    ql[lane] = lo_part<T>(x0, h0);
    ql[lane + 64] = lo_part<T>(x1, h1);
    return;
  }
  const int kvh = is_k ? head - Hq : head - Hq - Hkv;
  T* tile = (T*)a.kv_layer + (int64_t)kvh * a.kv_head_stride + (int64_t)(pos >> 5) * 8192;
  const int kk = pos & 31;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int hd = lane + 64 * e;
    const float val = e ? x1 : x0;
    if (is_k) {
      tile[(((hd >> 4) * 2 + ((hd >> 3) & 1)) * 32 + kk) * 8 + (hd & 7)] = cvt_to<T>(val);
    } else {
      const int q16 = kk & 15;
      tile[4096 + ((((hd >> 5) * 2 + (kk >> 4)) * 2 + ((q16 >> 2) & 1)) * 32 + (hd & 31)) * 8 +
           (q16 & 3) + 4 * (q16 >> 3)] = cvt_to<T>(val);
    }
  }
}

// Epilogue of one q/k/v head over 32 rows of a forward (backends/mlx_forward.py:
// 1164-1361): (+ bias), per-head RMSNorm of q/k (mlx_ops.py:21-35), split-half
// RoPE at the row's absolute position (mlx_ops.py:133-144), then Q out or K/V
// into the tiled cache. 256 threads: thread t owns local row t >> 3 and the head
// dims 8c .. 8c+7 and 64+8c .. 64+8c+7 (c = t & 7): the RoPE pairs of its dims
// are its own, the norm is a sum over 8 lanes, and every store is 16 bytes -
// except V, whose tile layout spreads a key over the tile: a whole aligned
// 32-key tile is assembled in LDS first (lds_v, 4096 elements; the call then
// holds a work-group barrier, so every thread must make it), otherwise V is
// written element-wise.
//   mrow0: forward row of local row 0 (Q rows are forward rows)
//   pos0 : absolute position of local row 0
//   rows : valid local rows (<= 32)
//   get(m, d): the linear's output (before bias) of local row m, head dim d
// The per-thread inputs of qkv_epilogue besides the linear's output: bias, q/k
// norm weights and the rotary angles of the thread's row and dims. Loaded by
// every thread without branches (absent tables read a valid stand-in and are
// not used), so a caller can issue them together with its last loads and the
// epilogue waits for no further memory round trip.
struct QkvTables {
  f32x4 c0, c1, s0, s1;  // cos / sin of angles 8c .. 8c+7
  u32x4 w0, w1;          // norm weights of dims 8c.., 64+8c.. (bf16 pairs)
  u32x4 b0, b1;          // bias of the same dims (bf16 pairs)
};
DRT_DEV QkvTables qkv_tables(const FusedArgs& a, int head, int pos0, int rows) {
  const int m = threadIdx.x >> 3, c = threadIdx.x & 7;
  const int pos_t = m < rows ? pos0 + m : pos0;  // rows past the end read a valid table row
  QkvTables t;
  // rotary tables: cos/sin [pos][64] fp32, angle i shared by dims i and i + 64
  const f32x4* cp = (const f32x4*)(a.rope_cos + (int64_t)pos_t * 64 + 8 * c);
  const f32x4* sp = (const f32x4*)(a.rope_sin + (int64_t)pos_t * 64 + 8 * c);
  t.c0 = cp[0];
  t.c1 = cp[1];
  t.s0 = sp[0];
  t.s1 = sp[1];
  const uint16_t* stand_in = (const uint16_t*)a.rope_cos;  // >= 64 floats
  const uint16_t* nw = head < a.Hq ? a.q_norm : a.k_norm;
  nw = nw ? nw : stand_in;
  t.w0 = *(const u32x4*)(nw + 8 * c);
  t.w1 = *(const u32x4*)(nw + 64 + 8 * c);
  const uint16_t* bias = a.bias ? a.bias + head * 128 : stand_in;
  t.b0 = *(const u32x4*)(bias + 8 * c);
  t.b1 = *(const u32x4*)(bias + 64 + 8 * c);
  return t;
}

// Sum over the 8 lanes of an aligned 8-lane group, with DPP moves (no LDS):
// two quad swaps, then the half-row mirror pairs quad 0 with quad 1.
DRT_DEV float sum8_dpp(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  return v;
}

template <typename T, typename Get>
DRT_DEV void qkv_epilogue(const FusedArgs& a, const QkvTables& t, int head, int mrow0, int pos0,
                          int rows, Get get, uint16_t* lds_v) {
  const int Hq = a.Hq, Hkv = a.Hkv;
  const int m = threadIdx.x >> 3, c = threadIdx.x & 7;
  const bool is_q = head < Hq, is_k = !is_q && head < Hq + Hkv, is_v = !is_q && !is_k;
  const int pos = pos0 + m;
  float x[8], y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    x[e] = get(m, 8 * c + e);
    y[e] = get(m, 64 + 8 * c + e);
  }
  if (a.bias) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] += bf16_bits_to_float(t.b0[e] & 0xffffu);
      x[2 * e + 1] += bf16_bits_to_float(t.b0[e] >> 16);
      y[2 * e] += bf16_bits_to_float(t.b1[e] & 0xffffu);
      y[2 * e + 1] += bf16_bits_to_float(t.b1[e] >> 16);
    }
  }
  if (!is_v) {
    const f32x4 c0 = t.c0, c1 = t.c1, s0 = t.s0, s1 = t.s1;
    if (is_q ? a.q_norm : a.k_norm) {
      const u32x4 w0 = t.w0, w1 = t.w1;
      float q = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) q += x[e] * x[e] + y[e] * y[e];
      q = sum8_dpp(q);
      const float inv = 1.f / sqrtf(q / 128.f + a.eps);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[2 * e] = (x[2 * e] * inv) * bf16_bits_to_float(w0[e] & 0xffffu);
        x[2 * e + 1] = (x[2 * e + 1] * inv) * bf16_bits_to_float(w0[e] >> 16);
        y[2 * e] = (y[2 * e] * inv) * bf16_bits_to_float(w1[e] & 0xffffu);
        y[2 * e + 1] = (y[2 * e + 1] * inv) * bf16_bits_to_float(w1[e] >> 16);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float cs = e < 4 ? c0[e] : c1[e - 4], sn = e < 4 ? s0[e] : s1[e - 4];
      const float r0 = x[e] * cs - y[e] * sn;
      const float r1 = y[e] * cs + x[e] * sn;
      x[e] = r0;
      y[e] = r1;
    }
  }
  T hx[8], hy[8];
  bool over = false;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    hx[e] = cvt_to<T>(x[e]);
    hy[e] = cvt_to<T>(y[e]);
    over = over || out_of_range<T>(x[e]) || out_of_range<T>(y[e]);
  }
  if (over && m < rows) raise_range(a);
  if (is_q) {
    if (m < rows) {
      // Q as hi / lo planes: lo at + M * Hq * 128 elements
      T* qo = (T*)a.q_out + ((int64_t)(mrow0 + m) * Hq + head) * 128 + 8 * c;
      T* ql = qo + (int64_t)a.M * Hq * 128;
      T lx[8], ly[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        lx[e] = lo_part<T>(x[e], hx[e]);
        ly[e] = lo_part<T>(y[e], hy[e]);
      }
      *(u32x4*)qo = __builtin_bit_cast(u32x4, hx);
      *(u32x4*)(qo + 64) = __builtin_bit_cast(u32x4, hy);
      *(u32x4*)ql = __builtin_bit_cast(u32x4, lx);
      *(u32x4*)(ql + 64) = __builtin_bit_cast(u32x4, ly);
    }
    return;
  }
  const int kvh = is_k ? head - Hq : head - Hq - Hkv;
  if (is_k) {
    if (m < rows) {
      // K[kk][hd] at ((hd/16*2 + (hd/8)&1)*32 + kk)*8 + hd%8: dims 8c.. are chunk c
      T* tile = (T*)a.kv_layer + (int64_t)kvh * a.kv_head_stride + (int64_t)(pos >> 5) * 8192;
      const int kk = pos & 31;
      *(u32x4*)(tile + (c * 32 + kk) * 8) = __builtin_bit_cast(u32x4, hx);
      *(u32x4*)(tile + ((8 + c) * 32 + kk) * 8) = __builtin_bit_cast(u32x4, hy);
    }
    return;
  }
  // V[kk][hd] at 4096 + ((((hd/32)*2 + kk/16)*2 + h)*32 + hd%32)*8 + j with
  // q = kk%16, h = (q/4)&1, j = q%4 + 4*(q/8)
  auto v_off = [](int hd, int kk) {
    const int q16 = kk & 15;
    return 4096 + ((((hd >> 5) * 2 + (kk >> 4)) * 2 + ((q16 >> 2) & 1)) * 32 + (hd & 31)) * 8 +
           (q16 & 3) + 4 * (q16 >> 3);
  };
  T* tile = (T*)a.kv_layer + (int64_t)kvh * a.kv_head_stride + (int64_t)(pos0 >> 5) * 8192;
  if (rows == 32 && (pos0 & 31) == 0) {
    T* vs = (T*)lds_v;  // the V half of the tile, [4096]
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      vs[v_off(8 * c + e, m) - 4096] = hx[e];
      vs[v_off(64 + 8 * c + e, m) - 4096] = hy[e];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int ch = threadIdx.x + 256 * i;  // 16-byte chunk of the 8 KiB half
      *(u32x4*)(tile + 4096 + ch * 8) = *(const u32x4*)(vs + ch * 8);
    }
  } else if (m < rows) {
    T* vt = (T*)a.kv_layer + (int64_t)kvh * a.kv_head_stride + (int64_t)(pos >> 5) * 8192;
    const int kk = pos & 31;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      vt[v_off(8 * c + e, kk)] = hx[e];
      vt[v_off(64 + 8 * c + e, kk)] = hy[e];
    }
  }
  (void)tile;
}

}  // namespace
