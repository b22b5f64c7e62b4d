// Block-over-prefix GQA attention for gfx950 (flash-decode over key splits).
//
// Queries of one KV head are flattened to query vectors qv = row * G + gi
// (G = Hq / Hkv, head = kvh * G + gi) and processed in 32-vector tiles, one
// tile per wave. Keys come in 32-key tiles staged through LDS (double
// buffered) and shared by the QW waves of a work-group.
//
// Per 32x32 tile the wave computes S^T = K Q^T (8 MFMAs over head_dim 128), so
// lane l owns query (l & 31) and 16 of its 32 keys; the partner lane l ^ 32
// owns the other 16. Online softmax keeps (m, l) per lane; one xor-32 exchange
// gives the tile max, and the partial sums are only joined at the end. P^T then
// feeds the B operand of O^T += V^T P^T (8 MFMAs) directly from registers.
//
// KV cache tile layout (T = _Float16 or __bf16), per (layer, kv head, tile of 32
// keys) a contiguous 16 KiB: K block (4096 elements) then V block (4096):
//   K[key kk][hd]: ((t*2 + h)*32 + kk)*8 + e        t = hd/16, h = (hd/8)&1, e = hd&7
//   V[key kk][hd]: (((hb*2 + kh)*2 + h)*32 + hl)*8 + j
//       hb = hd/32, hl = hd&31, kh = kk/16, q = kk&15, h = (q>>2)&1, j = (q&3) + 4*(q>>3)
// so that every MFMA operand a wave reads is one contiguous 1 KiB of LDS.
//
// Masks: kind 0 = none (bidirectional, or a block whose keys are all visible);
// kind 1 = d2f_hybrid: eff(p) = p < prompt_len ? -1 : (p - prompt_len) / block,
// key visible iff eff(key) <= eff(query position).
#include "common.h"
#include "launch.h"

namespace {

template <typename T> struct MfmaT;
template <> struct MfmaT<_Float16> {
  typedef f16x8 vec;
  static DRT_DEV f32x16 mma(vec a, vec b, f32x16 c) { return mfma_f16(a, b, c); }
  static DRT_DEV _Float16 from_float(float f) { return (_Float16)f; }
};
template <> struct MfmaT<__bf16> {
  typedef bf16x8 vec;
  static DRT_DEV f32x16 mma(vec a, vec b, f32x16 c) { return mfma_bf16(a, b, c); }
  static DRT_DEV __bf16 from_float(float f) {
    return __builtin_bit_cast(__bf16, float_to_bf16_bits(f));
  }
};

DRT_DEV int eff_block(int p, int prompt_len, int block) {
  return p < prompt_len ? -1 : (p - prompt_len) / block;
}

}  // namespace

constexpr int KV_TILE_ELEMS = 8192;  // K block + V block per 32-key tile

// Softmax bookkeeping of both attention kernels runs in base 2 on scaled scores:
// u = s * scale * log2(e), p = 2^(u - base). The base of a query vector is only
// raised when a tile's max exceeds it by more than DEC_RESCALE_LOG2 (or on its
// first visible keys), so p <= 2^DEC_RESCALE_LOG2 (exact in the MFMA operand
// types' range) and the rescale of O, which moves the accumulators through
// VGPRs, is rare instead of once per tile. Any base gives the same o / l.
constexpr float DEC_RESCALE_LOG2 = 8.f;

// max(v[l], v[l ^ 32]) on every lane (gfx950 v_permlane32_swap, no LDS trip).
DRT_DEV float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}


template <typename T, int QW>
__global__ __launch_bounds__(64 * QW) void attn_split_kernel(
    const T* __restrict__ q,       // [n_rows][Hq][128]
    const T* __restrict__ q_lo,    // its lo plane (the same layout), or null (zero)
    const T* __restrict__ kv,      // this layer: [Hkv][tile_cap][8192]
    int64_t kv_head_stride,        // elements between kv heads
    int n_rows, int Hq, int Hkv, int n_keys, int row_pos0,
    int mask_kind, int mask_prompt_len, int mask_block, int tiles_per_split,
    float* __restrict__ o_part,    // [splits][Hkv][n_qv][128]
    float* __restrict__ ml_part,   // [splits][Hkv][n_qv][2]
    float scale) {
  typedef typename MfmaT<T>::vec vec;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int G = Hq / Hkv;
  const int n_qv = n_rows * G;
  const int n_splits = gridDim.x / Hkv;
  const int split = blockIdx.x / Hkv;
  const int kvh = blockIdx.x - split * Hkv;
  const int qt = blockIdx.y * QW + wave;
  const int n_tiles = (n_keys + 31) >> 5;
  const int t_begin = split * tiles_per_split;
  const int t_end = min(n_tiles, t_begin + tiles_per_split);

  extern __shared__ __align__(16) char smem[];
  T* lds = (T*)smem;  // [2][8192]

  // This lane's query (B operand of S^T) and its absolute position.
  const int qv = qt * 32 + (lane & 31);
  const bool q_ok = qv < n_qv;
  const int qrow = q_ok ? qv / G : 0;
  const int qhead = kvh * G + (q_ok ? qv - (qv / G) * G : 0);
  vec qf[8], qfl[8];  // Q hi / lo planes
  {
    const int64_t qo = ((int64_t)qrow * Hq + qhead) * 128 + 8 * (lane >> 5);
    const T* qp = q + qo;
    const T* qpl = (q_lo ? q_lo : q) + qo;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (q_ok) {
        qf[i] = *(const vec*)(qp + 16 * i);
        qfl[i] = *(const vec*)(qpl + 16 * i);
        if (!q_lo) qfl[i] = vec{};
      } else {
        qf[i] = qfl[i] = vec{};
      }
    }
  }
  const int qpos = row_pos0 + qrow;
  const float c = scale * 1.44269504088896340736f;  // scores to base-2 exponents
  // d2f_hybrid: a query sees exactly the keys before the end of its own block
  // (the whole prompt, then whole blocks up to its own), so visibility is one
  // compare per key against q_key_end
  int q_key_end = n_keys;
  if (mask_kind == 1) {
    const int e = eff_block(qpos, mask_prompt_len, mask_block);
    q_key_end = min(n_keys, e < 0 ? mask_prompt_len : mask_prompt_len + (e + 1) * mask_block);
  }
  // Wave-uniform visibility bound: no key beyond the last visible key of the
  // wave's rows needs loading into this wave's math.
  int wave_key_end = n_keys;
  if (mask_kind == 1) {
    const int last_row = min(n_rows - 1, (qt * 32 + 31) / G);
    const int e = eff_block(row_pos0 + last_row, mask_prompt_len, mask_block);
    wave_key_end = min(n_keys, e < 0 ? mask_prompt_len : mask_prompt_len + (e + 1) * mask_block);
  }
  // WG-uniform bound (the last wave's rows are the latest).
  int wg_key_end = n_keys;
  if (mask_kind == 1) {
    const int last_row = min(n_rows - 1, (blockIdx.y * QW * 32 + QW * 32 - 1) / G);
    const int e = eff_block(row_pos0 + last_row, mask_prompt_len, mask_block);
    wg_key_end = min(n_keys, e < 0 ? mask_prompt_len : mask_prompt_len + (e + 1) * mask_block);
  }
  const int t_stop = min(t_end, (wg_key_end + 31) >> 5);

  float m_run = -INFINITY, l_run = 0.f;
  f32x16 o[4];
#pragma unroll
  for (int hb = 0; hb < 4; ++hb) o[hb] = f32x16{};

  const T* kvh_base = kv + (int64_t)kvh * kv_head_stride;
  constexpr int VEC_PER_TILE = KV_TILE_ELEMS / 8;  // 16-byte vectors per tile
  constexpr int PER_THREAD = VEC_PER_TILE / (64 * QW);
  // K/V tiles go global -> registers -> LDS (double buffered), loaded two tiles
  // ahead through two register stages (tile t + 2 is in flight while tile t is
  // computed and tile t + 1 is stored), so a tile's memory latency overlaps two
  // iterations' work instead of one.
  u32x4 stage_a[PER_THREAD], stage_b[PER_THREAD];
  auto load_tile = [&](u32x4 (&st)[PER_THREAD], int t) {
    const u32x4* src = (const u32x4*)(kvh_base + (int64_t)t * KV_TILE_ELEMS);
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) st[i] = src[threadIdx.x + i * 64 * QW];
  };
  auto store_tile = [&](const u32x4 (&st)[PER_THREAD], int buf) {
    u32x4* dst = (u32x4*)(lds + buf * KV_TILE_ELEMS);
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) dst[threadIdx.x + i * 64 * QW] = st[i];
  };
  auto compute = [&](int t, int buf) {
    const int key0 = t * 32;
    if (key0 < wave_key_end) {
      const T* kt = lds + buf * KV_TILE_ELEMS;
      const T* vt = kt + 4096;
      f32x16 s = f32x16{};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const vec kf = *(const vec*)(kt + (i * 64 + lane) * 8);
        s = MfmaT<T>::mma(kf, qf[i], s);
        s = MfmaT<T>::mma(kf, qfl[i], s);
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] = key0 + mfma_row(r, lane) < q_key_end ? s[r] * c : -INFINITY;
        tmax = fmaxf(tmax, s[r]);
      }
      tmax = max_xor32(tmax);  // -inf: no visible key in the tile
      const bool up = tmax > m_run + DEC_RESCALE_LOG2;
      if (__ballot(up)) {  // some base has to rise (rare after the first tiles)
        const float alpha = up ? __builtin_amdgcn_exp2f(m_run - tmax) : 1.f;  // 0 from -inf
        if (__ballot(up && m_run != -INFINITY)) {
#pragma unroll
          for (int hb = 0; hb < 4; ++hb) o[hb] *= alpha;
        }
        l_run *= alpha;
        m_run = up ? tmax : m_run;
      }
      const float base = m_run == -INFINITY ? 0.f : m_run;  // no key yet: p = 0
      float psum = 0.f;
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p[r] = __builtin_amdgcn_exp2f(s[r] - base);
        psum += p[r];
      }
      l_run += psum;
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        vec pf;
#pragma unroll
        for (int j = 0; j < 8; ++j) pf[j] = MfmaT<T>::from_float(p[kh * 8 + j]);
#pragma unroll
        for (int hb = 0; hb < 4; ++hb) {
          const vec vf = *(const vec*)(vt + (((hb * 2 + kh) * 64) + lane) * 8);
          o[hb] = MfmaT<T>::mma(vf, pf, o[hb]);
        }
      }
    }
  };

  if (t_begin < t_stop) {
    load_tile(stage_a, t_begin);
    store_tile(stage_a, 0);
  }
  if (t_begin + 1 < t_stop) load_tile(stage_b, t_begin + 1);
  __syncthreads();
  // two tiles per pass: buffer 0 / stage_a for tiles t_begin + 2k, buffer 1 /
  // stage_b for tiles t_begin + 2k + 1. A buffer is rewritten only after the
  // barrier that follows its last read.
  for (int t = t_begin; t < t_stop; t += 2) {
    if (t + 2 < t_stop) load_tile(stage_a, t + 2);
    compute(t, 0);
    if (t + 1 >= t_stop) break;
    store_tile(stage_b, 1);
    __syncthreads();
    if (t + 3 < t_stop) load_tile(stage_b, t + 3);
    compute(t + 1, 1);
    if (t + 2 >= t_stop) break;
    store_tile(stage_a, 0);
    __syncthreads();
  }
  l_run += __shfl_xor(l_run, 32, 64);

  // Transpose O^T through LDS so each query's 128 values are written contiguously.
  __syncthreads();
  float* ot = (float*)smem + wave * (32 * 132);
#pragma unroll
  for (int hb = 0; hb < 4; ++hb)
#pragma unroll
    for (int r = 0; r < 16; ++r) ot[(lane & 31) * 132 + hb * 32 + mfma_row(r, lane)] = o[hb][r];
  __syncthreads();
  const int64_t part_base = ((int64_t)split * Hkv + kvh) * n_qv;
  for (int i = lane; i < 32 * 32; i += 64) {
    const int qq = i >> 5, c4 = (i & 31) * 4;
    const int qv2 = qt * 32 + qq;
    if (qv2 < n_qv) {
      f32x4 v = {ot[qq * 132 + c4], ot[qq * 132 + c4 + 1], ot[qq * 132 + c4 + 2],
                 ot[qq * 132 + c4 + 3]};
      *(f32x4*)(o_part + (part_base + qv2) * 128 + c4) = v;
    }
  }
  if (lane < 32 && q_ok) {
    ml_part[(part_base + qv) * 2 + 0] = m_run;
    ml_part[(part_base + qv) * 2 + 1] = l_run;
  }
  (void)n_splits;
}

// Decode attention: rows of one mask segment (every key in [0, n_keys) is
// visible to every row) with at most 32*QT query vectors per KV head
// (attn_decode_kernel below). Grid (Hkv, R ranges), one work-group per CU (the
// host keeps R * Hkv <= 256): range r owns the tiles [n_tiles*r/R,
// n_tiles*(r+1)/R) of its KV head and writes one partial (m, l, O) in the MFMA
// register order ("slot" order, see attn_decode_combine_kernel) with coalesced
// stores; empty ranges write only m = -inf, l = 0, and the combine then skips
// their O. n_keys comes from `desc` when it is set (graph replays), else from
// the argument.
constexpr int DEC_QROW = 136;  // 16-bit elements per Q row in LDS (+16 B pad)
// elements from the Q hi plane to the lo plane in LDS (64 rows of hi plane up to
// two query tiles, 128 for four)
template <int QT> constexpr int dec_qlo() { return (QT <= 2 ? 64 : 32 * QT) * DEC_QROW; }
constexpr int DEC_QLO = dec_qlo<2>();

// The second half of a key group: keys at or beyond nk[g] masked, one max over
// the group, softmax weights against the running base, O^T += V^T P^T.
template <typename T, int QT, int NG>
DRT_DEV void softmax_pv(f32x16 (&sc)[NG][QT], const typename MfmaT<T>::vec (&vc)[NG][8],
                        const int (&key0)[NG], const int (&nk)[NG], float c, int lane,
                        float (&m_run)[QT], float (&l_run)[QT], f32x16 (&o)[QT][4]) {
  typedef typename MfmaT<T>::vec vec;
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    if (key0[g] + 32 > nk[g]) {  // uniform: a partial (or empty) tile masks its keys
#pragma unroll
      for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          sc[g][qt][r] = key0[g] + mfma_row(r, lane) < nk[g] ? sc[g][qt][r] : -INFINITY;
    }
  }
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    float tmax = sc[0][qt][0];
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, sc[g][qt][r]);
    const float mc = max_xor32(tmax) * c;  // -inf: no visible key in the group
    const bool up = mc > m_run[qt] + DEC_RESCALE_LOG2;
    if (__ballot(up)) {  // uniform: some base has to rise
      const float alpha = up ? __builtin_amdgcn_exp2f(m_run[qt] - mc) : 1.f;  // 0 from -inf
      if (__ballot(up && m_run[qt] != -INFINITY)) {  // O is still zero before the first key
#pragma unroll
        for (int hb = 0; hb < 4; ++hb) o[qt][hb] *= alpha;
      }
      l_run[qt] *= alpha;
      m_run[qt] = up ? mc : m_run[qt];
    }
  }
#pragma unroll
  for (int g = 0; g < NG; ++g)
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const float base = m_run[qt] == -INFINITY ? 0.f : m_run[qt];  // no key yet: p = 0
      float pr[16];
      float psum = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        pr[r] = __builtin_amdgcn_exp2f(fmaf(sc[g][qt][r], c, -base));
        psum += pr[r];
      }
      l_run[qt] += psum;
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        vec pf;
#pragma unroll
        for (int j = 0; j < 8; ++j) pf[j] = MfmaT<T>::from_float(pr[kh * 8 + j]);
#pragma unroll
        for (int hb = 0; hb < 4; ++hb)
          o[qt][hb] = MfmaT<T>::mma(vc[g][hb * 2 + kh], pf, o[qt][hb]);
      }
    }
}

// One 32-key tile for one query tile whose Q fragments the wave holds in
// registers (qh / ql: hi and lo planes, k-step i = head dims 16 i + 8 (lane >> 5)
// .. + 8 of query vector lane & 31): S^T = K Q^T as one MFMA chain per plane,
// then softmax_pv.
template <typename T>
DRT_DEV void attend_tile_rq(const typename MfmaT<T>::vec (&kc)[1][8],
                            const typename MfmaT<T>::vec (&vc)[1][8],
                            const typename MfmaT<T>::vec (&qh)[8],
                            const typename MfmaT<T>::vec (&ql)[8], int key0, int nk, float c,
                            int lane, float (&m_run)[1], float (&l_run)[1], f32x16 (&o)[1][4]) {
  f32x16 sc[1][1] = {{f32x16{}}};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    sc[0][0] = MfmaT<T>::mma(kc[0][i], qh[i], sc[0][0]);
    sc[0][0] = MfmaT<T>::mma(kc[0][i], ql[i], sc[0][0]);
  }
  const int k0[1] = {key0}, nk1[1] = {nk};
  softmax_pv<T, 1, 1>(sc, vc, k0, nk1, c, lane, m_run, l_run, o);
}

// attn_decode_kernel, the producer / consumer form. With every wave loading its
// own tiles a wave cannot compute while its loads wait to issue (the memory
// system paces them), so the compute would start only once the range had nearly
// streamed. Here five waves split the roles: wave 4 streams the range's 16 KiB K/V tiles
// with direct-to-LDS loads (global_load_lds, no registers held) into a ring of
// DECR_SLOTS tile slots, and after each s_waitcnt that proves a tile complete
// writes the tile's number (+1) into the slot's ready flag; waves 0-3 take tiles
// t = wave, wave + 4, ... as their flags appear, so the tiles are computed while
// the rest of the range is still streaming, and release each slot (freed flag)
// after reading it into registers. Every wait on a flag is bounded: a wait that
// runs out sets *err (the host reports it) and the kernel still finishes.
// Tile slots of the ring: as many as the LDS left by the Q planes holds (160
// KiB per work-group): 8 for 32 query vectors, 7 for 64, 5 for 128.
template <int QT> constexpr int decr_slots() { return QT == 1 ? 8 : (QT == 2 ? 7 : 5); }
// Consumer waves: 4, or 8 for four query tiles, whose 128 query vectors would
// otherwise give each consumer wave every tile of the range (the kernel then ran
// on the consumers' MFMA and softmax work, not on the stream). With 8 consumers
// three waves share a SIMD, so their Q fragments are read from LDS per tile
// instead of being held in registers for the whole range.
template <int QT> constexpr int decr_ncw() { return QT == 4 ? 8 : 4; }
constexpr int DECR_SPIN = 1 << 22;
// s_waitcnt immediates (gfx9: vmcnt bits 3:0 + 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr int DECR_VM48 = 0xCF70, DECR_VM32 = 0x8F70, DECR_VM16 = 0x4F70, DECR_VM0 = 0x0F70;
constexpr int DECR_LGKM0 = 0xC07F;
// cache policy of the tile loads: nontemporal (the K/V stream is read once per
// step; cached, it evicts the weights the linears find in the memory-side cache)
constexpr int DECR_NT = 2;

// s_waitcnt that the compiler may not move memory operations across
template <int IMM> DRT_DEV void decr_waitcnt() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(IMM);
  asm volatile("" ::: "memory");
}

// The flags are read and written with inline ds_read / ds_write: the compiler
// would otherwise put an s_waitcnt vmcnt(0) before every LDS access that follows
// a direct-to-LDS load (it cannot tell the flags from the tile slots), which
// would make the producer wait for every tile in flight before each signal.
DRT_DEV int decr_lds_read(const int* p) {
  int v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)"
               : "=v"(v)
               : "v"((uint32_t)(uintptr_t)p)
               : "memory");
  return v;
}
DRT_DEV void decr_lds_write(int* p, int v) {
  asm volatile("ds_write_b32 %0, %1" : : "v"((uint32_t)(uintptr_t)p), "v"(v) : "memory");
}

// LDS accesses after the wait stay after it (compiler barrier; one wave's LDS
// operations execute in order).
DRT_DEV bool decr_wait(const int* flag, int want, int* err) {
  bool ok = false;
  for (int it = 0; it < DECR_SPIN && !ok; ++it) {
    ok = decr_lds_read(flag) == want;
    if (!ok) __builtin_amdgcn_s_sleep(1);
  }
  if (!ok && err && (threadIdx.x & 63) == 0) atomicOr(err, 2);
  asm volatile("" ::: "memory");
  return ok;
}

template <typename T, int QT>
__global__ __launch_bounds__(64 * (decr_ncw<QT>() + 1)) void attn_decode_kernel(
    const T* __restrict__ q, const T* __restrict__ q_lo, const T* __restrict__ kv,
    int64_t kv_head_stride, int n_rows,
    int Hq, int Hkv, int n_keys_arg, const StepDesc* __restrict__ desc,
    float* __restrict__ o_part, float* __restrict__ ml_part, float scale, int* err) {
  typedef typename MfmaT<T>::vec vec;
  constexpr int DECR_SLOTS = decr_slots<QT>();
  constexpr int QLO = dec_qlo<QT>();
  constexpr int SLOTS = QT * 4096;
  constexpr int SLOT = SLOTS + QT * 64 * 2;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = Hq / Hkv;
  const int n_qv = n_rows * G;
  const int R = gridDim.y, rg = blockIdx.y, kvh = blockIdx.x;
  const int n_keys = desc ? desc->n_keys : n_keys_arg;
  const float c = scale * 1.44269504088896340736f;
  const int n_tiles = (n_keys + 31) >> 5;
  const int t_begin = (int)((int64_t)n_tiles * rg / R);
  const int t_end = (int)((int64_t)n_tiles * (rg + 1) / R);
  const int n = t_end - t_begin;
  const int64_t part = (int64_t)rg * Hkv + kvh;
  extern __shared__ __align__(16) char smem[];
  int* ready = (int*)smem;                               // [DECR_SLOTS]
  int* freed = ready + DECR_SLOTS;                       // [DECR_SLOTS]
  T* qs = (T*)(smem + 128);  // [QT*32][DEC_QROW] hi, lo plane at + QLO
  char* tiles = smem + 128 + (QLO + QT * 32 * DEC_QROW) * 2;  // [DECR_SLOTS][16 KiB]
  float* mrg = (float*)(smem + 128);                     // [4][SLOT], over Q and the tiles

  if (n <= 0) {
    if (threadIdx.x < QT * 32) {
      ml_part[(part * (QT * 32) + threadIdx.x) * 2] = -INFINITY;
      ml_part[(part * (QT * 32) + threadIdx.x) * 2 + 1] = 0.f;
    }
    return;
  }
  const T* base = kv + (int64_t)kvh * kv_head_stride + (int64_t)t_begin * KV_TILE_ELEMS;
  // tile t of the range into its slot: 16 wave-wide 1 KiB loads, LDS image = HBM image
  auto dma_tile = [&](int t) {
    const u32x4* src = (const u32x4*)(base + (int64_t)t * KV_TILE_ELEMS) + lane;
    char* dst = tiles + (t % DECR_SLOTS) * 16384;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)(src + i * 64),
                                       (__attribute__((address_space(3))) void*)(dst + i * 1024),
                                       16, 0, DECR_NT);
  };
  auto signal = [&](int t) {  // tile t's loads are complete
    asm volatile("" ::: "memory");
    decr_lds_write(&ready[t % DECR_SLOTS], t + 1);  // every lane writes the same value
  };

  constexpr int NCW = decr_ncw<QT>(), CT = 64 * NCW;  // consumer waves and threads
  constexpr int QCH = QT * 512 / CT;                   // Q chunks per consumer thread
  if (wave == NCW) {
    const int n0 = min(n, 2);
    for (int t = 0; t < n0; ++t) dma_tile(t);
  } else {
    const T* ql = q_lo ? q_lo : q;  // the Q lo plane (null: zero)
    u32x4 qraw[QCH], qrawl[QCH];
#pragma unroll
    for (int i = 0; i < QCH; ++i) {
      const int ch = threadIdx.x + CT * i;
      const int qvc = min(ch >> 4, n_qv - 1);
      const int row = qvc / G, head = kvh * G + (qvc - row * G);
      const int64_t off = ((int64_t)row * Hq + head) * 128 + (ch & 15) * 8;
      qraw[i] = *(const u32x4*)(q + off);
      qrawl[i] = *(const u32x4*)(ql + off);
    }
    if (threadIdx.x < 2 * DECR_SLOTS) ready[threadIdx.x] = 0;  // ready and freed
#pragma unroll
    for (int i = 0; i < QCH; ++i) {
      const int ch = threadIdx.x + CT * i;
      const bool ok = (ch >> 4) < n_qv;
      T* d = qs + (ch >> 4) * DEC_QROW + (ch & 15) * 8;
      *(u32x4*)d = ok ? qraw[i] : u32x4{0u, 0u, 0u, 0u};
      *(u32x4*)(d + QLO) = ok && q_lo ? qrawl[i] : u32x4{0u, 0u, 0u, 0u};
    }
    decr_waitcnt<DECR_LGKM0>();  // Q and the flags are written
  }
  // Q in LDS, flags zero. A bare s_barrier: __syncthreads() would first wait for
  // the producer's four tiles in flight.
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // Consumer waves split each tile by query tile: wave w takes query tile
  // w % QT of tiles w / QT, w / QT + NCW / QT, ..., so a tile's work is spread
  // over QT waves (a shorter dependency chain per tile) and the merge adds
  // NCW / QT partials per query tile.
  constexpr int TSTRIDE = NCW / QT;
  constexpr int SLOT1 = 4096 + 64 * 2;  // one wave's merge slot: O of one query tile + (m, l)
  const int my_qt = wave % QT, phase = wave / QT;
  // a first mask segment (desc->seg_rows rows, a whole number of query tiles)
  // sees only the keys before its end
  const int seg = desc ? desc->seg_rows : 0;
  const int nk_mine = seg > 0 && my_qt * 32 < seg * G ? desc->row0 + seg : n_keys;
  float m_run[1] = {-INFINITY}, l_run[1] = {0.f};
  f32x16 o[1][4];
#pragma unroll
  for (int hb = 0; hb < 4; ++hb) o[0][hb] = f32x16{};
  if (wave == NCW) {
    // Tiles 0 and 1 were issued before the barrier. The first two tiles are
    // proven with two newer tiles in flight (vmcnt(32) after issuing tiles 2, 3),
    // so the consumers start as soon as tile 0 lands; tile 4 then goes out
    // unproven and from tile 5 on each issue is followed by vmcnt(48), proving
    // tile t - 3 with three newer tiles in flight. Slot t % DECR_SLOTS is free
    // once its previous tile has been read by QT waves.
    int next = 0;  // the next tile to signal
    for (int t = 2; t < n; ++t) {
      if (t >= DECR_SLOTS) decr_wait(&freed[t % DECR_SLOTS], QT * (t / DECR_SLOTS), err);
      dma_tile(t);
      if (t < 4) {
        decr_waitcnt<DECR_VM32>();
        signal(next++);
      } else if (t > 4) {
        decr_waitcnt<DECR_VM48>();
        signal(next++);
      }
    }
    // the n - next tiles still unproven (<= 3) are the last ones issued
    if (n - next == 3) {
      decr_waitcnt<DECR_VM32>();
      signal(next++);
    }
    if (n - next == 2) {
      decr_waitcnt<DECR_VM16>();
      signal(next++);
    }
    decr_waitcnt<DECR_VM0>();
    while (next < n) signal(next++);
  } else {
    const T* qrow = qs + (my_qt * 32 + (lane & 31)) * DEC_QROW + 8 * (lane >> 5);
    auto release = [&](int t) {  // the producer reuses the slot for tile t + DECR_SLOTS
      if (t + DECR_SLOTS < n) {
        decr_waitcnt<DECR_LGKM0>();  // the slot's reads are complete
        if (lane == 0)
          asm volatile("ds_add_u32 %0, %1"
                       :
                       : "v"((uint32_t)(uintptr_t)&freed[t % DECR_SLOTS]), "v"(1)
                       : "memory");
      }
    };
    if (NCW == 4) {
      // the query tile's Q fragments, read from LDS once for the whole range
      typename MfmaT<T>::vec qh[8], ql[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        qh[i] = *(const vec*)(qrow + 16 * i);
        ql[i] = *(const vec*)(qrow + QLO + 16 * i);
      }
      for (int t = phase; t < n; t += TSTRIDE) {
        decr_wait(&ready[t % DECR_SLOTS], t + 1, err);
        const vec* tp = (const vec*)(tiles + (t % DECR_SLOTS) * 16384);
        vec kc[1][8], vc[1][8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          kc[0][i] = tp[i * 64 + lane];
          vc[0][i] = tp[512 + i * 64 + lane];
        }
        release(t);
        attend_tile_rq<T>(kc, vc, qh, ql, (t_begin + t) * 32, nk_mine, c, lane, m_run, l_run, o);
      }
    } else {
      // three waves share a SIMD: K, then the score chain with the Q fragments
      // read from LDS a k step at a time, then V (the slot is released after V)
      for (int t = phase; t < n; t += TSTRIDE) {
        decr_wait(&ready[t % DECR_SLOTS], t + 1, err);
        const vec* tp = (const vec*)(tiles + (t % DECR_SLOTS) * 16384);
        vec kc[8], vc[1][8];
#pragma unroll
        for (int i = 0; i < 8; ++i) kc[i] = tp[i * 64 + lane];
        f32x16 sc[1][1] = {{f32x16{}}};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const vec qh = *(const vec*)(qrow + 16 * i), ql = *(const vec*)(qrow + QLO + 16 * i);
          sc[0][0] = MfmaT<T>::mma(kc[i], qh, sc[0][0]);
          sc[0][0] = MfmaT<T>::mma(kc[i], ql, sc[0][0]);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) vc[0][i] = tp[512 + i * 64 + lane];
        release(t);
        const int k0[1] = {(t_begin + t) * 32}, nk1[1] = {nk_mine};
        softmax_pv<T, 1, 1>(sc, vc, k0, nk1, c, lane, m_run, l_run, o);
      }
    }
    l_run[0] += __shfl_xor(l_run[0], 32, 64);
  }
  // Merge: the waves of phase p > 0 leave their O (fragment layout) and (m, l)
  // in LDS; the phase-0 wave of each query tile folds them into its registers
  // in phase order and stores the range partial itself.
  __syncthreads();  // every tile consumed: Q and the slots become the merge area
  const int lane_f4 = lane;  // f32x4 (hb * 4 + r4) * 64 + lane of a slot
  if (wave < NCW && phase > 0) {
    float* mine = mrg + wave * SLOT1;
#pragma unroll
    for (int hb = 0; hb < 4; ++hb)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        ((f32x4*)mine)[(hb * 4 + r4) * 64 + lane_f4] =
            f32x4{o[0][hb][4 * r4], o[0][hb][4 * r4 + 1], o[0][hb][4 * r4 + 2], o[0][hb][4 * r4 + 3]};
    mine[4096 + lane * 2] = m_run[0];
    mine[4096 + lane * 2 + 1] = l_run[0];
  }
  __syncthreads();  // the phase-0 waves wait for the others' slots
  if (wave >= NCW || phase > 0) return;
  float mw[TSTRIDE], lw[TSTRIDE], wgt[TSTRIDE];
  mw[0] = m_run[0];
  lw[0] = l_run[0];
  float mm = mw[0];
#pragma unroll
  for (int p = 1; p < TSTRIDE; ++p) {
    mw[p] = mrg[(my_qt + QT * p) * SLOT1 + 4096 + lane * 2];
    lw[p] = mrg[(my_qt + QT * p) * SLOT1 + 4096 + lane * 2 + 1];
    mm = fmaxf(mm, mw[p]);
  }
  float ll = 0.f;
#pragma unroll
  for (int p = 0; p < TSTRIDE; ++p) {
    wgt[p] = mw[p] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw[p] - mm);
    ll += wgt[p] * lw[p];
  }
  if (lane < 32) {
    ml_part[(part * (QT * 32) + my_qt * 32 + lane) * 2] = mm;
    ml_part[(part * (QT * 32) + my_qt * 32 + lane) * 2 + 1] = ll;
  }
  f32x4* op = (f32x4*)(o_part + part * SLOTS) + my_qt * 1024;
#pragma unroll
  for (int hb = 0; hb < 4; ++hb)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int e = (hb * 4 + r4) * 64 + lane_f4;
      f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
      v += wgt[0] * f32x4{o[0][hb][4 * r4], o[0][hb][4 * r4 + 1], o[0][hb][4 * r4 + 2],
                          o[0][hb][4 * r4 + 3]};
#pragma unroll
      for (int p = 1; p < TSTRIDE; ++p) v += wgt[p] * ((const f32x4*)(mrg + (my_qt + QT * p) * SLOT1))[e];
      op[e] = v;
    }
}

// Combine the ranges of the decode attention. Float ((qt*4 + hb)*4 + r/4)*256 +
// l*4 + (r & 3) of a partial holds accumulator row r of lane l of the MFMA result
// (qt, hb): query vector qt*32 + (l & 31), head dim hb*32 + 8*(r >> 2) +
// 4*(l >> 5) + (r & 3). Work-group (kvh, qt, hb*4 + rq) owns the 256 contiguous
// floats with r in [4rq, 4rq + 4): 32 query vectors x the 8 consecutive head
// dims hb*32 + 8rq .. +8, so 256 work-groups share the reads. Each query
// vector's 8 dims are one 8-element chunk of the output row. Empty ranges
// (m = -inf) are skipped. MLR: range statistics per thread (R <= 8 MLR).
// out_fmt: 0 = ACT_F16P (no group sums: its consumer sums the hi + lo values
// itself), 1 = ACT_BF16, 2 = fp32 plain, 3 = bf16 plain. A value beyond the
// fp16 range sets DRT_ERR_F16_RANGE in *err.
template <int QT, int MLR>
__global__ __launch_bounds__(256) void attn_decode_combine_kernel(
    const float* __restrict__ o_part, const float* __restrict__ ml_part, int R, int n_rows,
    int Hq, int Hkv, void* __restrict__ out, int out_fmt, int* __restrict__ err) {
  constexpr int SLOTS = QT * 4096;
  const int kvh = blockIdx.x, qt = blockIdx.y, hb = blockIdx.z >> 2, rq = blockIdx.z & 3;
  const int j = threadIdx.x;
  const int G = Hq / Hkv;
  const int n_qv = n_rows * G;
  __shared__ float mx[8][32];
  __shared__ float ls[8][32];
  __shared__ f32x4 red[4][64];
  __shared__ float tile[32][9];
  extern __shared__ float wts[];  // [R][32] unnormalised weights
  // Thread j sums float4 f = j & 63 of the work-group's 256 floats (lane l = f of
  // the MFMA result: query vector c = f & 31, head dims 4 (f >> 5) .. + 4 of the
  // 8) over the ranges rgp, rgp + 4, ... (rgp = j >> 6); the four range groups
  // are added in LDS in a fixed order. One 16-byte load per range and thread
  // (a load instruction costs the CU about as long whatever its width).
  const int f = j & 63, rgp = j >> 6, c = f & 31;
  const int64_t sl4 = ((int64_t)qt * 4096 + (hb * 4 + rq) * 256) / 4 + f;
  const f32x4* op4 = (const f32x4*)o_part;
  // the O values of the first 4 RB ranges are loaded before (and independently
  // of) the statistics, so one memory latency covers both
  constexpr int RB = 8;
  f32x4 v[RB];
#pragma unroll
  for (int e = 0; e < RB; ++e)  // ranges >= R: clamped, unused
    v[e] = op4[((int64_t)min(rgp + 4 * e, R - 1) * Hkv + kvh) * (SLOTS / 4) + sl4];
  // 1. per query vector cc: max over ranges, weights, normaliser (8 range
  // groups; a thread holds ranges pg, pg + 8, ... < R <= 8 MLR)
  {
    const int cc = j & 31, pg = j >> 5;
    float2 ml[MLR];
#pragma unroll
    for (int k = 0; k < MLR; ++k) {
      const int rr = pg + 8 * k;
      const int64_t mi = ((int64_t)min(rr, R - 1) * Hkv + kvh) * (QT * 32) + qt * 32 + cc;
      ml[k] = ((const float2*)ml_part)[mi];
    }
    // every load above is issued before the ranges past R are masked (the
    // compiler would otherwise load under a branch and wait inside it)
    asm volatile("" ::: "memory");
    float mr[MLR], lr[MLR];
#pragma unroll
    for (int k = 0; k < MLR; ++k) {
      mr[k] = pg + 8 * k < R ? ml[k].x : -INFINITY;
      lr[k] = pg + 8 * k < R ? ml[k].y : 0.f;
    }
    float m_loc = -INFINITY;
#pragma unroll
    for (int k = 0; k < MLR; ++k) m_loc = fmaxf(m_loc, mr[k]);
    mx[pg][cc] = m_loc;
    __syncthreads();
    float mm = -INFINITY;
#pragma unroll
    for (int g = 0; g < 8; ++g) mm = fmaxf(mm, mx[g][cc]);
    float l_loc = 0.f;
#pragma unroll
    for (int k = 0; k < MLR; ++k) {
      const int rr = pg + 8 * k;
      const float w = mr[k] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mr[k] - mm);
      if (rr < R) wts[rr * 32 + cc] = w;
      l_loc += w * lr[k];
    }
    ls[pg][cc] = l_loc;
    __syncthreads();
  }
  // 2. weighted sum over the ranges (a zero weight never multiplies its O,
  // which an empty range does not write)
  float wv[RB];
#pragma unroll
  for (int e = 0; e < RB; ++e) wv[e] = wts[min(rgp + 4 * e, R - 1) * 32 + c];
  asm volatile("" ::: "memory");
  const f32x4 zero4 = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 acc = zero4;
#pragma unroll
  for (int e = 0; e < RB; ++e) {
    const float w = rgp + 4 * e < R ? wv[e] : 0.f;
    acc += w * (w == 0.f ? zero4 : v[e]);
  }
  for (int r0 = 4 * RB; r0 < R; r0 += 4 * RB) {
    f32x4 u[RB];
#pragma unroll
    for (int e = 0; e < RB; ++e)  // >= R: unused
      u[e] = op4[((int64_t)min(r0 + rgp + 4 * e, R - 1) * Hkv + kvh) * (SLOTS / 4) + sl4];
#pragma unroll
    for (int e = 0; e < RB; ++e) {
      const int rr = r0 + rgp + 4 * e;
      if (rr < R) {
        const float w = wts[rr * 32 + c];
        acc += w * (w == 0.f ? zero4 : u[e]);
      }
    }
  }
  red[rgp][f] = acc;
  __syncthreads();
  // 3. gather each query vector's 8 dims: dim offset 4 (f >> 5) + e
  if (j < 64) {
    float lsum = 0.f;
#pragma unroll
    for (int g = 0; g < 8; ++g) lsum += ls[g][c];
    const f32x4 sum = ((red[0][f] + red[1][f]) + red[2][f]) + red[3][f];
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[c][4 * (f >> 5) + e] = sum[e] / lsum;
  }
  __syncthreads();
  if (j >= 32) return;
  const int qv = qt * 32 + j;
  if (qv >= n_qv) return;
  const int row = qv / G, head = kvh * G + (qv - row * G);
  const int D = Hq * 128;
  const int col0 = head * 128 + hb * 32 + 8 * rq;
  float vals[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) vals[e] = tile[j][e];
  if (out_fmt == 0) {  // ACT_F16P: hi plane, lo plane at + n_rows * D
    _Float16 pk[8], pl[8];
    bool over = false;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const _Float16 h = (_Float16)vals[e];
      pk[f16p_index(e)] = h;
      pl[f16p_index(e)] = f16_lo(vals[e], h);
      over = over || f16_overflows(vals[e]);
    }
    _Float16* o = (_Float16*)out + (int64_t)row * D + col0;
    *(u32x4*)o = __builtin_bit_cast(u32x4, pk);
    *(u32x4*)(o + (int64_t)n_rows * D) = __builtin_bit_cast(u32x4, pl);
    if (over && err) atomicOr(err, DRT_ERR_F16_RANGE);
  } else if (out_fmt == 1 || out_fmt == 3) {
    uint16_t pk[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) pk[e] = float_to_bf16_bits(vals[e]);
    *(u32x4*)((uint16_t*)out + (int64_t)row * D + col0) = __builtin_bit_cast(u32x4, pk);
  } else {
    float* o = (float*)out + (int64_t)row * D + col0;
    *(f32x4*)o = f32x4{vals[0], vals[1], vals[2], vals[3]};
    *(f32x4*)(o + 4) = f32x4{vals[4], vals[5], vals[6], vals[7]};
  }
}

// Combine key splits (statistics in the base-2 units of attn_split_kernel).
// Sixteen threads per (row, head), thread c holding head dims 8c .. 8c + 7: it
// loads the (m, l) pair and its 32 bytes of O of up to 8 splits at once (one
// memory latency per 8 splits; their partial O are added against the batch's
// running maximum) and stores its 8 outputs as 16-byte chunks.
// out_fmt: 0 = ACT_F16P (+ xsum), 1 = ACT_BF16, 2 = fp32 plain, 3 = bf16 plain.
extern "C" __global__ __launch_bounds__(256) void attn_combine_kernel(
    const float* __restrict__ o_part, const float* __restrict__ ml_part, int n_splits, int n_rows,
    int Hq, int Hkv, void* __restrict__ out, float* __restrict__ xsum, int out_fmt,
    int* __restrict__ err) {
  constexpr int SB = 8;  // splits per batch of loads
  const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t n_wid = (int64_t)n_rows * Hq;
  if ((t >> 4) >= n_wid) return;  // whole groups of 16 (n_wid * 16 threads)
  const int64_t wid = t >> 4;
  const int ch = (int)(t & 15);
  const int row = (int)(wid / Hq), head = (int)(wid % Hq);
  const int G = Hq / Hkv;
  const int kvh = head / G, qv = row * G + (head - kvh * G);
  const int n_qv = n_rows * G;
  const int64_t stride = (int64_t)Hkv * n_qv;  // between splits
  const int64_t idx0 = (int64_t)kvh * n_qv + qv;
  float M = -INFINITY, L = 0.f;
  f32x4 a0 = f32x4{0.f, 0.f, 0.f, 0.f}, a1 = a0;
  for (int s0 = 0; s0 < n_splits; s0 += SB) {
    float2 ml[SB];
    f32x4 p0[SB], p1[SB];
#pragma unroll
    for (int j = 0; j < SB; ++j) {  // every load of the batch before the first use
      const int64_t at = idx0 + (int64_t)min(s0 + j, n_splits - 1) * stride;
      ml[j] = *(const float2*)(ml_part + at * 2);
      p0[j] = *(const f32x4*)(o_part + at * 128 + 8 * ch);
      p1[j] = *(const f32x4*)(o_part + at * 128 + 8 * ch + 4);
    }
    float mb = M;
#pragma unroll
    for (int j = 0; j < SB; ++j)
      if (s0 + j < n_splits) mb = fmaxf(mb, ml[j].x);
    const float sc = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - mb);
    a0 *= sc;
    a1 *= sc;
    L *= sc;
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      if (s0 + j < n_splits && ml[j].x != -INFINITY) {
        const float w = __builtin_amdgcn_exp2f(ml[j].x - mb);
        a0 += w * p0[j];
        a1 += w * p1[j];
        L += w * ml[j].y;
      }
    }
    M = mb;
  }
  const float inv = 1.f / L;
  float v[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = a0[e] * inv;
    v[e + 4] = a1[e] * inv;
  }
  const int D = Hq * 128;
  const int c0 = head * 128 + 8 * ch;  // first column of this thread's chunk
  if (out_fmt == 0) {  // ACT_F16P: hi plane, lo plane at + n_rows * D
    _Float16 h[8], lo[8];
    float gs = 0.f;
    bool over = false;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const _Float16 he = (_Float16)v[e], le = f16_lo(v[e], he);
      h[f16p_index(e)] = he;
      lo[f16p_index(e)] = le;
      gs += (float)he + (float)le;
      over = over || f16_overflows(v[e]);
    }
    _Float16* o = (_Float16*)out + (int64_t)row * D + c0;
    *(u32x4*)o = __builtin_bit_cast(u32x4, h);
    *(u32x4*)(o + (int64_t)n_rows * D) = __builtin_bit_cast(u32x4, lo);
    if (over && err) atomicOr(err, DRT_ERR_F16_RANGE);
    // the 64-column group sums: eight threads of aligned lanes per group
    gs += __shfl_xor(gs, 1, 64);
    gs += __shfl_xor(gs, 2, 64);
    gs += __shfl_xor(gs, 4, 64);
    if ((ch & 7) == 0) xsum[(int64_t)row * (D >> 6) + (c0 >> 6)] = gs;
  } else if (out_fmt == 1 || out_fmt == 3) {
    uint16_t hb[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) hb[e] = float_to_bf16_bits(v[e]);
    *(u32x4*)((uint16_t*)out + (int64_t)row * D + c0) = __builtin_bit_cast(u32x4, hb);
  } else {
    float* o = (float*)out + (int64_t)row * D + c0;
    *(f32x4*)o = f32x4{v[0], v[1], v[2], v[3]};
    *(f32x4*)(o + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
}

// Write K/V rows (logical [n][Hkv][128] fp32 or bf16) into the tiled cache of
// one layer at absolute positions pos0 .. pos0 + n - 1. One wave per (row, kv head).
template <typename T>
__global__ void kv_pack_kernel(const void* __restrict__ k_src, const void* __restrict__ v_src,
                               int src_is_bf16, int n, int Hkv, int pos0, T* __restrict__ kv,
                               int64_t kv_head_stride) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
  if (wid >= (int64_t)n * Hkv) return;
  const int row = (int)(wid / Hkv), h = (int)(wid % Hkv);
  const int pos = pos0 + row;
  T* tile = kv + (int64_t)h * kv_head_stride + (int64_t)(pos >> 5) * KV_TILE_ELEMS;
  const int kk = pos & 31;
  for (int e = 0; e < 2; ++e) {
    const int hd = lane + 64 * e;
    float kf, vf;
    const int64_t si = ((int64_t)row * Hkv + h) * 128 + hd;
    if (src_is_bf16) {
      kf = bf16_bits_to_float(((const uint16_t*)k_src)[si]);
      vf = bf16_bits_to_float(((const uint16_t*)v_src)[si]);
    } else {
      kf = ((const float*)k_src)[si];
      vf = ((const float*)v_src)[si];
    }
    const int ko = (((hd >> 4) * 2 + ((hd >> 3) & 1)) * 32 + kk) * 8 + (hd & 7);
    const int q16 = kk & 15;
    const int vo = ((((hd >> 5) * 2 + (kk >> 4)) * 2 + ((q16 >> 2) & 1)) * 32 + (hd & 31)) * 8 +
                   (q16 & 3) + 4 * (q16 >> 3);
    tile[ko] = MfmaT<T>::from_float(kf);
    tile[4096 + vo] = MfmaT<T>::from_float(vf);
  }
}

template __global__ void attn_split_kernel<_Float16, 2>(const _Float16*, const _Float16*, const _Float16*, int64_t,
                                                        int, int, int, int, int, int, int, int, int,
                                                        float*, float*, float);
template __global__ void attn_split_kernel<_Float16, 4>(const _Float16*, const _Float16*, const _Float16*, int64_t,
                                                        int, int, int, int, int, int, int, int, int,
                                                        float*, float*, float);
template __global__ void attn_split_kernel<__bf16, 2>(const __bf16*, const __bf16*, const __bf16*, int64_t, int,
                                                      int, int, int, int, int, int, int, int,
                                                      float*, float*, float);
template __global__ void attn_split_kernel<__bf16, 4>(const __bf16*, const __bf16*, const __bf16*, int64_t, int,
                                                      int, int, int, int, int, int, int, int,
                                                      float*, float*, float);
template __global__ void attn_decode_kernel<_Float16, 1>(const _Float16*, const _Float16*, const _Float16*,
                                                          int64_t, int, int, int, int,
                                                          const StepDesc*, float*, float*, float,
                                                          int*);
template __global__ void attn_decode_kernel<_Float16, 2>(const _Float16*, const _Float16*, const _Float16*,
                                                          int64_t, int, int, int, int,
                                                          const StepDesc*, float*, float*, float,
                                                          int*);
template __global__ void attn_decode_kernel<__bf16, 1>(const __bf16*, const __bf16*, const __bf16*, int64_t, int,
                                                        int, int, int, const StepDesc*, float*,
                                                        float*, float, int*);
template __global__ void attn_decode_kernel<_Float16, 4>(const _Float16*, const _Float16*, const _Float16*,
                                                       int64_t, int, int, int, int,
                                                       const StepDesc*, float*, float*, float,
                                                       int*);
template __global__ void attn_decode_kernel<__bf16, 4>(const __bf16*, const __bf16*, const __bf16*, int64_t, int,
                                                     int, int, int, const StepDesc*, float*,
                                                     float*, float, int*);
template __global__ void attn_decode_kernel<__bf16, 2>(const __bf16*, const __bf16*, const __bf16*, int64_t, int,
                                                        int, int, int, const StepDesc*, float*,
                                                        float*, float, int*);
template __global__ void kv_pack_kernel<_Float16>(const void*, const void*, int, int, int, int,
                                                  _Float16*, int64_t);
template __global__ void kv_pack_kernel<__bf16>(const void*, const void*, int, int, int, int,
                                                __bf16*, int64_t);

namespace drt {

AttnPlan plan_attention(int n_rows, int Hq, int Hkv, int n_keys, size_t part_budget_bytes) {
  AttnPlan p;
  const int G = Hq / Hkv;
  const int qtiles = (n_rows * G + 31) / 32;
  p.qw = qtiles <= 2 ? 2 : 4;
  p.qgroups = (qtiles + p.qw - 1) / p.qw;
  const int n_tiles = std::max(1, (n_keys + 31) / 32);
  // two work-groups per CU for long key ranges; one for short ones (<= 2048 keys),
  // where a split's fixed costs (Q staging, partial stores, the combine's reads)
  // outweigh the extra parallelism (Dream's 512-key canvas: 18.7 + 8.4 ->
  // 18.2 + 7.0 us per layer with two splits instead of four)
  const int target_wgs = n_tiles <= 64 ? 256 : 512;
  int splits = std::max(1, target_wgs / (Hkv * p.qgroups));
  splits = std::min({splits, n_tiles, 64});  // the combine reads <= 64 splits
  // keep the fp32 partials within budget
  const size_t per_split = (size_t)Hkv * n_rows * G * 130 * 4;
  if (per_split > 0) splits = (int)std::max<size_t>(1, std::min<size_t>(splits, part_budget_bytes / per_split));
  p.tiles_per_split = (n_tiles + splits - 1) / splits;
  p.splits = (n_tiles + p.tiles_per_split - 1) / p.tiles_per_split;
  return p;
}

size_t attention_part_bytes(const AttnPlan& p, int n_rows, int Hq, int Hkv) {
  const size_t n_qv = (size_t)n_rows * (Hq / Hkv);
  return (size_t)p.splits * Hkv * n_qv * 130 * 4;
}

void attention(bool bf16, const void* q, const void* kv_layer, int64_t kv_head_stride,
               int n_rows, int Hq, int Hkv, int n_keys, int row_pos0, int mask_kind,
               int mask_prompt_len, int mask_block, const AttnPlan& plan, float* o_part,
               float* ml_part, void* out, float* xsum, int out_fmt, hipStream_t s, int* err,
               bool q_has_lo) {
  require(Hq % Hkv == 0, "attention needs Hq % Hkv == 0");
  require(n_keys >= 1 && n_rows >= 1, "attention needs at least one query row and key");
  const float scale = 1.0f / sqrtf(128.0f);
  const size_t lds_kv = (size_t)2 * 8192 * 2;
  const size_t lds = std::max(lds_kv, (size_t)plan.qw * 32 * 132 * 4);
  const dim3 grid(plan.splits * Hkv, plan.qgroups);
  const dim3 block(64 * plan.qw);
  // algorithmic bytes of this launch: Q read + the K/V of n_keys keys
  const double bytes = 2.0 * n_rows * Hq * 128 + 4.0 * n_keys * Hkv * 128;
#define DRT_ATTN(T, QW)                                                                         \
  {                                                                                             \
    auto fn = attn_split_kernel<T, QW>;                                                         \
    static size_t granted = 0;                                                                  \
    grant_lds((const void*)fn, lds, granted);                                                   \
    DRT_LAUNCH(Profiler::ATTN, bytes, fn, grid, block, lds, s, (const T*)q,                     \
               q_has_lo ? (const T*)q + (int64_t)n_rows * Hq * 128 : (const T*)nullptr,         \
               (const T*)kv_layer, kv_head_stride, n_rows, Hq, Hkv, n_keys, row_pos0,           \
               mask_kind, mask_prompt_len, mask_block, plan.tiles_per_split, o_part, ml_part,   \
               scale);                                                                          \
  }
  if (bf16) {
    if (plan.qw == 2) DRT_ATTN(__bf16, 2) else DRT_ATTN(__bf16, 4)
  } else {
    if (plan.qw == 2) DRT_ATTN(_Float16, 2) else DRT_ATTN(_Float16, 4)
  }
#undef DRT_ATTN
  DRT_HIP(hipGetLastError());
  const int64_t threads = (int64_t)n_rows * Hq * 16;
  hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                     o_part, ml_part, plan.splits, n_rows, Hq, Hkv, out, xsum, out_fmt, err);
  DRT_HIP(hipGetLastError());
}

size_t attention_decode_part_bytes(int ranges, int Hkv, int n_qv) {
  const int qt = n_qv <= 64 ? (n_qv + 31) / 32 : 4;
  return (size_t)ranges * Hkv * ((size_t)qt * 4096 + (size_t)qt * 32 * 2) * 4;
}

// Key ranges per KV head: as many as spread the tiles one per wave, at most one
// work-group per CU of the 256 (beyond that a second round of work-groups would
// double the time), so a range holds <= 12 tiles up to 32 * 12 * 256 / Hkv keys.
int attention_decode_ranges(int n_keys, int Hkv) {
  const int tiles = (n_keys + 31) / 32;
  const int per_cu = std::max(1, 256 / std::max(1, Hkv));
  return std::max(1, std::min(std::min(per_cu, 128), (tiles + 3) / 4));
}

// Decode attention (one mask segment, or two whose split desc->seg_rows falls on
// a query-tile boundary; <= 128 query vectors per KV head) + combine.
// `part` holds attention_decode_part_bytes(ranges, Hkv, n_rows * Hq / Hkv).
void attention_decode(bool bf16, const void* q, const void* kv_layer, int64_t kv_head_stride,
                      int n_rows, int Hq, int Hkv, int n_keys, const StepDesc* desc, int ranges,
                      float* part, void* out, float* xsum, int out_fmt, hipStream_t s, int* err,
                      bool q_has_lo) {
  const int G = Hq / Hkv;
  require(Hq % Hkv == 0 && n_rows * G <= 128,
          "decode attention needs <= 128 query vectors per head");
  require(ranges >= 1 && ranges <= 128, "decode attention takes 1..128 key ranges");
  const int qt = n_rows * G <= 64 ? (n_rows * G + 31) / 32 : 4;
  const float scale = 1.0f / sqrtf(128.0f);
  const dim3 grid(Hkv, ranges);
  const double bytes = 2.0 * n_rows * Hq * 128 + 4.0 * n_keys * Hkv * 128;
  float* o_part = part;
  float* ml_part = part + (size_t)ranges * Hkv * qt * 4096;
#define DRT_DECR(T, QT)                                                                     \
  {                                                                                         \
    auto fn = attn_decode_kernel<T, QT>;                                                   \
    static size_t granted = 0;                                                              \
    grant_lds((const void*)fn, ldsr, granted);                                              \
    DRT_LAUNCH(Profiler::ATTN, bytes, fn, grid, dim3(64 * (decr_ncw<QT>() + 1)), ldsr, s,   \
               (const T*)q,                                                                 \
               q_has_lo ? (const T*)q + (int64_t)n_rows * Hq * 128 : (const T*)nullptr,     \
               (const T*)kv_layer, kv_head_stride, n_rows, Hq, Hkv, n_keys, desc, o_part,   \
               ml_part, scale, err);                                                        \
  }
  const size_t ldsr =
      qt == 4 ? 128 + (size_t)(dec_qlo<4>() + 4 * 32 * DEC_QROW) * 2 + (size_t)decr_slots<4>() * 16384
              : 128 + (size_t)(DEC_QLO + qt * 32 * DEC_QROW) * 2 +
                    (size_t)(qt == 1 ? decr_slots<1>() : decr_slots<2>()) * 16384;
  if (bf16) {
    if (qt == 1) DRT_DECR(__bf16, 1) else if (qt == 2) DRT_DECR(__bf16, 2) else DRT_DECR(__bf16, 4)
  } else {
    if (qt == 1) DRT_DECR(_Float16, 1) else if (qt == 2) DRT_DECR(_Float16, 2) else DRT_DECR(_Float16, 4)
  }
#undef DRT_DECR
  DRT_HIP(hipGetLastError());
  (void)xsum;  // the F16P output's consumer computes its own group sums
  const dim3 cgrid(Hkv, qt, 16);
  const size_t clds = (size_t)ranges * 32 * 4;
#define DRT_COMB(QT, MLR)                                                                   \
  DRT_LAUNCH(Profiler::ATTN_COMBINE, 0.0, (attn_decode_combine_kernel<QT, MLR>), cgrid,      \
             dim3(256), clds, s, o_part, ml_part, ranges, n_rows, Hq, Hkv, out, out_fmt, err)
  if (ranges <= 32) {
    if (qt == 1) DRT_COMB(1, 4); else if (qt == 2) DRT_COMB(2, 4); else DRT_COMB(4, 4);
  } else {
    if (qt == 1) DRT_COMB(1, 16); else if (qt == 2) DRT_COMB(2, 16); else DRT_COMB(4, 16);
  }
#undef DRT_COMB
  DRT_HIP(hipGetLastError());
}

void kv_pack(bool kv_bf16, const void* k, const void* v, bool src_bf16, int n, int Hkv, int pos0,
             void* kv_layer, int64_t kv_head_stride, hipStream_t s) {
  const int64_t waves = (int64_t)n * Hkv;
  const dim3 grid((unsigned)((waves + 3) / 4));
  if (kv_bf16)
    hipLaunchKernelGGL(kv_pack_kernel<__bf16>, grid, dim3(256), 0, s, k, v, (int)src_bf16, n, Hkv,
                       pos0, (__bf16*)kv_layer, kv_head_stride);
  else
    hipLaunchKernelGGL(kv_pack_kernel<_Float16>, grid, dim3(256), 0, s, k, v, (int)src_bf16, n,
                       Hkv, pos0, (_Float16*)kv_layer, kv_head_stride);
  DRT_HIP(hipGetLastError());
}

}  // namespace drt
