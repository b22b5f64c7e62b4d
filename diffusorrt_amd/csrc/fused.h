// Arguments and modes of the fused linear kernel (fused_linear.hip).
#pragma once
#include "common.h"

enum { W_Q4 = 0, W_BF16 = 1 };
enum { PRO_ACT = 0, PRO_NORM = 1 };
enum { EPI_STORE = 0, EPI_QKV = 1, EPI_RESID = 2, EPI_SWIGLU = 3, EPI_LMSTAT = 4 };
// launch kinds (prologue + epilogue pairs used by the runtime)
enum { FL_QKV = 0, FL_RESID = 1, FL_SWIGLU = 2, FL_STORE = 3, FL_LMSTAT = 4 };

struct FusedArgs {
  // weights: q4 tile32-g64 (qw, sb) or bf16 tiles (wb); optional bf16 bias [N]
  const uint32_t* qw = nullptr;
  const uint32_t* sb = nullptr;
  const uint16_t* wb = nullptr;
  const uint16_t* bias = nullptr;
  int M = 0, N = 0, K = 0;
  // XCDs of the device (work-group i runs on XCD i % n_xcc) and the flag a
  // work-group sets if it finds itself on another XCD (next to M, N, K: the
  // skinny kernels fetch these first, in one scalar load)
  int n_xcc = 1;
  // 1: the placement above is not assumed; split-K slices meet through
  // device-scope fences and atomics instead of one XCD's L2
  int fenced = 0;
  int* placement_err = nullptr;
  // PRO_ACT: activation [M][K] (ACT_F16P + xsum[M][K/64], or ACT_BF16); for
  // the split-K q4 store kernel also fp32 (x_in 1) or bf16 (x_in 2) rows
  const void* act = nullptr;
  int x_in = 0;
  const float* act_xsum = nullptr;
  // PRO_NORM: fp32 residual stream [M][K] and bf16 norm weight [K]
  const float* hidden = nullptr;
  const uint16_t* norm_w = nullptr;
  float eps = 1e-6f;
  int rnd_bf16 = 0;  // bf16 weights: round the linear output to bf16
  // EPI_STORE
  float* y = nullptr;
  // EPI_RESID
  float* hidden_out = nullptr;
  // EPI_SWIGLU: activation of the down projection [M][N/2]
  void* act_out = nullptr;
  float* xsum_out = nullptr;
  int act_fmt = 0;
  // EPI_QKV
  const uint16_t* q_norm = nullptr;
  const uint16_t* k_norm = nullptr;
  const float* rope_cos = nullptr;
  const float* rope_sin = nullptr;
  void* q_out = nullptr;
  void* kv_layer = nullptr;
  int64_t kv_head_stride = 0;
  int Hq = 0, Hkv = 0, kv_bf16 = 0;
  const StepDesc* desc = nullptr;  // row0: absolute position of row 0
  // Skinny (M <= 32 per row tile, q4) path: split-K partial tiles, arrival
  // counters (zero on entry, left zero on exit) and the RMSNorm row statistics
  // carried between kernels as per-32-column partial sums of squares ([K/32][32]
  // floats per row tile).
  float* part = nullptr;
  size_t part_floats = 0;
  int* counters = nullptr;
  int n_counters = 0;
  const float* ss_in = nullptr;  // PRO_NORM: partial sums of squares of `hidden` rows
  float* ss_out = nullptr;       // EPI_RESID: partial sums of squares of the new rows
  // 32-row tiles the skinny workspaces hold (part, counters and the sums of
  // squares, one block each per tile: part_floats and n_counters per tile, the
  // sums of squares [K/32][32] at + tile * K): M <= 32 * sk_row_tiles
  int sk_row_tiles = 1;
  // Pre-scaled norm inputs (q4 skinny path). The residual update that produces
  // a row also writes w * h * c as ACT_F16P planes ([M][N] hi, lo at + M * N),
  // with w the next RMSNorm's weight and c a power of two per row, plus the
  // planes' per-32-column sums (like ss_out); the next q|k|v or gate|up kernel
  // then stages the planes as they are and multiplies its output rows by
  // rsqrt(mean h^2 + eps) / c. c = (the largest power of two <= the row's
  // previous norm factor) / 16: the planes stay ~16x below the normalised
  // values' magnitude unless the row's RMS grew more than 16-fold.
  // Producer (EPI_RESID): planes out, their sums, norm weight, c per row.
  void* pre_out = nullptr;
  float* pre_xs_out = nullptr;
  const uint16_t* pre_norm = nullptr;
  const float* pre_sc = nullptr;
  // Consumer (q|k|v, gate|up): act / act_xsum are the planes and their sums,
  // pre_sc_in the producer's c per row; pre_sc_out receives c for the next
  // producer (from this kernel's norm factors).
  const float* pre_sc_in = nullptr;
  float* pre_sc_out = nullptr;
  // EPI_LMSTAT (the large-M LM head): one LmStat per (row, 64-column block) at
  // lm_stats[row * (N / 64) + block], the logits themselves only when lm_logits
  // is set; sampling controls (temperature, seed, forward, excluded column) from
  // desc when it is set, else from these fields
  void* lm_stats = nullptr;
  float* lm_logits = nullptr;
  const int32_t* lm_pos = nullptr;  // canvas position of each row (sampling keys)
  float lm_temp = 0.f;
  uint64_t lm_seed = 0;
  int lm_step = 0;
  int lm_excl = -1;
};

// Row tiles of the runtime's split-K workspaces: forwards of up to 64 rows (a
// block-diffusion step together with the commit of the block before it) run
// on the split-K linears.
constexpr int SK_ROW_TILES = 2;

namespace drt {
void fused_linear(const FusedArgs& a, int kind, hipStream_t s);
// The split-K skinny kernels for q4 weights and M <= 32 rows; returns false
// (launching nothing) when the arguments do not fit them.
bool skinny_linear(const FusedArgs& a, int kind, hipStream_t s);
// Workspace the skinny kernels need for a linear of N outputs and K inputs.
size_t skinny_part_floats(int N, int K);
// One probe launch: does work-group i run on XCD i % n_xcc? (scratch_dev: >= 256 ints)
bool probe_round_robin(int n_xcc, int* scratch_dev, hipStream_t s);
int skinny_counters(int N);
// Whether the split-K kernels take a linear of this kind and shape (given
// workspaces sized by skinny_part_floats / skinny_counters).
bool skinny_supported(int kind, int N, int K);
// The large-M q4 kernels (M > 32): ACT_F16P activation in, kinds FL_QKV,
// FL_SWIGLU (ACT_F16P out) and FL_STORE (KS > 1: fp32 partial slices
// y + ks * M * N for a reduce pass).
bool big_linear_supported(const FusedArgs& a, int kind);
int big_linear_splits(int M, int N, int K, int max_ks);
// tail_part / tail_count (optional): the workspace of the split last round (see
// big_linear.hip), big_tail_part_floats() floats and one counter per split tile,
// zero on entry and left zero.
void big_linear(const FusedArgs& a, int kind, int KS, hipStream_t s, float* tail_part = nullptr,
                size_t tail_part_floats = 0, int* tail_count = nullptr, int n_tail_count = 0);
size_t big_tail_part_floats(int M, int N, int K, int n_cu);
constexpr int BIG_TAIL_COUNTERS = 512;  // split tiles a runtime's counters cover
// q|k|v projection + epilogue: split-K into `part` (when the tiles alone would
// leave CUs idle and part_floats suffices) and a separate epilogue pass.
void big_qkv(const FusedArgs& a, float* part, size_t part_floats, hipStream_t s);
// The per-head q|k|v epilogue (bias, q/k norm, RoPE, Q out, K/V into the cache)
// of a projection given as ks <= BG_QKV_MAX_KS fp32 slices [ks][M][N].
void qkv_epilogue_slices(const FusedArgs& a, const float* part, int ks, hipStream_t s);
constexpr int BG_QKV_MAX_KS = 8;    // split-K slices of the q|k|v projection
constexpr int BG_RESID_MAX_KS = 9;  // ... of o_proj / down_proj (reduced with the next norm)
constexpr int ST_QKV_MAX_KS = 4;    // ... of the weight-streaming q|k|v projection
constexpr int BG_OP_MAX_KS = 8;     // ... of the per-op linear (summed into its output)
// Weight-streaming q4 linears (stream_linear.hip) for M <= 32 rows and at least
// STREAM_MIN_WEIGHTS weights: the activation's K slice in LDS, the weights of a
// range of 128-column blocks streamed past it; fp32 K slices y[ks][M][N] out.
constexpr int64_t STREAM_MIN_WEIGHTS = (int64_t)8 << 20;
struct StreamPlan {
  int KS = 0, R = 0, nblk = 0;  // K slices, block ranges, most blocks per range
  bool single = true;           // the slice's activation fits LDS whole
};
bool stream_supported(int M, int N, int K);
StreamPlan stream_plan(int M, int N, int K, int max_ks);  // KS == 0: not supported
size_t stream_part_floats(int M, int N, int K, int max_ks);
// a.hidden set: the input is the fp32 residual stream, RMSNormed (a.norm_w, the
// row statistics a.ss_in) while staged; else a.act (ACT_F16P).
void stream_linear(const FusedArgs& f, const StreamPlan& p, hipStream_t s);
// SwiGLU of [gate 64 | up 64]-interleaved fp32 slices [KS][M][N] -> ACT_F16P [M][N / 2]
void swiglu_slices(const float* part, int KS, int M, int N, void* act, int* err, hipStream_t s);
// hidden[M][N] += the KS slices, and the new rows' partial sums of squares ss[N / 32][32]
void residual_slices(const float* part, int KS, int M, int N, float* hidden, float* ss,
                     hipStream_t s);
// y[i] = sum_k part[k * n + i] (+ bias[i % N]) in slice order (the per-op linear's reduce)
void sum_slices(const float* part, int KS, int64_t n, const uint16_t* bias, int N, float* y,
                hipStream_t s);
}
