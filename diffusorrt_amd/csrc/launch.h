// Host-side launch helpers shared by the runtime and the per-op C-ABI.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

#include <algorithm>
#include <stdexcept>
#include <string>
#include <vector>

namespace drt {

enum Status : int32_t { OK = 0, VERSION_MISMATCH = 1, INVALID_ARGUMENT = 2, UNSUPPORTED = 3,
                        INTERNAL_ERROR = 4 };

struct Error : std::runtime_error {
  int32_t status;
  Error(int32_t s, const std::string& m) : std::runtime_error(m), status(s) {}
};

[[noreturn]] inline void fail(int32_t s, const std::string& m) { throw Error(s, m); }
inline void require(bool ok, const std::string& m) {
  if (!ok) fail(INVALID_ARGUMENT, m);
}

#define DRT_HIP(expr)                                                                   \
  do {                                                                                  \
    hipError_t e_ = (expr);                                                             \
    if (e_ != hipSuccess)                                                               \
      ::drt::fail(::drt::INTERNAL_ERROR,                                                \
                  std::string(#expr) + ": " + hipGetErrorString(e_));                   \
  } while (0)

// Owned device allocation.
struct DevBuf {
  void* p = nullptr;
  size_t bytes = 0;
  bool owned = true;  // false: a view into memory owned elsewhere (an arena)
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  DevBuf(DevBuf&& o) noexcept : p(o.p), bytes(o.bytes), owned(o.owned) {
    o.p = nullptr;
    o.bytes = 0;
  }
  DevBuf& operator=(DevBuf&& o) noexcept {
    if (this != &o) {
      release();
      p = o.p;
      bytes = o.bytes;
      owned = o.owned;
      o.p = nullptr;
      o.bytes = 0;
    }
    return *this;
  }
  ~DevBuf() { release(); }
  void alloc(size_t n) {
    release();
    if (n) DRT_HIP(hipMalloc(&p, n));
    bytes = n;
    owned = true;
  }
  void view(void* q, size_t n) {
    release();
    p = q;
    bytes = n;
    owned = false;
  }
  void ensure(size_t n) {
    if (n > bytes) alloc(n);
  }
  void release() {
    if (p && owned) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
  template <typename T> T* as() const { return (T*)p; }
};

// Raise a kernel's dynamic-LDS limit when a launch needs more than 64 KiB.
// `granted` caches the largest size already granted for that kernel.
inline void grant_lds(const void* fn, size_t bytes, size_t& granted) {
  if (bytes <= 65536 || bytes <= granted) return;
  DRT_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
  granted = bytes;
}

// Per-dispatch device timing for the hot kernel classes. When a profiler is
// installed on the calling thread and switched on, DRT_LAUNCH dispatches with
// hipExtLaunchKernelGGL, whose start/stop events are the dispatch packet's own
// timestamps (no extra packets in the stream); collect() reads them after the
// stream has drained.
struct Profiler {
  // ATTN_COMBINE: the decode attention's range combine (no algorithmic bytes of
  // its own: its partials are the attention's intermediate)
  enum Class : int { ATTN = 0, GEMM = 1, LMHEAD = 2, ATTN_COMBINE = 3, NCLASS = 4 };
  bool on = false;
  std::vector<hipEvent_t> pool;
  struct Rec { int cls; double bytes; };
  std::vector<Rec> recs;
  double ms[NCLASS] = {};
  double bytes[NCLASS] = {};
  int64_t launches[NCLASS] = {};

  void pair(hipEvent_t* a, hipEvent_t* b, int cls, double nbytes) {
    const size_t i = recs.size();
    while (pool.size() < 2 * (i + 1)) {
      hipEvent_t e;
      DRT_HIP(hipEventCreate(&e));
      pool.push_back(e);
    }
    *a = pool[2 * i];
    *b = pool[2 * i + 1];
    recs.push_back({cls, nbytes});
  }
  void collect() {
    for (size_t i = 0; i < recs.size(); ++i) {
      float t = 0.f;
      DRT_HIP(hipEventElapsedTime(&t, pool[2 * i], pool[2 * i + 1]));
      ms[recs[i].cls] += t;
      bytes[recs[i].cls] += recs[i].bytes;
      launches[recs[i].cls] += 1;
    }
    recs.clear();
  }
  void reset() {
    recs.clear();
    for (int c = 0; c < NCLASS; ++c) { ms[c] = 0; bytes[c] = 0; launches[c] = 0; }
  }
  ~Profiler() {
    for (hipEvent_t e : pool) (void)hipEventDestroy(e);
  }
};

// The profiler of the session running on this thread (null when none).
extern thread_local Profiler* g_prof;

// Launch `fn` (a kernel function pointer variable), timed when profiling.
#define DRT_LAUNCH(CLS, BYTES, FN, GRID, BLOCK, SHMEM, STREAM, ...)                        \
  do {                                                                                     \
    ::drt::Profiler* p_ = ::drt::g_prof;                                                   \
    if (p_ && p_->on) {                                                                    \
      hipEvent_t a_, b_;                                                                   \
      p_->pair(&a_, &b_, (CLS), (BYTES));                                                  \
      hipExtLaunchKernelGGL(FN, GRID, BLOCK, SHMEM, STREAM, a_, b_, 0, __VA_ARGS__);       \
    } else {                                                                               \
      hipLaunchKernelGGL(FN, GRID, BLOCK, SHMEM, STREAM, __VA_ARGS__);                     \
    }                                                                                      \
  } while (0)

// Activation formats (match ActFmt in common.h; 2 = fp32 plain).
enum Fmt : int { F16P = 0, BF16 = 1, F32 = 2 };

// A linear weight resident in the device layout (q4 tile32-g64 or bf16 tile).
struct LinearW {
  int N = 0, K = 0;
  bool q4 = false;
  DevBuf qw, sb;   // q4
  DevBuf wb;       // bf16
  DevBuf bias;     // bf16 [N] or empty
};

// --- launchers (stream-ordered, no synchronization) ---
void q4_repack(const uint32_t* w_q, const uint16_t* scales, const uint16_t* biases, int N, int K,
               uint32_t* qw, uint32_t* sb, hipStream_t s);
void bf16_repack(const uint16_t* w, int N, int K, uint16_t* wb, hipStream_t s);
// fp32 or bf16 W [N, K] -> MLX q4 g64 packing (w_q [N][K/8], scales/biases bf16 [N][K/64]).
void q4_quantize(const void* w, bool w_f32, int N, int K, uint32_t* w_q, uint16_t* scales,
                 uint16_t* biases, hipStream_t s);
void q4_act_prep(const void* x, bool x_bf16, int M, int K, _Float16* xp, float* xsum,
                 hipStream_t s);

// Attention over the tiled cache of one layer.
struct AttnPlan {
  int qw = 2, qgroups = 1, splits = 1, tiles_per_split = 1;
};
AttnPlan plan_attention(int n_rows, int Hq, int Hkv, int n_keys, size_t part_budget_bytes);
size_t attention_part_bytes(const AttnPlan& p, int n_rows, int Hq, int Hkv);
void attention(bool bf16, const void* q, const void* kv_layer, int64_t kv_head_stride,
               int n_rows, int Hq, int Hkv, int n_keys, int row_pos0, int mask_kind,
               int mask_prompt_len, int mask_block, const AttnPlan& plan, float* o_part,
               float* ml_part, void* out, float* xsum, int out_fmt, hipStream_t s,
               int* err = nullptr, bool q_has_lo = true);
// (Both attention launchers read Q as its hi plane and, when q_has_lo, its lo plane
// n_rows * Hq * 128 elements after it; without it the lo plane is zero.)
// Decode attention over `ranges` key ranges (attention_decode_ranges(n_keys, Hkv) when
// the key count is known at launch) + the range combine; `part` is a workspace of
// attention_decode_part_bytes(ranges, Hkv, n_rows * Hq / Hkv) bytes.
size_t attention_decode_part_bytes(int ranges, int Hkv, int n_qv);
int attention_decode_ranges(int n_keys, int Hkv);
void attention_decode(bool bf16, const void* q, const void* kv_layer, int64_t kv_head_stride,
                      int n_rows, int Hq, int Hkv, int n_keys, const StepDesc* desc, int ranges,
                      float* part, void* out, float* xsum, int out_fmt, hipStream_t s,
                      int* err = nullptr, bool q_has_lo = true);
void kv_pack(bool kv_bf16, const void* k, const void* v, bool src_bf16, int n, int Hkv, int pos0,
             void* kv_layer, int64_t kv_head_stride, hipStream_t s);

// Epilogues.
// ss_out (optional, M <= 32): per-32-column partial sums of squares of the rows,
// [d/32][32], the row statistics of the first decoder layer's RMSNorm.
// The first layer's pre-scaled norm input that embed() writes with the residual
// rows (the q4 split-K path): norm weight, eps, planes [M][d] x 2, their
// per-32-column sums, the scale per row, and the error word (fp16 range).
struct PreOut {
  const uint16_t* norm = nullptr;
  float eps = 0.f;
  uint16_t* planes = nullptr;
  float* xs = nullptr;
  float* sc = nullptr;
  int* err = nullptr;
};
void embed(const int32_t* tokens, const uint16_t* table, float* hidden, int M, int d,
           float* ss_out, hipStream_t s, const StepDesc* row_desc = nullptr,
           const PreOut* pre = nullptr);
void residual_norm(float* hidden, const float* part, int splits, int M_part, bool rnd_bf16,
                   const int32_t* src_rows, bool write_hidden, const uint16_t* norm_w, float eps,
                   int d, int fmt, void* act, float* xsum, int n_out_rows, hipStream_t s,
                   int* err = nullptr);
// LM head: per-row scores (f64) and tokens, optional raw logits.
size_t lmhead_stats_bytes(int M, int N);
void lmhead(const LinearW& w, const void* act, const float* xsum, int M, float* logits_out,
            void* stats, float temperature, uint64_t seed, int step, const int32_t* positions,
            double* scores, int32_t* tokens, hipStream_t s, const StepDesc* desc = nullptr,
            int exclude_col = -1, const int* err_dev = nullptr, int* err_host = nullptr,
            double* scores_d = nullptr, int32_t* tokens_d = nullptr);
// The device-side fixed-quota commit of a block step (desc->quota of the
// desc->n_lm LM rows at `positions`, from the LM head's device scores / tokens)
// into the device canvas. advance (optional): the descriptor of the next step,
// whose step becomes desc->step + 1 and quota quota_tab[that step % QUOTA_TAB].
void block_commit(const double* scores_d, const int32_t* tokens_d, const int32_t* positions,
                  int32_t* canvas, int mask_id, const StepDesc* desc, hipStream_t s,
                  StepDesc* advance = nullptr, const int32_t* quota_tab = nullptr);

// y = round_bf16(y) (+ bias after rounding); x fp32 -> bf16 bits.
void round_bf16_inplace(float* y, int64_t n, const uint16_t* bias, int N, hipStream_t s);
void to_bf16(const float* x, uint16_t* o, int64_t n, hipStream_t s);

// Per-op fp32 helpers (KernelTable seam).
void rms_norm_rows(const float* x, const uint16_t* w, float eps, float* y, int rows, int d,
                   hipStream_t s);
void rope_rows(const float* x, const float* cos_t, const float* sin_t, float* y, int rows, int H,
               int hd, hipStream_t s);
void swiglu_rows(const float* g, const float* u, float* y, int64_t n, hipStream_t s);

}  // namespace drt
