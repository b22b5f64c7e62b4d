// Host-side launch helpers shared by the runtime and the per-op C-ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <stdexcept>
#include <string>

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
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  DevBuf(DevBuf&& o) noexcept : p(o.p), bytes(o.bytes) { o.p = nullptr; o.bytes = 0; }
  DevBuf& operator=(DevBuf&& o) noexcept {
    if (this != &o) { release(); p = o.p; bytes = o.bytes; o.p = nullptr; o.bytes = 0; }
    return *this;
  }
  ~DevBuf() { release(); }
  void alloc(size_t n) {
    release();
    if (n) DRT_HIP(hipMalloc(&p, n));
    bytes = n;
  }
  void ensure(size_t n) {
    if (n > bytes) alloc(n);
  }
  void release() {
    if (p) (void)hipFree(p);
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
void q4_act_prep(const void* x, bool x_bf16, int M, int K, _Float16* xp, float* xsum,
                 hipStream_t s);

// Split-K plan for a linear on M rows.
struct SplitPlan {
  int splits = 1;
  int per_split = 1;  // q4: groups; bf16: 16-k chunks
};
SplitPlan plan_linear(const LinearW& w, int M);
// Writes partials [plan.splits][M][N] fp32 into part. act: F16P (+xsum) for q4, BF16 for bf16.
void linear_partials(const LinearW& w, const void* act, const float* xsum, int M, float* part,
                     const SplitPlan& plan, hipStream_t s);
void bf16_linear_partials(const uint16_t* wb, const uint16_t* x, int M, int N, int K, float* part,
                          int splits, int chunks_per_split, hipStream_t s);
void splitk_reduce(const float* part, int splits, const uint16_t* bias, float* y, int M, int N,
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
               float* ml_part, void* out, float* xsum, int out_fmt, hipStream_t s);
void kv_pack(bool kv_bf16, const void* k, const void* v, bool src_bf16, int n, int Hkv, int pos0,
             void* kv_layer, int64_t kv_head_stride, hipStream_t s);

// Epilogues.
void embed(const int32_t* tokens, const uint16_t* table, float* hidden, int M, int d,
           hipStream_t s);
void residual_norm(float* hidden, const float* part, int splits, int M_part, bool rnd_bf16,
                   const int32_t* src_rows, bool write_hidden, const uint16_t* norm_w, float eps,
                   int d, int fmt, void* act, float* xsum, int n_out_rows, hipStream_t s);
void qkv_epilogue(bool kv_bf16, const float* part, int splits, int M, const uint16_t* bias,
                  bool rnd_bf16, const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                  const float* rope_cos, const float* rope_sin, int row_pos0, int Hq, int Hkv,
                  void* q_out, void* kv_layer, int64_t kv_head_stride, hipStream_t s);
void swiglu(const float* part, int splits, int M, int F, bool rnd_bf16, int fmt, void* act,
            float* xsum, hipStream_t s);

// LM head: per-row scores (f64) and tokens, optional raw logits.
size_t lmhead_stats_bytes(int M, int N);
void lmhead(const LinearW& w, const void* act, const float* xsum, int M, float* logits_out,
            void* stats, float temperature, uint64_t seed, int step, const int32_t* positions,
            double* scores, int32_t* tokens, hipStream_t s);

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
