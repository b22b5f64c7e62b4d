/*
 * drt_rocm.h -- C-ABI of libdrt_rocm.so, the MI355X (gfx950) denoise-step engine.
 *
 * This is the native side of a `rocm` backend for DiffusorRT's diffusion-LM
 * decode. It implements the device-session contract that the reference's
 * compiled CUDA provider (`diffusorrt_runtime.Runtime`, absent from the
 * reference) exposes to Python, and the boundary ABI v0.1.0 the reference
 * declares in python/src/edllm/abi/. Paths below are relative to the
 * reference's python/src/edllm/.
 *
 * Conventions (abi/buffers.py:19-75, abi/handles.py:17-72, abi/forward.py:20-26):
 *  - every entry point returns an AbiStatus value (DRT_OK ... DRT_INTERNAL_ERROR);
 *    the message of the last failure on the calling thread is drt_last_error();
 *  - runtimes and sessions are kinded uint64 handles, monotonic and never reused;
 *    releasing a handle twice is DRT_INVALID_ARGUMENT;
 *  - weight tensors passed to drt_runtime_create are BORROWED device buffers:
 *    the runtime copies them into its own device layout before returning;
 *  - per-op entry points take device pointers and a hipStream_t (NULL = the
 *    null stream) and never synchronize; sessions run on their runtime's own
 *    stream and return only after results are on the host;
 *  - one session is used by one thread at a time (engine.py:143-157).
 */
#ifndef DRT_ROCM_H
#define DRT_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* AbiStatus (abi/forward.py:20-26). */
enum {
  DRT_OK = 0,
  DRT_VERSION_MISMATCH = 1,
  DRT_INVALID_ARGUMENT = 2,
  DRT_UNSUPPORTED = 3,
  DRT_INTERNAL_ERROR = 4
};

/* DType (abi/buffers.py:22-28); DRT_F16 is appended after the reference's values. */
enum { DRT_F32 = 0, DRT_F64 = 1, DRT_BF16 = 2, DRT_I32 = 3, DRT_I64 = 4, DRT_U8 = 5, DRT_F16 = 6 };

/* DecodeStrategy / CommitPolicy / AttentionMaskKind values (abi/enums.py:14-43). */
enum { DRT_DECODE_BLOCK_THRESHOLD = 0, DRT_DECODE_FIXED_QUOTA = 6, DRT_DECODE_BD3_FIXED_QUOTA = 7 };
enum { DRT_COMMIT_THRESHOLD = 2, DRT_COMMIT_FIXED_QUOTA = 3 };
enum { DRT_MASK_BIDIRECTIONAL = 0, DRT_MASK_D2F_HYBRID = 1, DRT_MASK_FULL = 2 };

/* Logits conventions (mlx_d2f_forward.py:74-93). */
enum { DRT_LOGITS_RAW = 0, DRT_LOGITS_DREAM_AR_SHIFT = 1 };

/* EngineConfig (abi/lifetimes.py:30-43, process lifetime); fields after
 * window_exec are this engine's own. */
typedef struct drt_engine_config {
  int32_t compute_dtype;            /* ComputeDtype: 0 = bf16 */
  int32_t linear_quant_bits;        /* -1 (UNSET) = bf16 weights, 4 = q4 affine */
  int32_t linear_quant_group_size;  /* 64 */
  int32_t layer0_kv_cache_enabled;  /* must be 0 */
  int32_t prefix_kv_cache;          /* must be 0 (approximate caches are not offered) */
  int32_t block_kv_cache;           /* must be 0 */
  int32_t d2f_exact_kv_cache;       /* 0 or 1: 1 is what cuda_engine_config(exact_kv=True)
                                     * sends for Dream's block_threshold (model.py:913, 991;
                                     * backends/device_runtime.py:53-58). Sessions of this
                                     * runtime serve block_threshold over the exact prompt +
                                     * frozen-block K/V either way; fixed-quota sessions refuse
                                     * exact_kv at start (device_runtime.py:223-231). */
  int32_t cross_request_cache;      /* must be 0 */
  int32_t canvas_cache;             /* must be 0 */
  int64_t canvas_cache_budget_bytes;
  int32_t window_exec;              /* WindowExec: 0 auto */
  int32_t device_ordinal;
  int32_t max_forward_rows;         /* rows per forward chunk (prefill chunk; >= canvas for bidirectional) */
  int32_t kv_dtype;                 /* DRT_F16 (default) or DRT_BF16 for the KV cache and Q */
  int64_t creation_memory_budget_bytes; /* 0 = unbounded */
} drt_engine_config;

/* ModelGeometry (abi/lifetimes.py:46-55) plus the architecture facts the
 * forward needs (model_definitions.py:418-448). */
typedef struct drt_model_geometry {
  int32_t layer_count;
  int32_t hidden_size;
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t vocab_size;
  int32_t max_position_embeddings;
  int32_t head_dim;             /* must be 128 */
  int32_t intermediate_size;
  float rms_norm_eps;
  float rope_theta;
  int32_t qk_norm;              /* Qwen3 per-head q/k RMSNorm */
  int32_t qkv_bias;             /* Qwen2/Dream q/k/v biases */
  int32_t logits_convention;    /* DRT_LOGITS_* */
} drt_model_geometry;

/* SessionDecodeConfig (abi/lifetimes.py:57-69). */
typedef struct drt_session_config {
  int32_t decode_strategy;
  int32_t commit_policy;
  int32_t attention_mask_kind;
  int32_t block_size;
  int32_t steps;
  int32_t max_tokens;
  int32_t trace_canvas;
  int32_t error_fixing;
  int32_t reserved[8];              /* must be 0 (SessionDecodeConfig.reserved) */
} drt_session_config;

/* A borrowed device tensor (TensorDesc + BufferView, abi/buffers.py:45-75),
 * C-contiguous, addressed by its package weight name. q4 weights come as three
 * tensors "<linear>.weight" (I32 bit-packed uint32 [N, K/8], MLX packing),
 * "<linear>.scales" and "<linear>.biases" (BF16 [N, K/64]). The rotary tables
 * are "rope.cos" / "rope.sin" (F32 [positions, head_dim/2]). */
typedef struct drt_tensor {
  const char* name;
  const void* data;
  int32_t dtype;
  int32_t ndim;
  int64_t shape[4];
} drt_tensor;

typedef struct drt_metrics {
  int64_t forward_count;          /* proposals + windows executed */
  int64_t active_rows;            /* rows forwarded for denoising (sum) */
  int64_t commit_rows;            /* rows forwarded once to write prefix K/V (sum) */
  int64_t lm_rows;                /* LM-head rows (sum) */
  int64_t kv_cache_len;           /* rows with exact committed K/V */
  int64_t kv_cache_bytes;         /* device bytes held by the prefix K/V cache */
  double last_forward_ms;         /* device time of the last forward (HIP events) */
  double total_forward_ms;
  /* per-dispatch device time while profiling is on (drt_session_set_profiling), by
   * kernel class 0 = attention, 1 = linear GEMMs, 2 = LM head, 3 = the decode
   * attention's range combine: summed ms, summed algorithmic bytes (none for the
   * combine, whose reads are the attention's partials), launch counts */
  double prof_ms[4];
  double prof_bytes[4];
  int64_t prof_launches[4];
} drt_metrics;

/* ---- library / handles ---- */

/* ABI version (abi/__init__.py:15): (0, 1, 0). */
void drt_abi_version(int32_t* major, int32_t* minor, int32_t* patch);
/* Copies the calling thread's last error message; returns its full length. */
size_t drt_last_error(char* buf, size_t len);
/* diffusorrt_release_handle (abi/buffers.py:45): releases a runtime or session. */
int32_t drt_release_handle(uint64_t handle);

/* ---- runtime + device session (model.py:873-920, 1026-1087;
 *      backends/device_runtime.py:108-183, 277-365) ---- */

/* Runtime(package, device="rocm", engine_config, precision, device_ordinal, budget). */
int32_t drt_runtime_create(const drt_engine_config* engine, const drt_model_geometry* geometry,
                           const drt_tensor* weights, int32_t n_weights, uint64_t* out_runtime);
/* runtime.session(session_config=...): bd3_fixed_quota (fixed_quota commit, d2f_hybrid),
 * fixed_quota (fixed_quota commit, bidirectional) or block_threshold (threshold commit,
 * d2f_hybrid; device_runtime.py:186-274); decode_strategy < 0 opens a window-only session. */
int32_t drt_session_open(uint64_t runtime, const drt_session_config* config,
                         uint64_t* out_session);
/* session.start_device(tokens, prompt_len=origin, block_size, mask_token_id, exact_kv,
 *                      steps, memory_budget_bytes, temperature, seed). exact_kv is for
 * block_threshold sessions only (greedy: temperature 0); their scores leave the MASK
 * column out of the softmax and argmax (diffusion_runtime.py:256-282). */
int32_t drt_session_start(uint64_t session, const int32_t* tokens, int32_t n_tokens,
                          int32_t prompt_len, int32_t block_size, int32_t mask_token_id,
                          int32_t exact_kv, int32_t steps, int64_t memory_budget_bytes,
                          double temperature, uint64_t seed);
/* session.propose_device(frontier, window_end, frozen_prefix) -> (scores f64, tokens,
 * forwarded_rows). Only these cross to the host. On a d2f_hybrid session rows
 * [0, frozen_prefix) are served from the exact K/V cache (forwarded once when they
 * freeze); under the Dream logits shift the forward also recomputes row
 * frozen_prefix - 1, which the block's first position reads (mlx_d2f_forward.py:226-232). */
int32_t drt_session_propose(uint64_t session, const int32_t* frontier, int32_t n_frontier,
                            int32_t window_end, int32_t frozen_prefix, double* out_scores,
                            int32_t* out_tokens, int32_t* out_forwarded_rows);
/* The BD3 fixed-quota loop (diffusion_runtime.py:1200-1346 driven as in :1829-1991) run inside
 * the library: up to max_forwards plan/propose/select/commit steps with no return to the caller
 * in between; the policy state persists in the session. No counterpart in the reference, whose
 * loop runs on the host; rows with exactly equal float64 scores commit lowest index first. */
int32_t drt_session_bd3_decode(uint64_t session, int32_t prompt_len, int32_t max_tokens,
                               int32_t steps, int32_t eos_token_id, int32_t requires_alignment,
                               int32_t max_forwards, int32_t* out_forwards,
                               int32_t* out_committed, int32_t* out_done);
/* The session's canvas: n_out >= its length (the length is returned in *out_len). */
int32_t drt_session_canvas(uint64_t session, int32_t* out, int32_t n_out, int32_t* out_len);
/* session.commit_device(positions, tokens). */
int32_t drt_session_commit(uint64_t session, const int32_t* positions, const int32_t* tokens,
                           int32_t n);
/* session.execute_window(token_ids, scope, mask_geometry=(prompt_len, block_size)):
 * convention-applied fp32 logits [n_scope][vocab] in scope order. mask_block_size
 * <= 0 means no geometry (bidirectional graph). */
int32_t drt_session_execute_window(uint64_t session, const int32_t* token_ids,
                                   int32_t n_tokens, const int32_t* scope, int32_t n_scope,
                                   int32_t mask_prompt_len, int32_t mask_block_size,
                                   float* out_logits, int64_t out_capacity,
                                   int32_t* out_n_vocab, int32_t* out_forwarded_rows);
/* session.device_metrics(). */
int32_t drt_session_metrics(uint64_t session, drt_metrics* out);
/* Time every attention / linear / LM-head dispatch of this session with its own
 * dispatch timestamps (1 = on, 0 = off; switching on clears the counters). No
 * counterpart in the reference: the stage timers of backends/mlx_forward.py:1447-1459
 * are host wall clock. */
int32_t drt_session_set_profiling(uint64_t session, int32_t enable);

/* ---- per-op kernels: the KernelTable seam (backends/kernel_table.py:118-126) ---- */

/* QuantizedWeight (mlx_ops.py:43-60) -> device tile layout: qw uint32 [N*K/8],
 * sb uint32 [N*K/64]. */
int32_t drt_op_q4_repack(const void* w_q, const void* scales, const void* biases, int32_t n,
                         int32_t k, void* qw, void* sb, void* stream);
/* quantize_linear_weight(w, group_size=64, bits=4) (mlx_ops.py:63-94, run once per load by
 * backends/mlx_dream.py:2073-2108): fp32 or bf16 W [n, k] (rounded to bf16 first) -> the
 * QuantizedWeight bundle in MLX packing: w_q uint32 [n, k/8], scales/biases bf16 [n, k/64].
 * k % 64 != 0 is DRT_UNSUPPORTED (the reference keeps such a weight in floating point). */
int32_t drt_op_q4_quantize(const void* w, int32_t w_dtype, int32_t n, int32_t k, void* w_q,
                           void* scales, void* biases, void* stream);
/* A floating-point package tensor cast to the resident bf16 dtype, round to nearest even
 * (the `.astype(target)` of backends/mlx_dream.py:1957-1963, 1998-1999): fp32 x [n] ->
 * bf16 y [n]. */
int32_t drt_op_cast_bf16(const float* x, void* y, int64_t n, void* stream);
/* linear(x, QuantizedWeight, bias) (mlx_ops.py:97-130): y fp32 [m, n] from x fp32 or
 * bf16 [m, k]; bias bf16 [n] or NULL. Needs drt_op_q4_linear_workspace_bytes(m, n, k).
 * m <= 32: one split-K launch that reads x as it is; its arrival counters are a block of a
 * library array reserved for (device, stream) on first use (32 per device; a further
 * stream's calls take a two-launch path), so calls on different streams never share
 * counters. Calls that overlap must not share a workspace. */
size_t drt_op_q4_linear_workspace_bytes(int32_t m, int32_t n, int32_t k);
int32_t drt_op_q4_linear(const void* qw, const void* sb, const void* x, int32_t x_dtype,
                         int32_t m, int32_t n, int32_t k, const void* bias, float* y,
                         void* workspace, size_t workspace_bytes, void* stream);
/* drt_op_q4_linear without a workspace argument and without any device allocation: for
 * callers that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. Its workspace is a
 * 64 MiB device array of the library, one per GPU (held until the process ends, its
 * address looked up once per device); shapes whose drt_op_q4_linear_workspace_bytes
 * exceed 64 MiB are refused with DRT_INVALID_ARGUMENT. The launch uses the calling
 * thread's current device. Calls that overlap on one GPU share that array and race:
 * serialize them (one stream, or events). Nothing in the array needs to start at zero. */
int32_t drt_op_q4_linear_noalloc(const void* qw, const void* sb, const void* x, int32_t x_dtype,
                                 int32_t m, int32_t n, int32_t k, const void* bias, float* y,
                                 void* stream);
/* bf16 weight W [n, k] -> device tile layout wb (same size). */
int32_t drt_op_bf16_repack(const void* w, int32_t n, int32_t k, void* wb, void* stream);
/* linear(x, bf16 W): y = bf16(bf16(x) @ W^T) as fp32 [m, n]; x bf16 [m, k]. */
size_t drt_op_bf16_linear_workspace_bytes(int32_t m, int32_t n, int32_t k);
int32_t drt_op_bf16_linear(const void* wb, const void* x, int32_t m, int32_t n, int32_t k,
                           const void* bias, float* y, void* workspace, size_t workspace_bytes,
                           void* stream);
/* Write K/V rows ([n, hkv, 128] fp32 or bf16) into a tiled cache of one layer at
 * positions pos0..pos0+n-1. cache holds hkv * head_stride elements of kv_dtype. */
int32_t drt_op_kv_pack(const void* k, const void* v, int32_t src_dtype, int32_t n, int32_t hkv,
                       int32_t pos0, void* cache, int64_t head_stride, int32_t kv_dtype,
                       void* stream);
/* attention(q, k, v, head_dim=128, kind, mask_geometry, q_positions) (mlx_ops.py:347-443)
 * over the tiled cache: q [rows, hq, 128] of kv_dtype, keys [0, n_keys), query row r at
 * absolute position row_pos0 + r. mask_kind: DRT_MASK_BIDIRECTIONAL or DRT_MASK_D2F_HYBRID
 * (with prompt_len / block_size). out [rows, hq*128] of out_dtype (DRT_F32 or DRT_BF16).
 * q is read in place by the kernels (no staging copy). */
size_t drt_op_attention_workspace_bytes(int32_t rows, int32_t hq, int32_t hkv, int32_t n_keys);
int32_t drt_op_attention(const void* q, const void* cache, int64_t head_stride, int32_t kv_dtype,
                         int32_t rows, int32_t hq, int32_t hkv, int32_t n_keys, int32_t row_pos0,
                         int32_t mask_kind, int32_t mask_prompt_len, int32_t mask_block_size,
                         void* out, int32_t out_dtype, void* workspace, size_t workspace_bytes,
                         void* stream);
/* rms_norm(x, weight, eps) (mlx_ops.py:21-35) on fp32 [rows, d], bf16 weight. */
int32_t drt_op_rms_norm(const float* x, const void* weight, float eps, float* y, int32_t rows,
                        int32_t d, void* stream);
/* rope(x [rows, h, hd], cos [rows, hd], sin [rows, hd]) split-half (mlx_ops.py:133-144). */
int32_t drt_op_rope(const float* x, const float* cos_t, const float* sin_t, float* y,
                    int32_t rows, int32_t h, int32_t hd, void* stream);
/* swiglu(gate, up) (mlx_ops.py:147-154) on fp32. */
int32_t drt_op_swiglu(const float* gate, const float* up, float* y, int64_t n, void* stream);
/* LM head + vocab softmax + scoring (diffusion_runtime.py:179-192, 203-275): rows of x
 * (fp32 [rows, k], already final-normed) against a q4 (qw/sb) or bf16 (wb) head of
 * vocab n; writes scores f64 [rows], tokens i32 [rows] and, if logits != NULL, the fp32
 * logits [rows, n]. positions [rows] key the sampling noise when temperature > 0. */
size_t drt_op_lm_head_workspace_bytes(int32_t rows, int32_t n, int32_t k);
int32_t drt_op_lm_head_score(const void* qw, const void* sb, const void* wb, int32_t rows,
                             int32_t n, int32_t k, const float* x, float temperature,
                             uint64_t seed, int32_t step, const int32_t* positions,
                             double* scores, int32_t* tokens, float* logits, void* workspace,
                             size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DRT_ROCM_H */
