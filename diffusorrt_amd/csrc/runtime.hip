// Runtime, device session and C-ABI of libdrt_rocm.so (see include/drt_rocm.h).
//
// A Runtime owns the model in device layouts (fused [q|k|v] and [gate|up]
// linears, q4 tile32-g64 or bf16 tiles), the rotary tables, one HIP stream and
// the forward workspace. A Session owns one request: the token canvas (host
// mirror + device copy) and the exact prefix K/V cache.
//
// Exact prefix K/V (BD3, d2f_hybrid with block origin 0): the reference
// recomputes the whole visible prefix x[:block_end] every denoise step
// (backends/diffusion_runtime.py:1331-1334). Under the absolute block-causal
// mask a row's K/V depend only on tokens of blocks <= its own, and a block's
// tokens never change once its rounds end (:1314-1322). So the K/V of every
// block before the active one is computed once, by one "commit" forward when
// the policy first proposes past it, and reused by every later step; each
// denoise step forwards only the active block's rows. This is the same math,
// re-associated.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/drt_rocm.h"
#include "fused.h"
#include "launch.h"

namespace drt {

thread_local std::string g_last_error;
thread_local Profiler* g_prof = nullptr;

// Installs a session's profiler on this thread for the duration of a call.
struct ProfScope {
  explicit ProfScope(Profiler* p) { g_prof = p; }
  ~ProfScope() { g_prof = nullptr; }
};

// ------------------------------------------------------------------ handles

enum class Kind : int { RUNTIME = 1, SESSION = 2 };

struct Runtime;
struct Session;

struct HandleTable {
  std::mutex mu;
  uint64_t next = 1;  // NULL_HANDLE = 0 is never issued
  std::map<uint64_t, std::pair<Kind, std::shared_ptr<void>>> live;

  uint64_t add(Kind k, std::shared_ptr<void> obj) {
    std::lock_guard<std::mutex> g(mu);
    const uint64_t h = next++;
    live.emplace(h, std::make_pair(k, std::move(obj)));
    return h;
  }
  template <typename T> std::shared_ptr<T> get(uint64_t h, Kind k) {
    std::lock_guard<std::mutex> g(mu);
    auto it = live.find(h);
    if (it == live.end()) fail(INVALID_ARGUMENT, "handle " + std::to_string(h) + " is not live");
    if (it->second.first != k)
      fail(INVALID_ARGUMENT, "handle " + std::to_string(h) + " has another kind");
    return std::static_pointer_cast<T>(it->second.second);
  }
  void release(uint64_t h) {
    std::shared_ptr<void> keep;
    {
      std::lock_guard<std::mutex> g(mu);
      auto it = live.find(h);
      if (it == live.end())
        fail(INVALID_ARGUMENT, "handle " + std::to_string(h) + " is not live; double release");
      keep = std::move(it->second.second);
      live.erase(it);
    }
    // `keep` is destroyed here, outside the lock (may free device memory).
  }
};

HandleTable& handles() {
  static HandleTable t;
  return t;
}

// ------------------------------------------------------------------ runtime

struct LayerW {
  LinearW qkv, o, gu, down;
  DevBuf in_norm, post_norm, q_norm, k_norm;
};

// All weights of a runtime live in one allocation: one mapping, large pages, and
// TLB reach for the whole model instead of a few hundred small buffers.
struct Arena {
  DevBuf mem;
  size_t off = 0;
  static size_t round(size_t n) { return (n + 255) & ~(size_t)255; }
  void place(DevBuf& b, size_t n) {
    require(off + round(n) <= mem.bytes, "weight arena overflow");
    b.view((char*)mem.p + off, n);
    off += round(n);
  }
};

struct Runtime {
  drt_engine_config engine{};
  drt_model_geometry geo{};
  bool q4 = false;
  bool kv_bf16 = false;
  int device = 0;
  hipStream_t stream = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  std::vector<LayerW> layers;
  DevBuf embed;       // bf16 [V][d]
  DevBuf final_norm;  // bf16 [d]
  LinearW lm_head;
  Arena warena;               // every weight below is a view into it
  DevBuf rope_cos, rope_sin;  // fp32 [P][64]
  int rope_positions = 0;
  int max_rows = 0;

  // workspace (sized for max_rows)
  DevBuf hidden, act, xsum, act_lm, xsum_lm, qbuf, attn_part, stats, lm_rows,
      lm_pos, logits;
  // split-K linears of <= 32-row forwards: partial tiles, arrival counters
  // (zeroed once; every kernel leaves them zero) and the residual stream's
  // per-32-column partial sums of squares
  DevBuf sk_part, sk_counters, sk_ss;
  // q4 models on the split-K linears: the next RMSNorm's input, pre-scaled by
  // the residual updates (two fp16 planes [rows][d], their per-32-column sums
  // [tile][d/32][32], and two alternating per-row scale vectors: each q|k|v or
  // gate|up kernel reads one and writes the other)
  bool sk_pre_on = false;
  DevBuf sk_pre, sk_pre_xs, sk_pre_sc;
  // large-M (> 32 rows) q4 forwards: the down projection's input activation and
  // the split-K partial slices of o_proj / down_proj
  DevBuf act2, big_part, big_tail_count;
  size_t big_part_floats = 0;
  size_t sk_part_floats = 0;
  // The split-K linears serve the <= 32-row q4 linears of small layers (their
  // residual epilogues carry the next norm's row statistics). Layers whose every
  // linear holds at least STREAM_MIN_WEIGHTS weights (the 7B shapes) forward
  // <= 32 rows through the weight-streaming linears instead (`streaming`): fp32 K
  // slices reduced by small passes (residual add + row statistics, q|k|v
  // epilogue, SwiGLU). The split-K units re-read the activation for every 128
  // columns there: gate|up 84 us, o / down 35, q|k|v 22 us per call.
  bool streaming = false;
  int sk_n_counters = 0;
  int n_xcc = 1;
  bool fenced = false;           // split-K exchange through device-scope fences (no placement assumed)
  DevBuf placement_err;          // int, set by a kernel that finds itself on an unexpected XCD
  int* placement_host = nullptr; // pinned copy, read after each synchronized forward
  // pinned landing area of a forward's scores and tokens, written by the LM head's
  // last kernel (the caller's arrays are pageable)
  char* out_host = nullptr;
  int lm_cap = 0;
  double* scores_host() const { return (double*)out_host; }
  // the same scores and tokens in device memory (the device-side block commit)
  DevBuf lm_scores_d, lm_tokens_d;
  int32_t* tokens_host() const { return (int32_t*)(out_host + (size_t)lm_cap * 8); }
  // Per-forward inputs: one pinned host slot + its device copy per forward, moved
  // by a single async copy. Slots 0-2 belong to the session graphs (commit, step,
  // commit + step); eager forwards rotate through the rest.
  struct StepUpload {
    StepDesc desc;
    int32_t lm_rows[32];
    int32_t lm_pos[32];
    int32_t tokens[64];
    int32_t quotas[QUOTA_TAB];  // a device block's quotas by step (block_commit's advance)
  };
  static constexpr int UPLOAD_SLOTS = 64;
  static constexpr int EAGER_SLOT0 = 3;
  StepUpload* up_host = nullptr;
  DevBuf up_dev;
  int up_next = EAGER_SLOT0;
  size_t attn_part_budget = 0;
  int logits_rows_cap = 0;

  ~Runtime() {
    if (stream) (void)hipStreamSynchronize(stream);
    if (up_host) (void)hipHostFree(up_host);
    if (placement_host) (void)hipHostFree(placement_host);
    if (out_host) (void)hipHostFree(out_host);
    if (ev0) (void)hipEventDestroy(ev0);
    if (ev1) (void)hipEventDestroy(ev1);
    if (stream) (void)hipStreamDestroy(stream);
  }

  int d() const { return geo.hidden_size; }
  int Hq() const { return geo.num_heads; }
  int Hkv() const { return geo.num_kv_heads; }
  int F() const { return geo.intermediate_size; }
  int V() const { return geo.vocab_size; }
  int fmt() const { return q4 ? F16P : BF16; }
};

namespace {

struct WeightMap {
  std::map<std::string, const drt_tensor*> by_name;
  const drt_tensor& get(const std::string& n) const {
    auto it = by_name.find(n);
    if (it == by_name.end()) fail(INVALID_ARGUMENT, "missing weight tensor '" + n + "'");
    return *it->second;
  }
  bool has(const std::string& n) const { return by_name.count(n) != 0; }
};

void check_tensor(const drt_tensor& t, int dtype, std::initializer_list<int64_t> shape) {
  const std::string n = t.name ? t.name : "?";
  if (t.dtype != dtype) fail(INVALID_ARGUMENT, "tensor '" + n + "' has dtype " +
                                                   std::to_string(t.dtype) + ", expected " +
                                                   std::to_string(dtype));
  if (t.ndim != (int)shape.size()) fail(INVALID_ARGUMENT, "tensor '" + n + "' has wrong rank");
  int i = 0;
  for (int64_t s : shape) {
    if (t.shape[i] != s)
      fail(INVALID_ARGUMENT, "tensor '" + n + "' dim " + std::to_string(i) + " is " +
                                 std::to_string(t.shape[i]) + ", expected " + std::to_string(s));
    ++i;
  }
  if (!t.data) fail(INVALID_ARGUMENT, "tensor '" + n + "' has a null data pointer");
}

void copy_bf16_vec(Arena& ar, DevBuf& dst, const WeightMap& wm, const std::string& name, int n,
                   hipStream_t s) {
  const drt_tensor& t = wm.get(name);
  check_tensor(t, DRT_BF16, {n});
  ar.place(dst, (size_t)n * 2);
  DRT_HIP(hipMemcpyAsync(dst.p, t.data, (size_t)n * 2, hipMemcpyDeviceToDevice, s));
}

// Device n-tile offsets of a part's 64-row block b when parts are interleaved in
// 64-column blocks ([gate 64 | up 64] per 128 columns, for the SwiGLU epilogue).
void repack_rows(LinearW& w, const WeightMap& wm, const std::string& part, int row0, int rows,
                 int dst_tile, int K, bool q4, hipStream_t s) {
  if (q4) {
    const drt_tensor& wq = wm.get(part + ".weight");
    const drt_tensor& sc = wm.get(part + ".scales");
    const drt_tensor& bi = wm.get(part + ".biases");
    const int G = K / 64;
    q4_repack((const uint32_t*)wq.data + (size_t)row0 * (K / 8),
              (const uint16_t*)sc.data + (size_t)row0 * G, (const uint16_t*)bi.data + (size_t)row0 * G,
              rows, K, w.qw.as<uint32_t>() + (size_t)dst_tile * G * 256,
              w.sb.as<uint32_t>() + (size_t)dst_tile * G * 32, s);
  } else {
    const drt_tensor& wt = wm.get(part + ".weight");
    bf16_repack((const uint16_t*)wt.data + (size_t)row0 * K, rows, K,
                w.wb.as<uint16_t>() + (size_t)dst_tile * 32 * K, s);
  }
}

// Build one fused linear from parts stacked along N (each part N_i rows, same K).
// interleave64: two parts of equal N laid out as [p0 64 | p1 64] per 128 columns.
size_t linear_arena_bytes(int N, int K, bool q4, bool with_bias) {
  size_t b = q4 ? Arena::round((size_t)N * K / 2) + Arena::round((size_t)N * (K / 64) * 4)
                : Arena::round((size_t)N * K * 2);
  if (with_bias) b += Arena::round((size_t)N * 2);
  return b;
}

void build_linear(Arena& ar, LinearW& w, const WeightMap& wm,
                  const std::vector<std::string>& parts, const std::vector<int>& Ns, int K,
                  bool q4, bool with_bias, hipStream_t s, bool interleave64 = false) {
  int N = 0;
  for (int n : Ns) N += n;
  w.N = N;
  w.K = K;
  w.q4 = q4;
  if (q4) {
    require(K % 64 == 0, "q4 linear in-dim must be a multiple of 64");
    ar.place(w.qw, (size_t)N * K / 2);
    ar.place(w.sb, (size_t)N * (K / 64) * 4);
  } else {
    ar.place(w.wb, (size_t)N * K * 2);
  }
  for (size_t i = 0; i < parts.size(); ++i) {
    const int n = Ns[i];
    require(n % (interleave64 ? 64 : 32) == 0, "linear out-dim must be a multiple of 32");
    if (q4) {
      check_tensor(wm.get(parts[i] + ".weight"), DRT_I32, {n, K / 8});
      check_tensor(wm.get(parts[i] + ".scales"), DRT_BF16, {n, K / 64});
      check_tensor(wm.get(parts[i] + ".biases"), DRT_BF16, {n, K / 64});
    } else {
      check_tensor(wm.get(parts[i] + ".weight"), DRT_BF16, {n, K});
    }
  }
  if (interleave64) {
    require(parts.size() == 2 && Ns[0] == Ns[1], "interleaving needs two equal parts");
    for (int b = 0; b < Ns[0] / 64; ++b)
      for (int i = 0; i < 2; ++i) repack_rows(w, wm, parts[i], 64 * b, 64, 4 * b + 2 * i, K, q4, s);
  } else {
    int n0 = 0;
    for (size_t i = 0; i < parts.size(); ++i) {
      repack_rows(w, wm, parts[i], 0, Ns[i], n0 / 32, K, q4, s);
      n0 += Ns[i];
    }
  }
  if (with_bias) {
    require(!interleave64, "biases are not interleaved");
    ar.place(w.bias, (size_t)N * 2);
    int n0 = 0;
    for (size_t i = 0; i < parts.size(); ++i) {
      const drt_tensor& b = wm.get(parts[i] + ".bias");
      check_tensor(b, DRT_BF16, {Ns[i]});
      DRT_HIP(hipMemcpyAsync(w.bias.as<uint16_t>() + n0, b.data, (size_t)Ns[i] * 2,
                             hipMemcpyDeviceToDevice, s));
      n0 += Ns[i];
    }
  }
}

}  // namespace

std::shared_ptr<Runtime> create_runtime(const drt_engine_config& e, const drt_model_geometry& g,
                                        const drt_tensor* ws, int nw) {
  require(g.head_dim == 128, "head_dim must be 128");
  require(g.layer_count >= 1 && g.hidden_size % 256 == 0 && g.hidden_size <= 3584,
          "hidden_size must be a multiple of 256 and <= 3584");
  require(g.num_heads >= 1 && g.num_kv_heads >= 1 && g.num_heads % g.num_kv_heads == 0,
          "num_heads must be a multiple of num_kv_heads");
  require(g.intermediate_size % 64 == 0, "intermediate_size must be a multiple of 64");
  require(g.vocab_size % 64 == 0, "vocab_size must be a multiple of 64");
  require(e.linear_quant_bits == 4 || e.linear_quant_bits == -1,
          "linear_quant_bits must be 4 (q4 affine) or -1 (bf16 weights)");
  if (e.linear_quant_bits == 4)
    require(e.linear_quant_group_size == 64, "only group size 64 is supported");
  if (e.layer0_kv_cache_enabled || e.prefix_kv_cache || e.block_kv_cache ||
      e.cross_request_cache || e.canvas_cache)
    fail(UNSUPPORTED, "the rocm runtime admits no approximate, cross-request or canvas caches");
  require(e.d2f_exact_kv_cache == 0 || e.d2f_exact_kv_cache == 1,
          "d2f_exact_kv_cache must be 0 or 1");
  require(e.kv_dtype == DRT_F16 || e.kv_dtype == DRT_BF16, "kv_dtype must be DRT_F16 or DRT_BF16");
  require(e.max_forward_rows >= 32, "max_forward_rows must be >= 32");

  auto rt = std::make_shared<Runtime>();
  rt->engine = e;
  rt->geo = g;
  rt->q4 = e.linear_quant_bits == 4;
  rt->kv_bf16 = e.kv_dtype == DRT_BF16;
  rt->device = e.device_ordinal;
  rt->max_rows = (e.max_forward_rows + 31) / 32 * 32;
  DRT_HIP(hipSetDevice(rt->device));
  DRT_HIP(hipStreamCreateWithFlags(&rt->stream, hipStreamNonBlocking));
  DRT_HIP(hipEventCreate(&rt->ev0));
  DRT_HIP(hipEventCreate(&rt->ev1));
  hipStream_t s = rt->stream;

  WeightMap wm;
  for (int i = 0; i < nw; ++i) {
    require(ws[i].name != nullptr, "weight tensor without a name");
    wm.by_name[ws[i].name] = &ws[i];
  }
  const int d = g.hidden_size, hd = 128, Hq = g.num_heads, Hkv = g.num_kv_heads,
            F = g.intermediate_size, V = g.vocab_size;
  {
    size_t total = Arena::round((size_t)V * d * 2) + Arena::round((size_t)d * 2) +
                   linear_arena_bytes(V, d, rt->q4, false);
    const size_t per_layer =
        linear_arena_bytes((Hq + 2 * Hkv) * hd, d, rt->q4, g.qkv_bias != 0) +
        linear_arena_bytes(d, Hq * hd, rt->q4, false) + linear_arena_bytes(2 * F, d, rt->q4, false) +
        linear_arena_bytes(d, F, rt->q4, false) + 2 * Arena::round((size_t)d * 2) +
        2 * Arena::round((size_t)hd * 2);
    total += per_layer * g.layer_count;
    rt->warena.mem.alloc(total);
  }
  Arena& ar = rt->warena;
  {
    const drt_tensor& t = wm.get("model.embed_tokens.weight");
    check_tensor(t, DRT_BF16, {V, d});
    ar.place(rt->embed, (size_t)V * d * 2);
    DRT_HIP(hipMemcpyAsync(rt->embed.p, t.data, (size_t)V * d * 2, hipMemcpyDeviceToDevice, s));
  }
  rt->layers.resize(g.layer_count);
  for (int l = 0; l < g.layer_count; ++l) {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    LayerW& L = rt->layers[l];
    build_linear(ar, L.qkv, wm,
                 {p + "self_attn.q_proj", p + "self_attn.k_proj", p + "self_attn.v_proj"},
                 {Hq * hd, Hkv * hd, Hkv * hd}, d, rt->q4, g.qkv_bias != 0, s);
    build_linear(ar, L.o, wm, {p + "self_attn.o_proj"}, {d}, Hq * hd, rt->q4, false, s);
    build_linear(ar, L.gu, wm, {p + "mlp.gate_proj", p + "mlp.up_proj"}, {F, F}, d, rt->q4, false, s,
                 /*interleave64=*/true);
    build_linear(ar, L.down, wm, {p + "mlp.down_proj"}, {d}, F, rt->q4, false, s);
    copy_bf16_vec(ar, L.in_norm, wm, p + "input_layernorm.weight", d, s);
    copy_bf16_vec(ar, L.post_norm, wm, p + "post_attention_layernorm.weight", d, s);
    if (g.qk_norm) {
      copy_bf16_vec(ar, L.q_norm, wm, p + "self_attn.q_norm.weight", hd, s);
      copy_bf16_vec(ar, L.k_norm, wm, p + "self_attn.k_norm.weight", hd, s);
    }
  }
  copy_bf16_vec(ar, rt->final_norm, wm, "model.norm.weight", d, s);
  build_linear(ar, rt->lm_head, wm, {"lm_head"}, {V}, d, rt->q4, false, s);
  {
    const drt_tensor& c = wm.get("rope.cos");
    const drt_tensor& sn = wm.get("rope.sin");
    require(c.ndim == 2 && c.shape[1] == 64 && c.dtype == DRT_F32, "rope.cos must be F32 [P, 64]");
    check_tensor(sn, DRT_F32, {c.shape[0], 64});
    rt->rope_positions = (int)c.shape[0];
    rt->rope_cos.alloc((size_t)c.shape[0] * 64 * 4);
    rt->rope_sin.alloc((size_t)c.shape[0] * 64 * 4);
    DRT_HIP(hipMemcpyAsync(rt->rope_cos.p, c.data, rt->rope_cos.bytes, hipMemcpyDeviceToDevice, s));
    DRT_HIP(hipMemcpyAsync(rt->rope_sin.p, sn.data, rt->rope_sin.bytes, hipMemcpyDeviceToDevice, s));
  }

  // Workspace for up to max_rows rows per forward.
  const int M = rt->max_rows;
  const int widest = std::max({d, Hq * hd, F});
  rt->hidden.alloc((size_t)M * d * 4);
  // activations and Q carry hi and lo fp16 planes (ACT_F16P)
  rt->act.alloc((size_t)2 * M * widest * 2);
  rt->xsum.alloc((size_t)M * (widest / 64) * 4);
  rt->qbuf.alloc((size_t)2 * M * Hq * hd * 2);
  DRT_HIP(hipHostMalloc((void**)&rt->up_host, sizeof(Runtime::StepUpload) * Runtime::UPLOAD_SLOTS,
                        hipHostMallocDefault));
  rt->up_dev.alloc(sizeof(Runtime::StepUpload) * Runtime::UPLOAD_SLOTS);
  rt->attn_part_budget = std::max<size_t>((size_t)64 << 20,
                                          (size_t)Hkv * M * (Hq / Hkv) * 130 * 4);
  rt->attn_part.alloc(rt->attn_part_budget);
  const int lm_cap = M;  // LM rows per forward <= rows forwarded
  rt->act_lm.alloc((size_t)2 * lm_cap * d * 2);
  rt->xsum_lm.alloc((size_t)lm_cap * (d / 64) * 4);
  rt->stats.alloc(lmhead_stats_bytes(lm_cap, V));
  // the forwards' scores and tokens land in pinned host memory, written by the
  // LM head's last kernel: [lm_cap] doubles, then [lm_cap] ints
  rt->lm_cap = lm_cap;
  DRT_HIP(hipHostMalloc((void**)&rt->out_host, (size_t)lm_cap * 12 + 16, hipHostMallocCoherent));
  rt->lm_scores_d.alloc((size_t)lm_cap * 8);
  rt->lm_tokens_d.alloc((size_t)lm_cap * 4);
  rt->lm_rows.alloc((size_t)lm_cap * 4);
  rt->lm_pos.alloc((size_t)lm_cap * 4);
  {
    const int n_qkv = (Hq + 2 * Hkv) * hd;
    size_t pf = 0;
    int nc = 0;
    for (auto nk : {std::make_pair(n_qkv, d), std::make_pair(d, Hq * hd), std::make_pair(2 * F, d),
                    std::make_pair(d, F)}) {
      pf = std::max(pf, skinny_part_floats(nk.first, nk.second));
      nc = std::max(nc, skinny_counters(nk.first));
    }

    rt->sk_part_floats = pf;
    rt->sk_n_counters = nc;
    // one block per 32-row tile of a <= SK_ROW_TILES * 32-row forward
    rt->sk_part.alloc(std::max<size_t>(pf, 1) * 4 * SK_ROW_TILES);
    rt->sk_counters.alloc((size_t)std::max(nc, 1) * 4 * SK_ROW_TILES);
    DRT_HIP(hipMemsetAsync(rt->sk_counters.p, 0, rt->sk_counters.bytes, s));
    rt->sk_ss.alloc((size_t)d * 4 * SK_ROW_TILES);  // [tile][d/32][32]
    rt->sk_pre_on = rt->q4 && skinny_supported(FL_QKV, n_qkv, d) &&
                    skinny_supported(FL_RESID, d, Hq * hd) &&
                    skinny_supported(FL_SWIGLU, 2 * F, d) && skinny_supported(FL_RESID, d, F);
    if (rt->sk_pre_on) {
      rt->sk_pre.alloc((size_t)2 * 32 * SK_ROW_TILES * d * 2);
      rt->sk_pre_xs.alloc((size_t)d * 4 * SK_ROW_TILES);
      rt->sk_pre_sc.alloc((size_t)2 * 32 * SK_ROW_TILES * 4);
    }
    rt->streaming = rt->q4 && stream_supported(32, n_qkv, d) && stream_supported(32, d, Hq * hd) &&
                 stream_supported(32, 2 * F, d) && stream_supported(32, d, F);
    if (rt->q4 && (M > 32 || rt->streaming)) {
      rt->act2.alloc((size_t)2 * M * widest * 2);
      size_t bf = 0;
      if (rt->streaming) {
        const int rows = std::min(M, 32);
        bf = std::max({stream_part_floats(rows, n_qkv, d, ST_QKV_MAX_KS),
                       stream_part_floats(rows, d, Hq * hd, BG_RESID_MAX_KS),
                       stream_part_floats(rows, 2 * F, d, 8),
                       stream_part_floats(rows, d, F, BG_RESID_MAX_KS)});
      }
      for (int mt = 1; mt <= (M + 127) / 128; ++mt) {
        const int rows = std::min(M, mt * 128);
        for (int K2 : {Hq * hd, F})
          bf = std::max(bf, (size_t)big_linear_splits(rows, d, K2, BG_RESID_MAX_KS) * rows * d);
        bf = std::max(bf, (size_t)big_linear_splits(rows, n_qkv, d, BG_QKV_MAX_KS) * rows * n_qkv);
      }
      // the gate|up projection's split last round shares the workspace (it runs
      // between the q|k|v and down projections, which use it too)
      int n_cu = 0;
      DRT_HIP(hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, rt->device));
      for (int mt = 1; mt <= (M + 127) / 128; ++mt)
        bf = std::max(bf, big_tail_part_floats(std::min(M, mt * 128), 2 * F, d, n_cu));
      rt->big_part_floats = bf;
      rt->big_part.alloc(bf * 4);
      rt->big_tail_count.alloc((size_t)BIG_TAIL_COUNTERS * 4);
      DRT_HIP(hipMemsetAsync(rt->big_tail_count.p, 0, rt->big_tail_count.bytes, s));
    }
    int nx = 1;
    if (hipDeviceGetAttribute(&nx, hipDeviceAttributeNumberOfXccs, rt->device) != hipSuccess)
      nx = 1;
    rt->n_xcc = std::max(1, nx);
    // DRT_N_XCC overrides the XCD count the split-K grids are laid out for (a
    // test hook: a wrong count must surface as the placement error); otherwise
    // one probe launch checks the round-robin placement, and where it does not
    // hold the split-K exchange runs fenced (DRT_SPLITK_FENCED=1 forces that).
    const char* nx_env = getenv("DRT_N_XCC");
    if (nx_env && atoi(nx_env) >= 1) {
      rt->n_xcc = atoi(nx_env);
    } else {
      DevBuf probe;
      probe.alloc(256 * sizeof(int));
      rt->fenced = !probe_round_robin(rt->n_xcc, probe.as<int>(), s);
    }
    if (getenv("DRT_SPLITK_FENCED") != nullptr) rt->fenced = true;
    rt->placement_err.alloc(4);
    DRT_HIP(hipMemsetAsync(rt->placement_err.p, 0, 4, s));
    DRT_HIP(hipHostMalloc((void**)&rt->placement_host, 4, hipHostMallocCoherent));
    *rt->placement_host = 0;
  }
  DRT_HIP(hipStreamSynchronize(s));
  size_t total = rt->embed.bytes + rt->final_norm.bytes + rt->lm_head.qw.bytes +
                 rt->lm_head.sb.bytes + rt->lm_head.wb.bytes + rt->hidden.bytes + rt->act.bytes +
                 rt->attn_part.bytes + rt->stats.bytes;
  for (auto& L : rt->layers)
    for (LinearW* w : {&L.qkv, &L.o, &L.gu, &L.down}) total += w->qw.bytes + w->sb.bytes + w->wb.bytes;
  if (e.creation_memory_budget_bytes > 0 && (int64_t)total > e.creation_memory_budget_bytes)
    fail(INVALID_ARGUMENT, "runtime needs " + std::to_string(total) +
                               " device bytes, above creation_memory_budget_bytes");
  return rt;
}

// ------------------------------------------------------------------ forward

// One forward over canvas rows [row0, row0 + n_rows) (absolute positions),
// attending keys [0, n_keys) of the session's cache. Writes every layer's K/V
// for these rows into the cache. If n_lm > 0, runs the final norm + LM head on
// the given row indices (relative to row0) and produces scores/tokens (and
// logits when `logits` is non-null).
struct ForwardArgs {
  const int32_t* tokens_dev = nullptr;  // device tokens of the whole canvas
  int row0 = 0, n_rows = 0, n_keys = 0;
  int mask_kind = 0, mask_prompt_len = 0, mask_block = 1;
  int n_lm = 0;
  std::vector<int32_t> lm_rows, lm_pos;  // host
  float* logits = nullptr;               // device [n_lm][V] or null
  float temperature = 0.f;
  uint64_t seed = 0;
  int step = 0;
  int exclude_col = -1;  // vocabulary column left out of the scores (-1: none)
  // rows [row0, row0 + seg_rows) form a first mask segment that sees only keys
  // [0, row0 + seg_rows) (a block committed with the next block's step; 0: none)
  int seg_rows = 0;
  int quota = 0;  // device-side block commit of this many proposals (0: none)
  // a device block's quotas indexed by step % QUOTA_TAB (host, QUOTA_TAB entries; null: zeros)
  const int32_t* quota_tab = nullptr;
};

// Rows [row0, row0 + n_rows) sit in one mask segment and see every key in
// [0, n_keys): the decode attention kernel applies.
bool one_segment(const ForwardArgs& a) {
  if (a.mask_kind == 0) return true;
  auto seg = [&](int p) { return p < a.mask_prompt_len ? -1 : (p - a.mask_prompt_len) / a.mask_block; };
  const int s0 = seg(a.row0), s1 = seg(a.row0 + a.n_rows - 1);
  if (s0 != s1) return false;
  const int seg_end = s0 < 0 ? a.mask_prompt_len : a.mask_prompt_len + (s0 + 1) * a.mask_block;
  return a.n_keys <= seg_end;
}

// Rows [row0, row0 + seg_rows) and the rest each sit in one mask segment, the
// first seeing keys up to its own end and the second every key in [0, n_keys),
// with the split on a query-tile boundary of the decode attention.
bool two_segments(const ForwardArgs& a, int G) {
  if (a.seg_rows <= 0 || a.seg_rows >= a.n_rows || (a.seg_rows * G) % 32) return false;
  ForwardArgs first, second;
  first.row0 = a.row0;
  first.n_rows = a.seg_rows;
  first.n_keys = a.row0 + a.seg_rows;
  second.row0 = a.row0 + a.seg_rows;
  second.n_rows = a.n_rows - a.seg_rows;
  second.n_keys = a.n_keys;
  for (ForwardArgs* f : {&first, &second}) {
    f->mask_kind = a.mask_kind;
    f->mask_prompt_len = a.mask_prompt_len;
    f->mask_block = a.mask_block;
  }
  return one_segment(first) && one_segment(second);
}



// Device addresses of one forward's inputs.
struct ForwardPtrs {
  const StepDesc* desc = nullptr;
  const int32_t* tokens_rel = nullptr;  // tokens of rows 0 .. n_rows-1 of this forward
  bool tokens_at_row0 = false;          // tokens_rel is the whole canvas: rows from desc->row0
  int32_t* canvas = nullptr;            // device canvas of the block commit (desc->quota)
  int mask_id = -1;
  const int32_t* lm_rows = nullptr;
  const int32_t* lm_pos = nullptr;
  int n_lm_launch = 0;  // LM rows launched (graph mode pads to 32)
  int ranges = 0;       // decode-attention ranges (0: from n_keys)
  // the block commit writes the next step's index and quota here (from quota_tab)
  StepDesc* advance = nullptr;
  const int32_t* quota_tab = nullptr;
};

// Upload the forward's descriptor and LM rows with one async copy from a pinned
// slot. slot < 0 takes the next eager slot. Graph forwards read their tokens from
// the device canvas at desc->row0; the slot's copy of the canvas rows is copied
// there first unless upload_tokens is false (the canvas rows were written on the
// device, by a block commit). dev_slot (>= 0) receives the slot's contents
// instead of the slot's own device copy (a graph's fixed descriptor). stage:
// STAGE_COPY writes the host slot and copies it; STAGE_HOST only writes it (the
// caller copies several adjacent slots at once); STAGE_PTRS leaves the host slot
// alone and only returns the pointers (the device slot holds or will hold these
// inputs: a device block's later steps, advanced by the block commit; a capture
// ahead of the slot's upload).
enum { STAGE_COPY = 0, STAGE_HOST = 1, STAGE_PTRS = 2 };
ForwardPtrs stage_forward(Runtime& rt, const ForwardArgs& a, int slot, bool graph_mode,
                          const int32_t* tokens_host, bool upload_tokens = true,
                          int dev_slot = -1, int stage = STAGE_COPY) {
  hipStream_t s = rt.stream;
  if (slot < 0) {
    if (rt.up_next >= Runtime::UPLOAD_SLOTS) {  // every slot in flight: drain first
      DRT_HIP(hipStreamSynchronize(s));
      rt.up_next = Runtime::EAGER_SLOT0;
    }
    slot = rt.up_next++;
  }
  Runtime::StepUpload* u = rt.up_host + slot;
  Runtime::StepUpload* d = rt.up_dev.as<Runtime::StepUpload>() + (dev_slot >= 0 ? dev_slot : slot);
  require(stage == STAGE_COPY || (graph_mode && !upload_tokens && a.n_lm <= 32),
          "only graph forwards of <= 32 LM rows stage a slot without copying it");
  Runtime::StepUpload scratch_slot;  // the writes below land here when the host slot is left alone
  if (stage == STAGE_PTRS) u = &scratch_slot;
  StepDesc& hd = u->desc;
  hd = StepDesc{};
  hd.row0 = a.row0;
  hd.n_rows = a.n_rows;
  hd.n_keys = a.n_keys;
  hd.n_lm = a.n_lm;
  hd.mask_kind = a.mask_kind;
  hd.mask_prompt_len = a.mask_prompt_len;
  hd.mask_block = a.mask_block;
  hd.step = a.step;
  hd.seed = a.seed;
  hd.temperature = a.temperature;
  hd.exclude_col = a.exclude_col;
  hd.seg_rows = a.seg_rows;
  hd.quota = a.quota;
  for (int i = 0; i < QUOTA_TAB; ++i) u->quotas[i] = a.quota_tab ? a.quota_tab[i] : 0;
  ForwardPtrs p;
  p.desc = &d->desc;
  p.quota_tab = d->quotas;
  if (a.n_lm <= 32) {
    const int n = graph_mode && a.n_lm > 0 ? 32 : a.n_lm;
    for (int i = 0; i < n; ++i) {
      // pad by repeating the last row (independent rows; padded results are unread)
      const int j = std::min(i, a.n_lm - 1);
      u->lm_rows[i] = a.lm_rows[j];
      u->lm_pos[i] = a.lm_pos[j];
    }
    p.lm_rows = d->lm_rows;
    p.lm_pos = d->lm_pos;
    p.n_lm_launch = n;
  } else {
    DRT_HIP(hipMemcpyAsync(rt.lm_rows.p, a.lm_rows.data(), a.n_lm * 4, hipMemcpyHostToDevice, s));
    DRT_HIP(hipMemcpyAsync(rt.lm_pos.p, a.lm_pos.data(), a.n_lm * 4, hipMemcpyHostToDevice, s));
    p.lm_rows = rt.lm_rows.as<int32_t>();
    p.lm_pos = rt.lm_pos.as<int32_t>();
    p.n_lm_launch = a.n_lm;
  }
  if (stage == STAGE_COPY)
    DRT_HIP(hipMemcpyAsync(d, u, sizeof(Runtime::StepUpload), hipMemcpyHostToDevice, s));
  if (graph_mode) {
    require(a.n_rows <= 64 && tokens_host && a.tokens_dev, "graph forwards take at most 64 rows");
    if (upload_tokens) {
      for (int i = 0; i < a.n_rows; ++i) u->tokens[i] = tokens_host[a.row0 + i];
      DRT_HIP(hipMemcpyAsync(const_cast<int32_t*>(a.tokens_dev) + a.row0, u->tokens,
                             (size_t)a.n_rows * 4, hipMemcpyHostToDevice, s));
    }
    p.tokens_rel = a.tokens_dev;
    p.tokens_at_row0 = true;
  } else {
    p.tokens_rel = a.tokens_dev + a.row0;
  }
  return p;
}

// The kernels of one forward (no host copies: capturable into a HIP graph when
// the shapes and pointers are fixed and every per-step value is in p.desc).
void launch_forward(Runtime& rt, void* kv, int64_t head_stride, int64_t layer_stride,
                    const ForwardArgs& a, const ForwardPtrs& p) {
  hipStream_t s = rt.stream;
  const int M = a.n_rows, d = rt.d(), Hq = rt.Hq(), Hkv = rt.Hkv();
  const int fmt = rt.fmt();
  const int G = Hq / Hkv;
  const float eps = rt.geo.rms_norm_eps;
  require(M >= 1 && M <= rt.max_rows, "forward rows exceed max_forward_rows");
  require(a.row0 + M <= rt.rope_positions, "positions exceed the rotary table");
  require(a.n_lm <= M, "more LM rows than forwarded rows");
  float* hidden = rt.hidden.as<float>();
  float* xs = rt.xsum.as<float>();
  // both cache dtypes are 2 bytes per element
  auto kv_layer = [&](int l) { return (void*)((char*)kv + (size_t)l * layer_stride * 2); };
  const StepDesc* desc = p.desc;

  const bool decode_attn = a.seg_rows > 0 ? M * G <= 128 && two_segments(a, G)
                                           : M * G <= 64 && one_segment(a);
  AttnPlan ap;
  int ranges = 1;
  size_t apb;
  if (decode_attn) {
    ranges = p.ranges > 0 ? p.ranges : attention_decode_ranges(a.n_keys, Hkv);
    apb = attention_decode_part_bytes(ranges, Hkv, M * G);
  } else {
    ap = plan_attention(M, Hq, Hkv, a.n_keys, rt.attn_part_budget);
    apb = attention_part_bytes(ap, M, Hq, Hkv);
  }
  require(apb <= rt.attn_part.bytes, "attention partials exceed the workspace");
  const int splits = decode_attn ? ranges : ap.splits;
  float* o_part = rt.attn_part.as<float>();
  float* ml_part = o_part + (size_t)splits * Hkv * M * G * 128;

  // forwards of up to SK_ROW_TILES 32-row tiles use the split-K linears, which
  // carry the RMSNorm row statistics from each residual update to the next norm
  float* ss = M <= 32 * SK_ROW_TILES ? rt.sk_ss.as<float>() : nullptr;
  // longer q4 forwards use the large-M kernels: each linear reads an ACT_F16P
  // activation, the RMSNorms run as their own passes, fused with the split-K
  // reduce and residual add of the projection before them
  const bool big = rt.q4 && M > 32 * SK_ROW_TILES;
  // <= 32-row forwards of 7B-class layers: the weight-streaming linears (fp32 K
  // slices, reduced by small passes: residual add + row statistics, q|k|v
  // epilogue, SwiGLU; the RMSNorms run inside the next linear's staging)
  const bool stream = !big && rt.streaming && M <= 32;
  const bool pipe = big || stream;
  float* bpart = pipe ? rt.big_part.as<float>() : nullptr;
  const int L = (int)rt.layers.size();
  // q4 on the split-K linears: each residual update (and the embedding) also
  // writes the next RMSNorm's input pre-scaled (FusedArgs::pre_out), which the
  // q|k|v and gate|up kernels stage without normalising
  const bool pre = rt.sk_pre_on && ss && !big && !stream && L > 0;
  uint16_t* pre_planes = pre ? rt.sk_pre.as<uint16_t>() : nullptr;
  float* pre_xs = pre ? rt.sk_pre_xs.as<float>() : nullptr;
  float* sc_a = pre ? rt.sk_pre_sc.as<float>() : nullptr;  // written by q|k|v
  float* sc_b = pre ? sc_a + 32 * SK_ROW_TILES : nullptr;  // by gate|up and the embedding
  {
    PreOut po;
    if (pre) {
      po.norm = rt.layers[0].in_norm.as<uint16_t>();
      po.eps = eps;
      po.planes = pre_planes;
      po.xs = pre_xs;
      po.sc = sc_b;
      po.err = rt.placement_err.as<int>();
    }
    embed(p.tokens_rel, rt.embed.as<uint16_t>(), hidden, M, d, ss, s,
          p.tokens_at_row0 ? desc : nullptr, pre ? &po : nullptr);
  }
  if (big && L > 0)
    residual_norm(hidden, nullptr, 0, M, false, nullptr, false,
                  rt.layers[0].in_norm.as<uint16_t>(), eps, d, ACT_F16P, rt.act.p, xs, M, s,
                  rt.placement_err.as<int>());
  // split-K projection (o_proj / down_proj) into partial slices, then
  // hidden += sum of the slices and the next norm's activation
  // fp32 K slices of a projection into bpart (the streaming or the large-M
  // kernels); returns the slice count
  auto slices = [&](FusedArgs f, int max_ks) {
    f.bias = nullptr;  // added by the reduce pass
    f.y = bpart;
    if (stream) {
      const StreamPlan sp = stream_plan(M, f.N, f.K, max_ks);
      require(sp.KS >= 1 && (size_t)sp.KS * M * f.N <= rt.big_part_floats,
              "streaming linear: no plan or partials exceed the workspace");
      stream_linear(f, sp, s);
      return sp.KS;
    }
    const int ks = big_linear_splits(M, f.N, f.K, max_ks);
    require((size_t)ks * M * f.N <= rt.big_part_floats, "large-M partials exceed the workspace");
    big_linear(f, FL_STORE, ks, s);
    return ks;
  };
  auto big_resid = [&](FusedArgs f, const uint16_t* next_norm) {
    require(f.bias == nullptr, "o_proj / down_proj bias is not supported on this path");
    const int ks = slices(f, BG_RESID_MAX_KS);
    residual_norm(hidden, bpart, ks, M, false, nullptr, true, next_norm, eps, d, ACT_F16P,
                  rt.act.p, xs, M, s, rt.placement_err.as<int>());
  };
  for (int l = 0; l < L; ++l) {
    LayerW& w = rt.layers[l];
    auto base = [&](const LinearW& lw) {
      FusedArgs f;
      f.qw = lw.q4 ? lw.qw.as<uint32_t>() : nullptr;
      f.sb = lw.q4 ? lw.sb.as<uint32_t>() : nullptr;
      f.wb = lw.q4 ? nullptr : lw.wb.as<uint16_t>();
      f.bias = lw.bias.as<uint16_t>();
      f.M = M;
      f.N = lw.N;
      f.K = lw.K;
      f.eps = eps;
      f.rnd_bf16 = !rt.q4;
      f.desc = desc;
      f.part = rt.sk_part.as<float>();  // bf16 weights: single-pass kernels
      f.part_floats = rt.sk_part_floats;
      f.counters = rt.sk_counters.as<int>();
      f.n_counters = rt.sk_n_counters;
      f.sk_row_tiles = SK_ROW_TILES;
      f.n_xcc = rt.n_xcc;
      f.fenced = rt.fenced ? 1 : 0;
      f.placement_err = rt.placement_err.as<int>();
      return f;
    };
    {  // input RMSNorm -> fused q|k|v -> q/k norm + RoPE -> Q, K/V cache
      FusedArgs f = base(w.qkv);
      f.hidden = hidden;
      f.norm_w = w.in_norm.as<uint16_t>();
      f.q_norm = w.q_norm.as<uint16_t>();
      f.k_norm = w.k_norm.as<uint16_t>();
      f.rope_cos = rt.rope_cos.as<float>();
      f.rope_sin = rt.rope_sin.as<float>();
      f.q_out = rt.qbuf.p;
      f.kv_layer = kv_layer(l);
      f.kv_head_stride = head_stride;
      f.Hq = Hq;
      f.Hkv = Hkv;
      f.kv_bf16 = rt.kv_bf16;
      f.ss_in = ss;
      if (pre) {
        f.act = pre_planes;
        f.act_xsum = pre_xs;
        f.pre_sc_in = sc_b;
        f.pre_sc_out = sc_a;
      }
      if (big) {
        f.act = rt.act.p;
        big_qkv(f, bpart, rt.big_part_floats, s);
      } else if (stream) {  // normed from the residual stream while staged
        qkv_epilogue_slices(f, bpart, slices(f, ST_QKV_MAX_KS), s);
      } else {
        fused_linear(f, FL_QKV, s);
      }
    }
    const bool last = l == L - 1;
    // commit-only forward: the last layer's K/V is written by its q|k|v epilogue;
    // nothing after it is read
    if (last && a.n_lm == 0) break;
    if (decode_attn)
      attention_decode(rt.kv_bf16, rt.qbuf.p, kv_layer(l), head_stride, M, Hq, Hkv, a.n_keys, desc,
                       ranges, o_part, rt.act.p, xs, fmt, s, rt.placement_err.as<int>());
    else
      attention(rt.kv_bf16, rt.qbuf.p, kv_layer(l), head_stride, M, Hq, Hkv, a.n_keys, a.row0,
                a.mask_kind, a.mask_prompt_len, a.mask_block, ap, o_part, ml_part, rt.act.p, xs,
                fmt, s, rt.placement_err.as<int>());
    if (stream) {
      // o_proj slices -> hidden += (+ the row statistics of the next norm)
      FusedArgs fo = base(w.o);
      require(fo.bias == nullptr, "o_proj bias is not supported on this path");
      fo.act = rt.act.p;
      residual_slices(bpart, slices(fo, BG_RESID_MAX_KS), M, d, hidden, ss, s);
      // post-attention RMSNorm (while staged) -> gate|up slices -> SwiGLU
      FusedArgs fg = base(w.gu);
      require(fg.bias == nullptr, "gate|up bias is not supported on this path");
      fg.hidden = hidden;
      fg.norm_w = w.post_norm.as<uint16_t>();
      fg.ss_in = ss;
      swiglu_slices(bpart, slices(fg, 8), M, fg.N, rt.act2.p, rt.placement_err.as<int>(), s);
      // down_proj slices -> hidden +=
      FusedArgs fd = base(w.down);
      require(fd.bias == nullptr, "down_proj bias is not supported on this path");
      fd.act = rt.act2.p;
      residual_slices(bpart, slices(fd, BG_RESID_MAX_KS), M, d, hidden, ss, s);
      continue;
    }
    if (big) {
      FusedArgs fo = base(w.o);
      fo.act = rt.act.p;
      big_resid(fo, w.post_norm.as<uint16_t>());  // act = post-attention norm
      FusedArgs fg = base(w.gu);
      fg.act = rt.act.p;
      fg.act_out = rt.act2.p;
      fg.act_fmt = ACT_F16P;
      big_linear(fg, FL_SWIGLU, 1, s, bpart, rt.big_part_floats, rt.big_tail_count.as<int>(),
                 BIG_TAIL_COUNTERS);
      FusedArgs fd = base(w.down);
      fd.act = rt.act2.p;
      big_resid(fd, last ? nullptr : rt.layers[l + 1].in_norm.as<uint16_t>());
      continue;
    }
    {  // o_proj + residual
      FusedArgs f = base(w.o);
      f.act = rt.act.p;
      f.act_xsum = xs;
      f.hidden_out = hidden;
      f.ss_out = ss;
      if (pre) {
        f.pre_out = pre_planes;
        f.pre_xs_out = pre_xs;
        f.pre_norm = w.post_norm.as<uint16_t>();
        f.pre_sc = sc_a;
      }
      fused_linear(f, FL_RESID, s);
    }
    {  // post-attention RMSNorm -> [gate | up] -> SwiGLU -> down activation
      FusedArgs f = base(w.gu);
      f.hidden = hidden;
      f.norm_w = w.post_norm.as<uint16_t>();
      f.act_out = rt.act.p;
      f.xsum_out = xs;
      f.act_fmt = fmt;
      f.ss_in = ss;
      if (pre) {
        f.act = pre_planes;
        f.act_xsum = pre_xs;
        f.pre_sc_in = sc_a;
        f.pre_sc_out = sc_b;
      }
      fused_linear(f, FL_SWIGLU, s);
    }
    {  // down_proj + residual
      FusedArgs f = base(w.down);
      f.act = rt.act.p;
      f.act_xsum = xs;
      f.hidden_out = hidden;
      f.ss_out = ss;
      if (pre && !last) {
        f.pre_out = pre_planes;
        f.pre_xs_out = pre_xs;
        f.pre_norm = rt.layers[l + 1].in_norm.as<uint16_t>();
        f.pre_sc = sc_b;
      }
      fused_linear(f, FL_RESID, s);
    }
  }
  if (a.n_lm > 0) {
    residual_norm(hidden, nullptr, 0, M, false, p.lm_rows, false, rt.final_norm.as<uint16_t>(),
                  eps, d, fmt, rt.act_lm.p, rt.xsum_lm.as<float>(), p.n_lm_launch, s,
                  rt.placement_err.as<int>());
    lmhead(rt.lm_head, rt.act_lm.p, rt.xsum_lm.as<float>(), p.n_lm_launch, a.logits, rt.stats.p,
           a.temperature, a.seed, a.step, p.lm_pos, rt.scores_host(), rt.tokens_host(), s, desc,
           a.exclude_col, rt.placement_err.as<int>(), rt.placement_host,
           rt.lm_scores_d.as<double>(), rt.lm_tokens_d.as<int32_t>());
    if (p.canvas && desc)
      block_commit(rt.lm_scores_d.as<double>(), rt.lm_tokens_d.as<int32_t>(), p.lm_pos, p.canvas,
                   p.mask_id, desc, s, p.advance, p.quota_tab);
  }
}

// The split-K linears rely on work-group i running on XCD i % n_xcc; a kernel
// that observed otherwise left a flag (read back with the forward's results).
// Bit 2 of the same flag: a wave of the decode attention gave up waiting for a K/V
// tile (its bounded wait ran out), so that forward's attention is not valid.
void check_placement(const Runtime& rt) {
  // the placement first: a split-K exchange across XCDs produces garbage, which
  // may also trip the other two checks
  const int e = *rt.placement_host;
  if (e & 1)
    fail(INTERNAL_ERROR,
         "a split-K linear ran on an unexpected XCD (work-group placement is not the "
         "round-robin the kernels assume); results of this runtime are not valid");
  if (e & 2)
    fail(INTERNAL_ERROR,
         "decode attention: a bounded wait for a K/V tile expired; results of this runtime "
         "are not valid");
  if (e & DRT_ERR_F16_RANGE)
    fail(INTERNAL_ERROR,
         "an activation, Q, K or V value exceeded the fp16 range (|x| >= 65504); results of "
         "this forward are not valid");
  if (e != 0) fail(INTERNAL_ERROR, "a kernel reported an unknown error word");
}

void run_forward(Runtime& rt, void* kv, int64_t head_stride, int64_t layer_stride,
                 const ForwardArgs& a) {
  const ForwardPtrs p = stage_forward(rt, a, -1, false, nullptr);
  launch_forward(rt, kv, head_stride, layer_stride, a, p);
}

// ------------------------------------------------------------------ session

struct Session {
  std::shared_ptr<Runtime> rt;
  drt_session_config cfg{};
  bool started = false;
  std::vector<int32_t> canvas;
  DevBuf tokens_dev;
  DevBuf kv;
  int tile_cap = 0;
  int64_t head_stride = 0, layer_stride = 0;
  int origin = 0, block = 32, mask_id = 0, steps = 0;
  double temperature = 0.0;
  uint64_t seed = 0;
  int cache_len = 0;  // rows [0, cache_len) hold exact K/V of the current canvas
  int proposals = 0;
  // execute_window identity of the cached prefix
  int win_prompt_len = -1, win_block = -1;
  // Under the Dream logits shift the first position of a d2f block reads the
  // last row before the block, which is frozen: its score and token stay fixed
  // while the block decodes, so they are computed once (a one-row forward with
  // the LM head) and kept here for position feeder_pos (-1: none).
  int feeder_pos = -1;
  double feeder_score = 0.0;
  int32_t feeder_token = 0;
  // the native BD3 fixed-quota loop (drt_session_bd3_decode): its policy state
  struct Bd3Loop {
    bool on = false;
    int prompt_len = 0, gen = 0, steps = 0, eos = 0, spb = 0, count = 0, limit = 0;
    bool align = true;
    int step = 0, active = -1, base = 0, rem = 0;
  } loop;
  std::vector<int32_t> win_tokens;
  drt_metrics m{};
  Profiler prof;
  // HIP graphs of the fixed-shape forwards of a block-diffusion decode: the
  // commit of one finished block, the denoise step of the active block, and the
  // two together (a block's first step after the block before it finished).
  // G_BLOCK: a whole block of the native loop, the merged commit + step forward
  // then g_block_n - 1 step forwards on the step slot (each advanced on the
  // device by the step before), replayed with one launch per block.
  enum GraphKind { G_COMMIT = 0, G_STEP = 1, G_PAIR = 2, G_BLOCK = 3, G_KINDS = 4 };
  hipGraphExec_t g_exec[G_KINDS] = {nullptr, nullptr, nullptr, nullptr};
  bool g_warm[G_KINDS] = {false, false, false, false};
  int g_block_n = 0;
  // forwards with a quota in a whole block of the native loop (0: unknown)
  int full_block_steps = 0;
  int g_ranges = 0;
  bool use_graphs = getenv("DRT_DISABLE_GRAPHS") == nullptr;
  // DRT_SEPARATE_COMMIT=1 keeps the commit forward of a finished block apart
  // from the next step (an A/B switch for parity and timing comparisons)
  bool pair_commit = getenv("DRT_SEPARATE_COMMIT") == nullptr;

  void drop_graphs() {
    for (int k = 0; k < G_KINDS; ++k) {
      if (g_exec[k]) (void)hipGraphExecDestroy(g_exec[k]);
      g_exec[k] = nullptr;
      g_warm[k] = false;
    }
  }
  ~Session() {
    if (rt && rt->stream) (void)hipStreamSynchronize(rt->stream);
    drop_graphs();
    for (QueuedBlock& q : qblk) {
      if (q.t0) (void)hipEventDestroy(q.t0);
      if (q.t1) (void)hipEventDestroy(q.t1);
      if (q.done) (void)hipEventDestroy(q.done);
      if (q.tokens) (void)hipHostFree(q.tokens);
    }
  }

  // Run a <= 64-row forward whose inputs live in a fixed upload slot: eager the
  // first time (grants kernel attributes), captured into a graph the second
  // time, replayed afterwards. The step forwards end with the device-side block
  // commit (a no-op unless the descriptor carries a quota). host_slot >= 0: the
  // inputs are staged in that pinned slot (a block's steps queued without a
  // synchronisation keep one slot each) and copied to the graph's own.
  // upload false: the graph's slot already holds this step's inputs (a device
  // block's step after another step forward, whose block commit advanced the
  // slot's step and quota).
  void graph_forward(GraphKind kind, const ForwardArgs& a, int host_slot = -1,
                     bool upload_tokens = true, bool upload = true) {
    Runtime& r = *rt;
    hipGraphExec_t& exec = g_exec[kind];
    bool& warm = g_warm[kind];
    const ForwardPtrs p =
        graph_ptrs(kind, a, host_slot, upload_tokens, upload ? STAGE_COPY : STAGE_PTRS);
    if (!warm) {
      launch_forward(r, kv.p, head_stride, layer_stride, a, p);
      warm = true;
      return;
    }
    if (!exec) capture_into(exec, a, p);
    DRT_HIP(hipGraphLaunch(exec, r.stream));
  }

  // Stage a graph forward's inputs in the slot of its kind (see graph_forward)
  // and return its device pointers.
  ForwardPtrs graph_ptrs(GraphKind kind, const ForwardArgs& a, int host_slot, bool upload_tokens,
                         int stage) {
    ForwardPtrs p = stage_forward(*rt, a, host_slot >= 0 ? host_slot : (int)kind, true,
                                  canvas.data(), upload_tokens, host_slot >= 0 ? (int)kind : -1,
                                  stage);
    if (kind != G_COMMIT) {
      p.canvas = tokens_dev.as<int32_t>();
      p.mask_id = mask_id;
    }
    // a step forward's block commit sets up its own slot for the step after it
    if (kind == G_STEP) p.advance = const_cast<StepDesc*>(p.desc);
    p.ranges = g_ranges;
    return p;
  }

  // The inputs of step j of the native loop's block [fp, fp + block): the first
  // step of a paired block also commits the block before it.
  ForwardArgs block_step(int fp, int j, bool pair, int quota, const int32_t* quota_tab) const {
    ForwardArgs a;
    a.tokens_dev = tokens_dev.as<int32_t>();
    a.temperature = (float)temperature;
    a.seed = seed;
    a.step = proposals + j;
    a.row0 = j == 0 && pair ? fp - block : fp;
    a.n_rows = fp + block - a.row0;
    a.n_keys = fp + block;
    a.mask_kind = 1;
    a.mask_prompt_len = origin;
    a.mask_block = block;
    a.seg_rows = a.row0 < fp ? block : 0;
    a.quota = quota;
    a.quota_tab = quota_tab;
    for (int p = fp; p < fp + block; ++p) {
      a.lm_rows.push_back(p - a.row0);
      a.lm_pos.push_back(p);
    }
    a.n_lm = block;
    return a;
  }

  // Record the kernels of one forward into an instantiated graph (nothing runs).
  void capture_into(hipGraphExec_t& exec, const ForwardArgs& a, const ForwardPtrs& p) {
    capture_with(exec, [&] { launch_forward(*rt, kv.p, head_stride, layer_stride, a, p); });
  }

  // Record what `record` launches on the session stream into an instantiated graph.
  template <class F> void capture_with(hipGraphExec_t& exec, F&& record) {
    Runtime& r = *rt;
    hipGraph_t g = nullptr;
    DRT_HIP(hipStreamBeginCapture(r.stream, hipStreamCaptureModeThreadLocal));
    try {
      record();
    } catch (...) {
      (void)hipStreamEndCapture(r.stream, &g);
      if (g) (void)hipGraphDestroy(g);
      throw;
    }
    DRT_HIP(hipStreamEndCapture(r.stream, &g));
    const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    DRT_HIP(e);
  }

  // The merged commit + step forward of the block starting at next_fp (its
  // first step commits [next_fp - block, next_fp)), captured ahead of its first
  // use while the steps already queued run: a capture records and executes
  // nothing, so that first use replays it instead of running eagerly and then
  // capturing on the host's time in the middle of a decode. Its descriptor slot
  // is its own (written before every replay); the upload here lands after the
  // queued steps, in stream order.
  void precapture_pair(int next_fp) {
    Runtime& r = *rt;
    const int hi = next_fp + block;
    if (!use_graphs || prof.on || !pairable() || !graphable(block) || g_exec[G_PAIR] ||
        next_fp < block || hi > (int)canvas.size() || hi > r.rope_positions)
      return;
    ForwardArgs a;
    a.tokens_dev = tokens_dev.as<int32_t>();
    a.temperature = (float)temperature;
    a.seed = seed;
    a.step = proposals;
    a.row0 = next_fp - block;
    a.n_rows = 2 * block;
    a.n_keys = hi;
    a.mask_kind = 1;
    a.mask_prompt_len = origin;
    a.mask_block = block;
    a.seg_rows = block;
    a.quota = 0;
    for (int q = next_fp; q < hi; ++q) {
      a.lm_rows.push_back(q - a.row0);
      a.lm_pos.push_back(q);
    }
    a.n_lm = block;
    ForwardPtrs p = stage_forward(r, a, (int)G_PAIR, true, canvas.data(), false, (int)G_PAIR);
    p.canvas = tokens_dev.as<int32_t>();
    p.mask_id = mask_id;
    p.ranges = g_ranges;
    // an optimisation only: if the capture fails, the first use takes the usual
    // path (eager, then captured), which reports an error that persists
    try {
      capture_into(g_exec[G_PAIR], a, p);
      g_warm[G_PAIR] = true;
    } catch (const std::exception&) {
      (void)hipGetLastError();
      g_exec[G_PAIR] = nullptr;
    }
  }

  // A whole paired block of n steps as one graph (G_BLOCK), captured ahead of
  // its first use like the merged step above, once the pair and step forwards
  // have each run (their kernels' attributes granted). Its slots (the pair's and
  // the step's) are uploaded before each replay; nothing is staged here.
  void precapture_block(int next_fp, int n) {
    Runtime& r = *rt;
    const int hi = next_fp + block;
    if (!use_graphs || prof.on || !pairable() || !graphable(block) || g_exec[G_BLOCK] ||
        !g_warm[G_PAIR] || !g_warm[G_STEP] || n < 2 ||
        n > Runtime::UPLOAD_SLOTS - Runtime::EAGER_SLOT0 || next_fp < block ||
        hi > (int)canvas.size() || hi > r.rope_positions)
      return;
    const ForwardArgs a0 = block_step(next_fp, 0, true, 0, nullptr);
    const ForwardArgs a1 = block_step(next_fp, 1, true, 0, nullptr);
    const ForwardPtrs p0 = graph_ptrs(G_PAIR, a0, -1, false, STAGE_PTRS);
    const ForwardPtrs p1 = graph_ptrs(G_STEP, a1, -1, false, STAGE_PTRS);
    try {  // an optimisation only, as above: on failure the blocks replay step by step
      capture_with(g_exec[G_BLOCK], [&] {
        launch_forward(r, kv.p, head_stride, layer_stride, a0, p0);
        for (int j = 1; j < n; ++j) launch_forward(r, kv.p, head_stride, layer_stride, a1, p1);
      });
      g_block_n = n;
    } catch (const std::exception&) {
      (void)hipGetLastError();
      g_exec[G_BLOCK] = nullptr;
    }
  }

  // Commit forwards for the rows [cache_len, frozen_prefix) (exact prefix K/V):
  // block by block through the commit graph for up to four aligned blocks, else
  // in max_forward_rows chunks. Returns the rows committed.
  int commit_to(int frozen_prefix) {
    Runtime& r = *rt;
    if (cache_len >= frozen_prefix) return 0;
    const int todo = frozen_prefix - cache_len;
    const bool by_block = graphable(block) && origin == 0 && cache_len % block == 0 &&
                          todo % block == 0 && todo <= 4 * block;
    if (by_block) {
      for (int b = cache_len; b < frozen_prefix; b += block) {
        ForwardArgs c;
        c.tokens_dev = tokens_dev.as<int32_t>();
        c.row0 = b;
        c.n_rows = block;
        c.n_keys = b + block;
        c.mask_kind = 1;
        c.mask_prompt_len = origin;
        c.mask_block = block;
        graph_forward(G_COMMIT, c);
        if (b + block < frozen_prefix) DRT_HIP(hipStreamSynchronize(r.stream));  // slot reuse
        m.commit_rows += block;
      }
    } else {
      upload_tokens(cache_len, frozen_prefix);
      commit_rows(cache_len, frozen_prefix, origin, block);
    }
    cache_len = frozen_prefix;
    return todo;
  }

  // One block [fp, fp + block) of the native BD3 loop with no host
  // synchronisation between its steps: the commit of what precedes it (merged
  // into the first step when pairable), then one graph-replayed step forward per
  // quota, each ending in the device-side choice and commit of its quota into the
  // device canvas (a whole paired block replays as one graph). Every LM row of
  // the block is scored (graph forwards score 32 rows either way); the rows
  // already committed are left out of the choice. queue_block enqueues the block
  // and the readback of its tokens (into pinned staging); finish_block waits for
  // them and accounts the block, so that the loop can queue the next block ahead
  // while this one runs; discard_block drops a block queued ahead that the loop
  // does not run after all (an end token or a full canvas stops the decode at
  // the boundary before it).
  struct QueuedBlock {
    bool on = false, pair = false;
    int fp = 0, S = 0;
    std::vector<int> quotas;
    int cache_len_before = 0;
    int64_t commit_rows_before = 0;
    hipEvent_t t0 = nullptr, t1 = nullptr, done = nullptr;
    int32_t* tokens = nullptr;  // pinned, block entries
  };
  QueuedBlock qblk[2];
  int qblk_next = 0;  // the QueuedBlock (and half of the eager slots) the next queue takes
  // eager upload slots per queued block: two blocks in flight take disjoint halves
  static constexpr int QB_SLOTS = (Runtime::UPLOAD_SLOTS - Runtime::EAGER_SLOT0) / 2;

  QueuedBlock& queue_block(int fp, const std::vector<int>& quotas, bool upload_canvas) {
    Runtime& r = *rt;
    const int hi = fp + block, S = (int)quotas.size();
    QueuedBlock& q = qblk[qblk_next];
    require(!q.on, "internal: a queued block's record is still in use");
    require(S >= 1 && Runtime::EAGER_SLOT0 + S <= Runtime::UPLOAD_SLOTS,
            "a device block takes 1..61 steps");
    // a block of more steps than half the slots takes them all (nothing else queued)
    require(S <= QB_SLOTS || !other_queued(q), "internal: a long block queued behind another");
    const int slot0 = Runtime::EAGER_SLOT0 + (S <= QB_SLOTS ? qblk_next * QB_SLOTS : 0);
    if (!q.done) {
      DRT_HIP(hipEventCreate(&q.t0));
      DRT_HIP(hipEventCreate(&q.t1));
      DRT_HIP(hipEventCreate(&q.done));
      DRT_HIP(hipHostMalloc((void**)&q.tokens, (size_t)block * 4, hipHostMallocDefault));
    }
    q.fp = fp;
    q.S = S;
    q.quotas = quotas;
    q.cache_len_before = cache_len;
    q.commit_rows_before = m.commit_rows;
    DRT_HIP(hipEventRecord(q.t0, r.stream));
    q.pair = pairable() && cache_len + block == fp && cache_len % block == 0;
    if (!q.pair) {
      require(!other_queued(q), "internal: an unpaired block queued behind another");
      commit_to(fp);
      // commit forwards run eagerly (a prefix longer than four blocks) staged their
      // descriptors in the eager slots that the steps below rewrite: their copies
      // must have left those slots first
      if (r.up_next != Runtime::EAGER_SLOT0) {
        DRT_HIP(hipStreamSynchronize(r.stream));
        r.up_next = Runtime::EAGER_SLOT0;
      }
    }
    // the device canvas is the forwards' from here on (a block queued behind
    // another finds its rows there: the earlier block's written on the device,
    // its own still masked on both sides)
    if (upload_canvas) upload_tokens(q.pair ? fp - block : fp, hi);
    // the quotas by step: the first step forward's upload carries them, and each
    // step's block commit writes the next step's index and quota into the slot
    int32_t quota_tab[QUOTA_TAB] = {};
    for (int j = 0; j < S; ++j) quota_tab[(proposals + j) & (QUOTA_TAB - 1)] = quotas[j];
    if (q.pair && S == g_block_n && g_exec[G_BLOCK]) {
      // the whole block in one launch: the step slot (the first step forward
      // after the pair) and the pair's slot, adjacent on both sides, in one copy
      static_assert(G_PAIR == G_STEP + 1, "the step and pair slots are adjacent");
      const ForwardArgs a0 = block_step(fp, 0, true, quotas[0], quota_tab);
      const ForwardArgs a1 = block_step(fp, 1, true, quotas[1], quota_tab);
      (void)graph_ptrs(G_STEP, a1, slot0, false, STAGE_HOST);
      (void)graph_ptrs(G_PAIR, a0, slot0 + 1, false, STAGE_HOST);
      DRT_HIP(hipMemcpyAsync(r.up_dev.as<Runtime::StepUpload>() + G_STEP, r.up_host + slot0,
                             2 * sizeof(Runtime::StepUpload), hipMemcpyHostToDevice, r.stream));
      DRT_HIP(hipGraphLaunch(g_exec[G_BLOCK], r.stream));
    } else {
      for (int j = 0; j < S; ++j) {
        const ForwardArgs a = block_step(fp, j, q.pair, quotas[j], quota_tab);
        const GraphKind kind = a.seg_rows > 0 ? G_PAIR : G_STEP;
        const bool after_step = j > 0 && kind == G_STEP && (j > 1 || !q.pair);
        graph_forward(kind, a, slot0 + j, false, !after_step);
      }
    }
    if (!other_queued(q)) {  // (with a block in flight the graphs exist already)
      precapture_pair(hi);  // the next block's first step, while these run
      if (full_block_steps > 0) precapture_block(hi, full_block_steps);
    }
    if (q.pair) {
      m.commit_rows += block;
      cache_len = fp;
    }
    DRT_HIP(hipEventRecord(q.t1, r.stream));
    DRT_HIP(hipMemcpyAsync(q.tokens, tokens_dev.as<int32_t>() + fp, (size_t)block * 4,
                           hipMemcpyDeviceToHost, r.stream));
    DRT_HIP(hipEventRecord(q.done, r.stream));
    proposals += S;  // a block queued behind this one continues the sampling index
    q.on = true;
    qblk_next ^= 1;
    return q;
  }

  bool other_queued(const QueuedBlock& q) const { return qblk[&q == &qblk[0] ? 1 : 0].on; }

  // A block may be queued behind another: every graph it replays is captured
  // (whole paired blocks), and nothing else is queued ahead.
  bool queue_ahead_ready() const {
    return use_graphs && !prof.on && pairable() && graphable(block) && g_exec[G_PAIR] &&
           g_exec[G_STEP] && g_exec[G_BLOCK] && !qblk[0].on != !qblk[1].on;
  }

  // The block queued ahead at fp, or null.
  QueuedBlock* queued_at(int fp) {
    for (QueuedBlock& q : qblk)
      if (q.on && q.fp == fp) return &q;
    return nullptr;
  }

  // Wait for a queued block's tokens and account it. Returns its forwards.
  int finish_block(QueuedBlock& q) {
    Runtime& r = *rt;
    DRT_HIP(hipEventSynchronize(q.done));
    std::memcpy(canvas.data() + q.fp, q.tokens, (size_t)block * 4);
    q.on = false;
    if (!other_queued(q)) r.up_next = Runtime::EAGER_SLOT0;
    check_placement(r);
    float ms = 0.f;
    DRT_HIP(hipEventElapsedTime(&ms, q.t0, q.t1));
    m.last_forward_ms = ms;
    m.total_forward_ms += ms;
    m.forward_count += q.S;
    m.active_rows += (int64_t)q.S * block;
    m.lm_rows += (int64_t)q.S * block;
    m.kv_cache_len = cache_len;
    return q.S;
  }

  // Drop a block queued ahead: drain the stream, put its rows of the device
  // canvas back to the host's (still masked) and undo its accounting. The
  // commit its first step made (the block before it) stays on the device, not
  // counted: those K/V rows are exact, and a later commit rewrites them.
  void discard_block(QueuedBlock& q) {
    Runtime& r = *rt;
    DRT_HIP(hipStreamSynchronize(r.stream));
    q.on = false;
    upload_tokens(q.fp, q.fp + block);
    DRT_HIP(hipStreamSynchronize(r.stream));
    proposals -= q.S;
    cache_len = q.cache_len_before;
    m.commit_rows = q.commit_rows_before;
    m.kv_cache_len = cache_len;
    if (!other_queued(q)) r.up_next = Runtime::EAGER_SLOT0;
    check_placement(r);
  }

  // Drop whatever is queued ahead (the loop stops, or runs something else next).
  void discard_queued() {
    for (QueuedBlock& q : qblk)
      if (q.on) discard_block(q);
  }

  // Graph forwards apply to block-sized rows of a session whose decode
  // attention covers the whole block (block rows x GQA group <= 64 vectors).
  bool graphable(int rows) const {
    const Runtime& r = *rt;
    return use_graphs && !prof.on && rows == block && rows <= 32 &&
           rows * (r.Hq() / r.Hkv()) <= 64;
  }

  // The native loop runs whole blocks on the device (graph forwards, no
  // profiling); other blocks take the per-step host choice.
  bool block_on_device() const {
    return graphable(block) && origin == 0;
  }

  // A block's commit can run with the next block's step as one forward when
  // both blocks fit the decode attention's 128 query vectors, the split falls
  // on a query tile, and the rows fit the split-K linears' row tiles.
  bool pairable() const {
    const Runtime& r = *rt;
    const int G = r.Hq() / r.Hkv();
    return pair_commit && origin == 0 && 2 * block <= std::min(r.max_rows, 32 * SK_ROW_TILES) &&
           2 * block * G <= 128 && (block * G) % 32 == 0;
  }

  void publish_profile() {
    prof.collect();
    for (int c = 0; c < Profiler::NCLASS; ++c) {
      m.prof_ms[c] = prof.ms[c];
      m.prof_bytes[c] = prof.bytes[c];
      m.prof_launches[c] = prof.launches[c];
    }
  }

  // Grow the cache to hold n_tokens rows. Existing tiles keep their contents
  // (copied head by head), so a longer window does not lose the exact prefix.
  void ensure_cache(int n_tokens) {
    const int want = std::max(n_tokens, cfg.max_tokens);
    const int tiles = (want + 31) / 32;
    if (tiles <= tile_cap) return;
    const Runtime& r = *rt;
    const int64_t new_head = (int64_t)tiles * 8192;
    const size_t rows = r.layers.size() * (size_t)r.Hkv();
    DevBuf grown;
    grown.alloc(rows * new_head * 2);
    // Zero once: partially filled tiles are multiplied by exactly-zero
    // probabilities, and 0 * NaN from stale bits would poison the sums.
    DRT_HIP(hipMemsetAsync(grown.p, 0, grown.bytes, r.stream));
    if (kv.p && tile_cap > 0)
      DRT_HIP(hipMemcpy2DAsync(grown.p, new_head * 2, kv.p, head_stride * 2, head_stride * 2,
                               rows, hipMemcpyDeviceToDevice, r.stream));
    DRT_HIP(hipStreamSynchronize(r.stream));
    drop_graphs();  // captured forwards point at the old cache
    kv = std::move(grown);
    tile_cap = tiles;
    g_ranges = attention_decode_ranges(tile_cap * 32, r.Hkv());
    head_stride = new_head;
    layer_stride = head_stride * r.Hkv();
    m.kv_cache_bytes = (int64_t)kv.bytes;
  }

  void upload_tokens(int lo, int hi) {
    if (hi <= lo) return;
    DRT_HIP(hipMemcpyAsync(tokens_dev.as<int32_t>() + lo, canvas.data() + lo, (size_t)(hi - lo) * 4,
                           hipMemcpyHostToDevice, rt->stream));
  }

  // d2f block start of position p under geometry (prompt_len, block).
  static int seg_start(int p, int prompt_len, int blk) {
    if (p < prompt_len) return 0;
    return prompt_len + ((p - prompt_len) / blk) * blk;
  }

  // Commit forwards for rows [lo, hi): chunks end on block boundaries.
  void commit_rows(int lo, int hi, int prompt_len, int blk) {
    const Runtime& r = *rt;
    int row = lo;
    while (row < hi) {
      int end = std::min(hi, row + r.max_rows);
      if (end < hi) {
        const int snapped = seg_start(end, prompt_len, blk);
        require(snapped > row, "a mask segment is longer than max_forward_rows");
        end = snapped;
      }
      ForwardArgs a;
      a.tokens_dev = tokens_dev.as<int32_t>();
      a.row0 = row;
      a.n_rows = end - row;
      a.n_keys = end;
      a.mask_kind = 1;
      a.mask_prompt_len = prompt_len;
      a.mask_block = blk;
      run_forward(*rt, kv.p, head_stride, layer_stride, a);
      m.commit_rows += end - row;
      row = end;
    }
  }

  double finish_timing() {
    Runtime& r = *rt;
    DRT_HIP(hipEventSynchronize(r.ev1));
    float ms = 0.f;
    DRT_HIP(hipEventElapsedTime(&ms, r.ev0, r.ev1));
    m.last_forward_ms = ms;
    m.total_forward_ms += ms;
    return ms;
  }

  int raw_row(int p) const {
    if (rt->geo.logits_convention == DRT_LOGITS_DREAM_AR_SHIFT) return p >= 1 ? p - 1 : 0;
    return p;
  }
};

}  // namespace drt

// ====================================================================== C-ABI

using namespace drt;

namespace {

template <typename Fn> int32_t guarded(Fn&& fn) {
  try {
    fn();
    return DRT_OK;
  } catch (const Error& e) {
    g_last_error = e.what();
    return e.status;
  } catch (const std::bad_alloc&) {
    g_last_error = "host allocation failed";
    return DRT_INTERNAL_ERROR;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return DRT_INTERNAL_ERROR;
  }
}

hipStream_t as_stream(void* s) { return (hipStream_t)s; }

}  // namespace

extern "C" {

void drt_abi_version(int32_t* major, int32_t* minor, int32_t* patch) {
  if (major) *major = 0;
  if (minor) *minor = 1;
  if (patch) *patch = 0;
}

size_t drt_last_error(char* buf, size_t len) {
  const std::string& e = g_last_error;
  if (buf && len) {
    const size_t n = std::min(len - 1, e.size());
    std::memcpy(buf, e.data(), n);
    buf[n] = 0;
  }
  return e.size();
}

int32_t drt_release_handle(uint64_t handle) {
  return guarded([&] { handles().release(handle); });
}

int32_t drt_runtime_create(const drt_engine_config* engine, const drt_model_geometry* geometry,
                           const drt_tensor* weights, int32_t n_weights, uint64_t* out_runtime) {
  return guarded([&] {
    require(engine && geometry && weights && out_runtime && n_weights > 0,
            "drt_runtime_create needs engine, geometry, weights and an output handle");
    auto rt = create_runtime(*engine, *geometry, weights, n_weights);
    *out_runtime = handles().add(Kind::RUNTIME, rt);
  });
}

int32_t drt_session_open(uint64_t runtime, const drt_session_config* config,
                         uint64_t* out_session) {
  return guarded([&] {
    require(config && out_session, "drt_session_open needs a config and an output handle");
    auto rt = handles().get<Runtime>(runtime, Kind::RUNTIME);
    const drt_session_config& c = *config;
    for (int i = 0; i < 8; ++i) require(c.reserved[i] == 0, "session config reserved fields must be 0");
    const bool bd3 = c.decode_strategy == DRT_DECODE_BD3_FIXED_QUOTA;
    const bool fq = c.decode_strategy == DRT_DECODE_FIXED_QUOTA;
    const bool bt = c.decode_strategy == DRT_DECODE_BLOCK_THRESHOLD;
    const bool window_only = c.decode_strategy < 0;  // forward-only window session
    if (!bd3 && !fq && !bt && !window_only)
      fail(UNSUPPORTED, "rocm sessions run only block_threshold, fixed_quota and bd3_fixed_quota");
    if (bd3 || bt) require(c.attention_mask_kind == DRT_MASK_D2F_HYBRID,
                           "bd3_fixed_quota and block_threshold run only on a d2f_hybrid graph");
    if (fq) require(c.attention_mask_kind == DRT_MASK_BIDIRECTIONAL,
                    "fixed_quota runs only on a bidirectional graph");
    if (bd3 || fq) require(c.commit_policy == DRT_COMMIT_FIXED_QUOTA,
                           "fixed-quota strategies need the fixed_quota commit policy");
    if (bt) require(c.commit_policy == DRT_COMMIT_THRESHOLD,
                    "block_threshold needs the threshold commit policy");
    auto sess = std::make_shared<Session>();
    sess->rt = rt;
    sess->cfg = c;
    DRT_HIP(hipSetDevice(rt->device));
    *out_session = handles().add(Kind::SESSION, sess);
  });
}

int32_t drt_session_start(uint64_t session, const int32_t* tokens, int32_t n_tokens,
                          int32_t prompt_len, int32_t block_size, int32_t mask_token_id,
                          int32_t exact_kv, int32_t steps, int64_t memory_budget_bytes,
                          double temperature, uint64_t seed) {
  return guarded([&] {
    auto s = handles().get<Session>(session, Kind::SESSION);
    Runtime& r = *s->rt;
    require(tokens && n_tokens > 0, "start_device needs a non-empty canvas");
    require(n_tokens <= r.rope_positions, "canvas longer than the rotary table");
    require(block_size >= 1 && prompt_len >= 0 && prompt_len <= n_tokens, "bad block geometry");
    require(steps >= 1, "steps must be >= 1");
    require(!(temperature < 0.0) && std::isfinite(temperature), "temperature must be >= 0");
    const bool threshold = s->cfg.decode_strategy == DRT_DECODE_BLOCK_THRESHOLD;
    // block_threshold runs over the exact prompt + frozen-block K/V either way:
    // every cached row is what a full forward of the canvas computes for it
    if (exact_kv && !threshold)
      fail(UNSUPPORTED, "D2F exact K/V belongs to block_threshold, not the fixed-quota path");
    if (threshold) require(temperature == 0.0, "block_threshold decodes greedily (temperature 0)");
    if (s->cfg.attention_mask_kind == DRT_MASK_BIDIRECTIONAL)
      require(n_tokens <= r.max_rows, "a bidirectional canvas must fit max_forward_rows");
    for (int i = 0; i < n_tokens; ++i)
      require(tokens[i] >= 0 && tokens[i] < r.V(), "token id outside the vocabulary");
    DRT_HIP(hipSetDevice(r.device));
    s->canvas.assign(tokens, tokens + n_tokens);
    const void* canvas_was = s->tokens_dev.p;
    s->tokens_dev.ensure((size_t)n_tokens * 4);
    if (s->tokens_dev.p != canvas_was) s->drop_graphs();  // captured forwards read the canvas
    s->ensure_cache(n_tokens);
    s->cache_len = 0;  // a new request: nothing in the cache belongs to it yet
    s->feeder_pos = -1;
    s->loop = Session::Bd3Loop{};
    s->origin = prompt_len;
    s->block = block_size;
    s->mask_id = mask_token_id;
    s->steps = steps;
    s->temperature = temperature;
    s->seed = seed;
    s->proposals = 0;
    s->win_prompt_len = -1;
    s->started = true;
    if (memory_budget_bytes > 0 && s->kv.bytes > (size_t)memory_budget_bytes)
      fail(INVALID_ARGUMENT, "prefix K/V cache needs " + std::to_string(s->kv.bytes) +
                                 " bytes, above memory_budget_bytes");
    s->upload_tokens(0, n_tokens);
    DRT_HIP(hipStreamSynchronize(r.stream));
  });
}

// The frontier entry whose raw row precedes the forward's first row (the Dream
// shift's feeder position), or -1.
static int feeder_i_of(const std::shared_ptr<Session>& s, const int32_t* frontier, int n,
                       int row0) {
  for (int i = 0; i < n; ++i)
    if (s->raw_row(frontier[i]) < row0) return i;
  return -1;
}

static void propose_impl(uint64_t session, const int32_t* frontier, int32_t n_frontier,
                         int32_t window_end, int32_t frozen_prefix, double* out_scores,
                         int32_t* out_tokens, int32_t* out_forwarded_rows) {
  {
    auto s = handles().get<Session>(session, Kind::SESSION);
    Runtime& r = *s->rt;
    require(s->started, "propose_device before start_device");
    require(frontier && n_frontier > 0 && out_scores && out_tokens,
            "propose_device needs a non-empty frontier and outputs");
    ProfScope ps(&s->prof);
    const int n = (int)s->canvas.size();
    DRT_HIP(hipSetDevice(r.device));
    ForwardArgs a;
    a.tokens_dev = s->tokens_dev.as<int32_t>();
    a.temperature = (float)s->temperature;
    a.seed = s->seed;
    a.step = s->proposals;
    int forwarded = 0;
    bool graph = false;  // the forward is a session graph's (D2F block forwards)
    if (s->cfg.attention_mask_kind == DRT_MASK_D2F_HYBRID) {
      require(window_end >= 1 && window_end <= n, "window_end outside the canvas");
      require(frozen_prefix >= 0 && frozen_prefix < window_end, "frozen_prefix outside the window");
      require(Session::seg_start(frozen_prefix, s->origin, s->block) == frozen_prefix,
              "frozen_prefix must start a block of the session geometry");
      // Under the Dream logits shift position p reads row p - 1, so the block's
      // first position reads the last row before the block: the forward then
      // starts one row early and recomputes that row over its own (cached)
      // context -- the reference's shift-feeder row
      // (backends/mlx_d2f_forward.py:226-232). Its K/V is rewritten with what
      // the cache already holds for it.
      int feeder_i = -1;  // the frontier entry that reads row frozen_prefix - 1
      for (int i = 0; i < n_frontier; ++i) {
        const int p = frontier[i];
        require(p >= frozen_prefix && p < window_end,
                "frontier position outside [frozen_prefix, window_end)");
        const int rr = s->raw_row(p);
        require(rr >= frozen_prefix - 1, "frontier reads a row before frozen_prefix - 1");
        if (rr < frozen_prefix) {
          require(feeder_i < 0, "a position appears twice in the frontier");
          feeder_i = i;
        }
      }
      // An earlier frozen prefix shrinks the exact cache; a later one commits blocks.
      if (s->cache_len > frozen_prefix) {
        s->cache_len = frozen_prefix;
        s->feeder_pos = -1;
      }
      DRT_HIP(hipEventRecord(r.ev0, r.stream));
      // One block left to commit right before this forward's block: both run as
      // one forward, the committed block a first mask segment (its rows see keys
      // up to their block's end, exactly what the commit forward computes).
      const bool pair = s->pairable() && s->cache_len + s->block == frozen_prefix &&
                        s->cache_len % s->block == 0 && window_end - frozen_prefix == s->block &&
                        feeder_i < 0 && n_frontier <= 32;
      const int row0 = pair ? s->cache_len : frozen_prefix;
      if (pair) {
        forwarded += s->block;
        s->m.commit_rows += s->block;
        s->cache_len = frozen_prefix;
      }
      forwarded += s->commit_to(frozen_prefix);
      if (s->cfg.decode_strategy == DRT_DECODE_BLOCK_THRESHOLD) a.exclude_col = s->mask_id;
      if (feeder_i >= 0 && s->feeder_pos != frozen_prefix) {
        // the frozen row's score and token: one row over its own (cached) context
        ForwardArgs f;
        f.tokens_dev = s->tokens_dev.as<int32_t>();
        f.row0 = frozen_prefix - 1;
        f.n_rows = 1;
        f.n_keys = frozen_prefix;
        f.mask_kind = 1;
        f.mask_prompt_len = s->origin;
        f.mask_block = s->block;
        f.exclude_col = a.exclude_col;
        f.temperature = a.temperature;
        f.seed = a.seed;
        f.step = a.step;
        f.n_lm = 1;
        f.lm_rows.push_back(0);
        f.lm_pos.push_back(frozen_prefix);
        s->upload_tokens(frozen_prefix - 1, frozen_prefix);
        run_forward(r, s->kv.p, s->head_stride, s->layer_stride, f);
        DRT_HIP(hipStreamSynchronize(r.stream));
        r.up_next = Runtime::EAGER_SLOT0;
        check_placement(r);
        s->feeder_pos = frozen_prefix;
        s->feeder_score = r.scores_host()[0];
        s->feeder_token = r.tokens_host()[0];
        forwarded += 1;
      }
      a.row0 = row0;
      a.n_rows = window_end - row0;
      a.n_keys = window_end;
      a.mask_kind = 1;
      a.mask_prompt_len = s->origin;
      a.mask_block = s->block;
      a.seg_rows = pair ? s->block : 0;
      graph = n_frontier <= 32 && (pair ? s->use_graphs && !s->prof.on
                                        : s->graphable(a.n_rows));
      if (!graph) s->upload_tokens(row0, window_end);
    } else {
      // Full bidirectional canvas, no cache (Dream / MDLM fixed_quota).
      for (int i = 0; i < n_frontier; ++i)
        require(frontier[i] >= 0 && frontier[i] < n, "frontier position outside the canvas");
      DRT_HIP(hipEventRecord(r.ev0, r.stream));
      s->upload_tokens(0, n);
      a.row0 = 0;
      a.n_rows = n;
      a.n_keys = n;
      a.mask_kind = 0;
    }
    // the feeder position (if any) is served from the session, not the forward
    const int skip = a.mask_kind == 1 ? feeder_i_of(s, frontier, n_frontier, a.row0) : -1;
    for (int i = 0; i < n_frontier; ++i) {
      if (i == skip) continue;
      a.lm_rows.push_back(s->raw_row(frontier[i]) - a.row0);
      a.lm_pos.push_back(frontier[i]);
    }
    a.n_lm = (int)a.lm_rows.size();
    if (a.n_lm > 0) {
      if (graph)
        s->graph_forward(a.seg_rows > 0 ? Session::G_PAIR : Session::G_STEP, a);
      else
        run_forward(r, s->kv.p, s->head_stride, s->layer_stride, a);
      forwarded += a.n_rows - a.seg_rows;
    }
    r.up_next = Runtime::EAGER_SLOT0;  // the stream is drained below before any slot is reused
    DRT_HIP(hipEventRecord(r.ev1, r.stream));
    // the LM head's last kernel wrote scores, tokens and the placement flags
    // into pinned host memory: nothing to copy once the stream has drained
    DRT_HIP(hipStreamSynchronize(r.stream));
    check_placement(r);
    for (int i = 0, j = 0; i < n_frontier; ++i) {
      if (i == skip) {
        out_scores[i] = s->feeder_score;
        out_tokens[i] = s->feeder_token;
      } else {
        out_scores[i] = r.scores_host()[j];
        out_tokens[i] = r.tokens_host()[j];
        ++j;
      }
    }
    s->finish_timing();
    s->publish_profile();
    s->proposals += 1;
    s->m.forward_count += 1;
    s->m.active_rows += a.n_rows - a.seg_rows;  // a committed block's rows are commit rows
    s->m.lm_rows += n_frontier;
    s->m.kv_cache_len = s->cache_len;
    if (out_forwarded_rows) *out_forwarded_rows = forwarded;
  }
}

int32_t drt_session_propose(uint64_t session, const int32_t* frontier, int32_t n_frontier,
                            int32_t window_end, int32_t frozen_prefix, double* out_scores,
                            int32_t* out_tokens, int32_t* out_forwarded_rows) {
  return guarded([&] {
    propose_impl(session, frontier, n_frontier, window_end, frozen_prefix, out_scores, out_tokens,
                 out_forwarded_rows);
  });
}

// The BD3 fixed-quota loop of decode.py (BD3FixedQuotaCommit over absolute blocks,
// diffusion_runtime.py:1200-1346, driven as run_decode_loop does, :1829-1991) run
// natively: plan, propose, pick the quota's best rows, commit, with no return to
// the caller between steps. Same schedule and commits as the host loop; rows with
// exactly equal float64 scores are taken lowest index first.
int32_t drt_session_bd3_decode(uint64_t session, int32_t prompt_len, int32_t max_tokens,
                               int32_t steps, int32_t eos_token_id, int32_t requires_alignment,
                               int32_t max_forwards, int32_t* out_forwards,
                               int32_t* out_committed, int32_t* out_done) {
  return guarded([&] {
    auto s = handles().get<Session>(session, Kind::SESSION);
    require(s->started, "bd3_decode before start_device");
    require(s->cfg.decode_strategy == DRT_DECODE_BD3_FIXED_QUOTA && s->origin == 0,
            "bd3_decode runs a bd3_fixed_quota session (block origin 0)");
    const int n = (int)s->canvas.size();
    require(prompt_len >= 0 && max_tokens >= 0 && prompt_len + max_tokens == n,
            "bd3_decode: prompt_len + max_tokens must equal the canvas length");
    require(steps >= 1 && max_forwards >= 0, "bd3_decode: steps >= 1, max_forwards >= 0");
    const int B = s->block;
    Session::Bd3Loop& L = s->loop;
    if (!L.on || L.prompt_len != prompt_len || L.gen != max_tokens || L.steps != steps) {
      L = Session::Bd3Loop{};
      L.on = true;
      L.prompt_len = prompt_len;
      L.gen = max_tokens;
      L.steps = steps;
      L.eos = eos_token_id;
      L.align = requires_alignment != 0;
      if (max_tokens > 0) {
        const int first = prompt_len / B, last = (prompt_len + max_tokens - 1) / B;
        L.count = last - first + 1;
        const int sched = (max_tokens + B - 1) / B;
        L.spb = (steps + sched - 1) / sched;
      }
      L.limit = L.count * L.spb;
    }
    int forwards = 0, committed = 0, done = 0;
    // a block queued ahead that the loop does not reach is dropped on the way out
    struct DropQueued {
      Session* s;
      ~DropQueued() {
        try {
          s->discard_queued();
        } catch (...) {
        }
      }
    } drop_queued{&*s};
    std::vector<int32_t> frontier, pos, tok;
    std::vector<double> sc;
    std::vector<int32_t> tk, order;
    while (forwards < max_forwards) {
      const int step = L.step;
      if (step >= L.limit) { done = 1; break; }
      if (L.align && prompt_len % B)
        fail(INVALID_ARGUMENT, "BD3LM Candidate prompt length must be a multiple of block_size");
      const int32_t* gen = s->canvas.data() + prompt_len;
      // EOS ends the decode only at a block boundary
      if (step % L.spb == 0 && std::find(gen, gen + max_tokens, L.eos) != gen + max_tokens) {
        done = 1;
        break;
      }
      if (std::find(gen, gen + max_tokens, s->mask_id) == gen + max_tokens) { done = 1; break; }
      const int block_id = step / L.spb;
      const int grid = (prompt_len / B + block_id) * B;
      const int lo = std::max(prompt_len, grid), hi = std::min(prompt_len + max_tokens, grid + B);
      frontier.clear();
      for (int p = lo; p < hi; ++p)
        if (s->canvas[p] == s->mask_id) frontier.push_back(p);
      if (L.active != block_id) {
        L.active = block_id;
        L.base = (int)frontier.size() / L.spb;
        L.rem = (int)frontier.size() % L.spb;
      }
      // A whole aligned block, from this step to its last one or to the call's
      // forward limit: the forwards run back to back, each step's choice made on
      // the device (the steps with a quota; a step without one forwards nothing,
      // as below). A block entered mid-way (an earlier call stopped inside it)
      // continues the same way.
      if (lo == grid && hi == grid + B && !frontier.empty() && s->block_on_device()) {
        std::vector<int> quotas;
        int j = step % L.spb;
        for (; j < L.spb && (int)quotas.size() < max_forwards - forwards; ++j) {
          const int q = L.base + (j < L.rem ? 1 : 0);
          if (q > 0) quotas.push_back(q);
        }
        if (!quotas.empty() &&
            (int)quotas.size() <= Runtime::UPLOAD_SLOTS - Runtime::EAGER_SLOT0) {
          // a fresh block's forwards with a quota (every row masked)
          s->full_block_steps = std::min(L.spb, B);
          // this block, unless it was queued ahead (with the same quotas)
          Session::QueuedBlock* qb = s->queued_at(grid);
          if (qb && qb->quotas != quotas) {
            s->discard_block(*qb);
            qb = nullptr;
          }
          if (!qb) {
            s->discard_queued();
            qb = &s->queue_block(grid, quotas, true);
          }
          // Queue the next block behind it while it runs, when the loop will run
          // that block next in this call unless the decode stops at the boundary
          // (then it is dropped): a whole block from its first step, fresh (every
          // row masked), within the step and forward budgets, on the captured graphs.
          const int ngrid = grid + B;
          if (j == L.spb && s->queue_ahead_ready() && block_id + 1 < L.count &&
              ngrid + B <= prompt_len + max_tokens && !s->queued_at(ngrid)) {
            bool fresh = true;
            for (int p = ngrid; p < ngrid + B && fresh; ++p) fresh = s->canvas[p] == s->mask_id;
            std::vector<int> nq;
            for (int k = 0; k < L.spb; ++k) {
              const int q = B / L.spb + (k < B % L.spb ? 1 : 0);
              if (q > 0) nq.push_back(q);
            }
            if (fresh && (int)nq.size() == s->g_block_n && qb->S <= Session::QB_SLOTS &&
                (int)nq.size() <= Session::QB_SLOTS &&
                forwards + qb->S + (int)nq.size() <= max_forwards)
              s->queue_block(ngrid, nq, false);
          }
          forwards += s->finish_block(*qb);
          for (int q : quotas) committed += q;
          L.step = step + (j - step % L.spb);  // the steps run, quota-less ones included
          continue;
        }
      }
      s->discard_queued();  // (a block queued ahead is always the loop's next block)
      const int quota = L.base + (step % L.spb < L.rem ? 1 : 0);
      if (frontier.empty() || quota == 0) {
        L.step = step + 1;
        continue;
      }
      const int nf = (int)frontier.size();
      sc.assign(nf, 0.0);
      tk.assign(nf, 0);
      int32_t fwd = 0;
      propose_impl(session, frontier.data(), nf, hi, (frontier[0] / B) * B, sc.data(), tk.data(),
                   &fwd);
      ++forwards;
      order.resize(nf);
      for (int i = 0; i < nf; ++i) order[i] = i;
      // highest score first, equal scores in row order; a NaN score ranks as
      // -inf (a strict weak order for the sort)
      auto key = [&](int i) { return std::isnan(sc[i]) ? -INFINITY : sc[i]; };
      std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return key(a) > key(b); });
      const int k = std::min(quota, nf);
      for (int i = 0; i < k; ++i) {
        const int r = order[i];
        require(tk[r] >= 0 && tk[r] < s->rt->V(), "proposed token outside the vocabulary");
        s->canvas[frontier[r]] = tk[r];
      }
      committed += k;
      L.step = step + 1;  // only once the step is committed: a failed call repeats it
    }
    if (out_forwards) *out_forwards = forwards;
    if (out_committed) *out_committed = committed;
    if (out_done) *out_done = done;
  });
}

// The session's canvas (the committed tokens of a native loop): n_out >= its length.
int32_t drt_session_canvas(uint64_t session, int32_t* out, int32_t n_out, int32_t* out_len) {
  return guarded([&] {
    auto s = handles().get<Session>(session, Kind::SESSION);
    require(s->started, "canvas before start_device");
    const int n = (int)s->canvas.size();
    if (out_len) *out_len = n;
    require(out && n_out >= n, "canvas output buffer too small");
    std::memcpy(out, s->canvas.data(), (size_t)n * 4);
  });
}

int32_t drt_session_commit(uint64_t session, const int32_t* positions, const int32_t* tokens,
                           int32_t n) {
  return guarded([&] {
    auto s = handles().get<Session>(session, Kind::SESSION);
    require(s->started, "commit_device before start_device");
    require(n >= 0 && (n == 0 || (positions && tokens)), "commit_device needs positions and tokens");
    const int len = (int)s->canvas.size();
    for (int i = 0; i < n; ++i) {
      require(positions[i] >= 0 && positions[i] < len, "commit position outside the canvas");
      require(positions[i] >= s->cache_len,
              "commit position inside the committed prefix K/V (a frozen block)");
      require(tokens[i] >= 0 && tokens[i] < s->rt->V(), "commit token outside the vocabulary");
    }
    for (int i = 0; i < n; ++i) s->canvas[positions[i]] = tokens[i];
  });
}

int32_t drt_session_execute_window(uint64_t session, const int32_t* token_ids, int32_t n_tokens,
                                   const int32_t* scope, int32_t n_scope,
                                   int32_t mask_prompt_len, int32_t mask_block_size,
                                   float* out_logits, int64_t out_capacity,
                                   int32_t* out_n_vocab, int32_t* out_forwarded_rows) {
  return guarded([&] {
    auto s = handles().get<Session>(session, Kind::SESSION);
    Runtime& r = *s->rt;
    require(token_ids && n_tokens > 0 && scope && n_scope > 0 && out_logits,
            "execute_window needs tokens, a non-empty scope and an output buffer");
    require((int64_t)n_scope * r.V() <= out_capacity, "execute_window output buffer too small");
    require(n_tokens <= r.rope_positions, "window longer than the rotary table");
    for (int i = 0; i < n_tokens; ++i)
      require(token_ids[i] >= 0 && token_ids[i] < r.V(), "token id outside the vocabulary");
    for (int i = 0; i < n_scope; ++i)
      require(scope[i] >= 0 && scope[i] < n_tokens, "scope position outside the window");
    const bool d2f = mask_block_size > 0;
    ProfScope ps(&s->prof);
    if (s->cfg.attention_mask_kind == DRT_MASK_D2F_HYBRID)
      require(d2f, "a d2f_hybrid session needs the window's mask geometry");
    else
      require(!d2f, "mask geometry is only consumed by the d2f_hybrid kind");
    DRT_HIP(hipSetDevice(r.device));
    // The window replaces the session canvas.
    const int old_n = (int)s->canvas.size();
    s->canvas.assign(token_ids, token_ids + n_tokens);
    if ((size_t)n_tokens * 4 > s->tokens_dev.bytes) {
      DevBuf t;
      t.alloc((size_t)std::max(n_tokens, s->cfg.max_tokens) * 4);
      s->tokens_dev = std::move(t);  // rows below the reuse point are never re-read
    }
    s->ensure_cache(n_tokens);
    (void)old_n;
    ForwardArgs a;
    a.tokens_dev = s->tokens_dev.as<int32_t>();
    int forwarded = 0;
    int min_raw = n_tokens;
    for (int i = 0; i < n_scope; ++i) min_raw = std::min(min_raw, s->raw_row(scope[i]));
    DRT_HIP(hipEventRecord(r.ev0, r.stream));
    if (d2f) {
      require(mask_prompt_len >= 0 && mask_prompt_len <= n_tokens, "bad mask geometry");
      const int frozen = Session::seg_start(min_raw, mask_prompt_len, mask_block_size);
      // Reuse the cached exact prefix only for the same geometry and tokens.
      int valid = 0;
      if (s->win_prompt_len == mask_prompt_len && s->win_block == mask_block_size) {
        const int lim = std::min({s->cache_len, frozen, (int)s->win_tokens.size()});
        while (valid < lim && s->win_tokens[valid] == token_ids[valid]) ++valid;
        valid = valid < mask_prompt_len ? 0 : Session::seg_start(valid, mask_prompt_len, mask_block_size);
        if (valid > lim) valid = 0;
      }
      s->cache_len = valid;
      if (valid < frozen) {
        s->upload_tokens(valid, frozen);
        s->commit_rows(valid, frozen, mask_prompt_len, mask_block_size);
        forwarded += frozen - valid;
      }
      s->cache_len = frozen;
      s->win_prompt_len = mask_prompt_len;
      s->win_block = mask_block_size;
      s->win_tokens.assign(token_ids, token_ids + frozen);
      s->upload_tokens(frozen, n_tokens);
      a.row0 = frozen;
      a.n_rows = n_tokens - frozen;
      a.n_keys = n_tokens;
      a.mask_kind = 1;
      a.mask_prompt_len = mask_prompt_len;
      a.mask_block = mask_block_size;
    } else {
      require(n_tokens <= r.max_rows, "a bidirectional window must fit max_forward_rows");
      s->upload_tokens(0, n_tokens);
      a.row0 = 0;
      a.n_rows = n_tokens;
      a.n_keys = n_tokens;
      a.mask_kind = 0;
      s->cache_len = 0;
    }
    a.n_lm = n_scope;
    for (int i = 0; i < n_scope; ++i) {
      a.lm_rows.push_back(s->raw_row(scope[i]) - a.row0);
      a.lm_pos.push_back(scope[i]);
    }
    require(a.n_rows <= r.max_rows, "the active window exceeds max_forward_rows");
    s->rt->logits.ensure((size_t)n_scope * r.V() * 4);
    a.logits = r.logits.as<float>();
    run_forward(r, s->kv.p, s->head_stride, s->layer_stride, a);
    forwarded += a.n_rows;
    DRT_HIP(hipEventRecord(r.ev1, r.stream));
    DRT_HIP(hipMemcpyAsync(out_logits, r.logits.p, (size_t)n_scope * r.V() * 4,
                           hipMemcpyDeviceToHost, r.stream));
    DRT_HIP(hipMemcpyAsync(r.placement_host, r.placement_err.p, 4, hipMemcpyDeviceToHost,
                           r.stream));
    DRT_HIP(hipStreamSynchronize(r.stream));
    check_placement(r);
    s->finish_timing();
    s->publish_profile();
    s->m.forward_count += 1;
    s->m.active_rows += a.n_rows;
    s->m.lm_rows += n_scope;
    s->m.kv_cache_len = s->cache_len;
    if (out_n_vocab) *out_n_vocab = r.V();
    if (out_forwarded_rows) *out_forwarded_rows = forwarded;
  });
}

int32_t drt_session_metrics(uint64_t session, drt_metrics* out) {
  return guarded([&] {
    require(out != nullptr, "drt_session_metrics needs an output struct");
    auto s = handles().get<Session>(session, Kind::SESSION);
    *out = s->m;
  });
}

int32_t drt_session_set_profiling(uint64_t session, int32_t enable) {
  return guarded([&] {
    auto s = handles().get<Session>(session, Kind::SESSION);
    if (enable && !s->prof.on) {
      s->prof.reset();
      for (int c = 0; c < Profiler::NCLASS; ++c) {
        s->m.prof_ms[c] = 0;
        s->m.prof_bytes[c] = 0;
        s->m.prof_launches[c] = 0;
      }
    }
    s->prof.on = enable != 0;
  });
}

// ------------------------------------------------------------------ per-op

// ACT_F16P activation (hi and lo planes) + group sums, then (more than 32
// rows) the split-K slices
static size_t q4_op_act_bytes(int32_t m, int32_t k) {
  return ((size_t)2 * m * k * 2 + (size_t)m * (k / 64) * 4 + 255) / 256 * 256;
}

size_t drt_op_q4_linear_workspace_bytes(int32_t m, int32_t n, int32_t k) {
  if (m <= 0 || k <= 0) return 0;
  size_t b = q4_op_act_bytes(m, k) + 256;
  if (m > 32 && n > 0) b += (size_t)big_linear_splits(m, n, k, BG_OP_MAX_KS) * m * n * 4;
  if (m <= 32 && n > 0)
    b += std::max(stream_part_floats(m, n, k, BG_OP_MAX_KS), skinny_part_floats(n, k)) * 4;
  return b;
}

// The split-K store kernel of the per-op path (<= 32 rows): its arrival counters
// live in a device array of the library, zero from load and left zero by every
// launch, one block of OP_COUNTERS per (device, stream) so that calls on
// different streams never share one; the XCD placement is probed once per
// device (on a stream of its own, synchronised once).
constexpr int OP_COUNTER_BLOCKS = 32, OP_COUNTERS = 4096;
static __device__ int op_counters[OP_COUNTER_BLOCKS * OP_COUNTERS];
static __device__ int op_probe[256];
namespace {
struct OpDevice {
  int* counters = nullptr;
  int n_xcc = 1;
  bool fenced = false;
  std::map<hipStream_t, int> blocks;
};
std::mutex g_op_mu;
std::map<int, OpDevice> g_op_dev;

// The counter block of (current device, stream) and the device's placement,
// or nullptr when every block is taken (the caller then takes another path).
int* op_counters_for(hipStream_t stream, int& n_xcc, bool& fenced) {
  int dev = -1;
  DRT_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_op_mu);
  OpDevice& d = g_op_dev[dev];
  if (!d.counters) {
    void* c = nullptr;
    void* pr = nullptr;
    DRT_HIP(hipGetSymbolAddress(&c, HIP_SYMBOL(op_counters)));
    DRT_HIP(hipGetSymbolAddress(&pr, HIP_SYMBOL(op_probe)));
    int nx = 1;
    if (hipDeviceGetAttribute(&nx, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess) nx = 1;
    d.n_xcc = std::max(1, nx);
    hipStream_t ps = nullptr;
    DRT_HIP(hipStreamCreateWithFlags(&ps, hipStreamNonBlocking));
    bool rr = false;
    try {
      rr = probe_round_robin(d.n_xcc, (int*)pr, ps);
    } catch (...) {
      (void)hipStreamDestroy(ps);
      throw;
    }
    DRT_HIP(hipStreamDestroy(ps));
    d.fenced = !rr;
    d.counters = (int*)c;
  }
  n_xcc = d.n_xcc;
  fenced = d.fenced;
  auto it = d.blocks.find(stream);
  if (it == d.blocks.end()) {
    if ((int)d.blocks.size() >= OP_COUNTER_BLOCKS) return nullptr;
    it = d.blocks.emplace(stream, (int)d.blocks.size()).first;
  }
  return d.counters + (size_t)it->second * OP_COUNTERS;
}
}  // namespace

int32_t drt_op_q4_repack(const void* w_q, const void* scales, const void* biases, int32_t n,
                         int32_t k, void* qw, void* sb, void* stream) {
  return guarded([&] {
    require(w_q && scales && biases && qw && sb && n > 0 && k > 0, "bad q4_repack arguments");
    q4_repack((const uint32_t*)w_q, (const uint16_t*)scales, (const uint16_t*)biases, n, k,
              (uint32_t*)qw, (uint32_t*)sb, as_stream(stream));
  });
}

int32_t drt_op_q4_quantize(const void* w, int32_t w_dtype, int32_t n, int32_t k, void* w_q,
                           void* scales, void* biases, void* stream) {
  return guarded([&] {
    require(w && w_q && scales && biases && n > 0 && k > 0, "bad q4_quantize arguments");
    require(w_dtype == DRT_F32 || w_dtype == DRT_BF16, "q4_quantize weight must be F32 or BF16");
    if (k % 64 != 0) fail(UNSUPPORTED, "q4_quantize needs k % 64 == 0 (group size 64)");
    q4_quantize(w, w_dtype == DRT_F32, n, k, (uint32_t*)w_q, (uint16_t*)scales,
                (uint16_t*)biases, as_stream(stream));
  });
}

int32_t drt_op_cast_bf16(const float* x, void* y, int64_t n, void* stream) {
  return guarded([&] {
    require(x && y && n > 0, "bad cast_bf16 arguments");
    to_bf16(x, (uint16_t*)y, n, as_stream(stream));
  });
}

static void q4_linear_into(const void* qw, const void* sb, const void* x, int32_t x_dtype,
                           int32_t m, int32_t n, int32_t k, const void* bias, float* y,
                           void* workspace, size_t workspace_bytes, void* stream) {
  {
    require(qw && sb && x && y && m > 0 && n > 0 && k > 0, "bad q4_linear arguments");
    require(n % 32 == 0 && k % 64 == 0, "q4_linear needs n % 32 == 0 and k % 64 == 0");
    require(x_dtype == DRT_F32 || x_dtype == DRT_BF16, "q4_linear x must be F32 or BF16");
    require(workspace && workspace_bytes >= drt_op_q4_linear_workspace_bytes(m, n, k),
            "q4_linear workspace too small");
    char* ws = (char*)workspace;
    _Float16* xp = (_Float16*)ws;
    float* xs = (float*)(ws + (size_t)2 * m * k * 2);
    hipStream_t st = as_stream(stream);
    const StreamPlan sp = stream_plan(m, n, k, BG_OP_MAX_KS);
    if (m <= 32 && sp.KS < 1 && n / 32 <= OP_COUNTERS) {
      // one launch: the split-K store kernel reads the fp32 / bf16 rows itself
      FusedArgs g;
      g.qw = (const uint32_t*)qw;
      g.sb = (const uint32_t*)sb;
      g.bias = (const uint16_t*)bias;
      g.M = m;
      g.N = n;
      g.K = k;
      g.act = x;
      g.x_in = x_dtype == DRT_BF16 ? 2 : 1;
      g.y = y;
      g.part = (float*)(ws + q4_op_act_bytes(m, k));
      g.part_floats = skinny_part_floats(n, k);
      g.sk_row_tiles = 1;
      bool fenced = false;
      g.counters = op_counters_for(st, g.n_xcc, fenced);
      g.n_counters = OP_COUNTERS;
      g.fenced = fenced ? 1 : 0;
      if (g.counters && skinny_linear(g, FL_STORE, st)) return;
    }
    q4_act_prep(x, x_dtype == DRT_BF16, m, k, xp, xs, st);
    FusedArgs f;
    f.qw = (const uint32_t*)qw;
    f.sb = (const uint32_t*)sb;
    f.bias = (const uint16_t*)bias;
    f.M = m;
    f.N = n;
    f.K = k;
    f.act = xp;
    f.act_xsum = xs;
    f.y = y;
    const int ks = m > 32 ? big_linear_splits(m, n, k, BG_OP_MAX_KS) : 1;
    if (sp.KS >= 1) {
      // large weights, <= 32 rows: streamed in fp32 K slices, summed (+ bias) into y
      float* part = (float*)(ws + q4_op_act_bytes(m, k));
      FusedArgs g = f;
      g.bias = nullptr;
      g.y = part;
      stream_linear(g, sp, st);
      sum_slices(part, sp.KS, (int64_t)m * n, (const uint16_t*)bias, n, y, st);
    } else if (ks > 1 && big_linear_supported(f, FL_STORE)) {
      // split-K slices in the workspace, summed (+ bias) into y in a fixed order
      float* part = (float*)(ws + q4_op_act_bytes(m, k));
      FusedArgs g = f;
      g.bias = nullptr;
      g.y = part;
      big_linear(g, FL_STORE, ks, st);
      sum_slices(part, ks, (int64_t)m * n, (const uint16_t*)bias, n, y, st);
    } else {
      fused_linear(f, FL_STORE, st);
    }
  }
}

int32_t drt_op_q4_linear(const void* qw, const void* sb, const void* x, int32_t x_dtype,
                         int32_t m, int32_t n, int32_t k, const void* bias, float* y,
                         void* workspace, size_t workspace_bytes, void* stream) {
  return guarded([&] {
    q4_linear_into(qw, sb, x, x_dtype, m, n, k, bias, y, workspace, workspace_bytes, stream);
  });
}

// ---- the allocation-free variant: its workspace is a file-scope device array

// The workspace of drt_op_q4_linear_noalloc: one copy per GPU the library runs
// on (each device holds its own, at its own address, until the process ends).
// In host code `scratch` only names the symbol; its device address comes from
// hipGetSymbolAddress, once per device (scratch_on_current_device).
constexpr size_t DRT_NOALLOC_SCRATCH_BYTES = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[DRT_NOALLOC_SCRATCH_BYTES];

static std::mutex g_scratch_mu;
static std::map<int, void*> g_scratch_ptr;  // device ordinal -> address of its scratch

static void* scratch_on_current_device() {
  int dev = -1;
  DRT_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  auto it = g_scratch_ptr.find(dev);
  if (it != g_scratch_ptr.end()) return it->second;
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || ptr == nullptr)
    fail(INTERNAL_ERROR, std::string("hipGetSymbolAddress of the q4 linear scratch failed on "
                                     "device ") + std::to_string(dev) + ": " +
                             hipGetErrorString(e));
  g_scratch_ptr[dev] = ptr;
  return ptr;
}

int32_t drt_op_q4_linear_noalloc(const void* qw, const void* sb, const void* x, int32_t x_dtype,
                                 int32_t m, int32_t n, int32_t k, const void* bias, float* y,
                                 void* stream) {
  return guarded([&] {
    require(m > 0 && n > 0 && k > 0, "bad q4_linear_noalloc arguments");
    const size_t need = drt_op_q4_linear_workspace_bytes(m, n, k);
    if (need > DRT_NOALLOC_SCRATCH_BYTES)
      fail(INVALID_ARGUMENT, "q4_linear_noalloc: m=" + std::to_string(m) + ", n=" +
                                 std::to_string(n) + ", k=" + std::to_string(k) + " needs " +
                                 std::to_string(need) + " bytes of workspace, above its " +
                                 std::to_string(DRT_NOALLOC_SCRATCH_BYTES) + "-byte scratch");
    q4_linear_into(qw, sb, x, x_dtype, m, n, k, bias, y, scratch_on_current_device(),
                   DRT_NOALLOC_SCRATCH_BYTES, stream);
  });
}

int32_t drt_op_bf16_repack(const void* w, int32_t n, int32_t k, void* wb, void* stream) {
  return guarded([&] {
    require(w && wb && n > 0 && k > 0, "bad bf16_repack arguments");
    bf16_repack((const uint16_t*)w, n, k, (uint16_t*)wb, as_stream(stream));
  });
}

size_t drt_op_bf16_linear_workspace_bytes(int32_t m, int32_t n, int32_t k) {
  (void)m; (void)n; (void)k;
  return 256;
}

int32_t drt_op_bf16_linear(const void* wb, const void* x, int32_t m, int32_t n, int32_t k,
                           const void* bias, float* y, void* workspace, size_t workspace_bytes,
                           void* stream) {
  return guarded([&] {
    require(wb && x && y && m > 0 && n > 0 && k > 0, "bad bf16_linear arguments");
    require(n % 32 == 0 && k % 16 == 0, "bf16_linear needs n % 32 == 0 and k % 16 == 0");
    (void)workspace;
    (void)workspace_bytes;
    FusedArgs f;
    f.wb = (const uint16_t*)wb;
    f.bias = (const uint16_t*)bias;
    f.M = m;
    f.N = n;
    f.K = k;
    f.act = x;
    f.rnd_bf16 = 1;  // the bf16 matmul output is bf16; the bias is added after
    f.y = y;
    fused_linear(f, FL_STORE, as_stream(stream));
  });
}

int32_t drt_op_kv_pack(const void* k, const void* v, int32_t src_dtype, int32_t n, int32_t hkv,
                       int32_t pos0, void* cache, int64_t head_stride, int32_t kv_dtype,
                       void* stream) {
  return guarded([&] {
    require(k && v && cache && n > 0 && hkv > 0 && pos0 >= 0, "bad kv_pack arguments");
    require(src_dtype == DRT_F32 || src_dtype == DRT_BF16, "kv_pack source must be F32 or BF16");
    require(kv_dtype == DRT_F16 || kv_dtype == DRT_BF16, "kv_pack cache must be F16 or BF16");
    require(head_stride >= (int64_t)((pos0 + n + 31) / 32) * 8192,
            "kv_pack positions exceed the cache head stride");
    kv_pack(kv_dtype == DRT_BF16, k, v, src_dtype == DRT_BF16, n, hkv, pos0, cache, head_stride,
            as_stream(stream));
  });
}

size_t drt_op_attention_workspace_bytes(int32_t rows, int32_t hq, int32_t hkv, int32_t n_keys) {
  if (rows <= 0 || hq <= 0 || hkv <= 0 || hq % hkv || n_keys <= 0) return 0;
  const AttnPlan p = plan_attention(rows, hq, hkv, n_keys, (size_t)256 << 20);
  const size_t general = attention_part_bytes(p, rows, hq, hkv);
  const size_t decode = attention_decode_part_bytes(attention_decode_ranges(n_keys, hkv), hkv, rows * (hq / hkv));
  // + the kernels' Q operand: the caller's Q as the hi plane and a zero lo plane
  const size_t q_planes = ((size_t)2 * rows * hq * 128 * 2 + 255) / 256 * 256;
  return std::max(general, decode) + q_planes + 256;
}

int32_t drt_op_attention(const void* q, const void* cache, int64_t head_stride, int32_t kv_dtype,
                         int32_t rows, int32_t hq, int32_t hkv, int32_t n_keys, int32_t row_pos0,
                         int32_t mask_kind, int32_t mask_prompt_len, int32_t mask_block_size,
                         void* out, int32_t out_dtype, void* workspace, size_t workspace_bytes,
                         void* stream) {
  return guarded([&] {
    require(q && cache && out && rows > 0 && hq > 0 && hkv > 0 && hq % hkv == 0 && n_keys > 0,
            "bad attention arguments");
    require(kv_dtype == DRT_F16 || kv_dtype == DRT_BF16, "attention cache must be F16 or BF16");
    require(out_dtype == DRT_F32 || out_dtype == DRT_BF16, "attention out must be F32 or BF16");
    require(mask_kind == DRT_MASK_BIDIRECTIONAL || mask_kind == DRT_MASK_D2F_HYBRID,
            "attention mask kind must be bidirectional or d2f_hybrid");
    if (mask_kind == DRT_MASK_D2F_HYBRID)
      require(mask_block_size >= 1 && mask_prompt_len >= 0, "d2f_hybrid needs a mask geometry");
    require(head_stride >= (int64_t)((n_keys + 31) / 32) * 8192, "n_keys exceed the cache");
    require(workspace && workspace_bytes >= drt_op_attention_workspace_bytes(rows, hq, hkv, n_keys),
            "attention workspace too small");
    ForwardArgs fa;
    fa.row0 = row_pos0;
    fa.n_rows = rows;
    fa.n_keys = n_keys;
    fa.mask_kind = mask_kind == DRT_MASK_D2F_HYBRID ? 1 : 0;
    fa.mask_prompt_len = mask_prompt_len;
    fa.mask_block = std::max(1, mask_block_size);
    // the caller's Q (already in the operand type) is the kernels' hi plane and
    // their lo plane is zero: read in place, nothing staged
    const size_t q_bytes = (size_t)rows * hq * 128 * 2;
    float* o_part = (float*)((char*)workspace + (2 * q_bytes + 255) / 256 * 256);
    const int ofmt = out_dtype == DRT_F32 ? 2 : 3;
    if (rows * (hq / hkv) <= 128 && one_segment(fa)) {
      const int ranges = attention_decode_ranges(n_keys, hkv);
      attention_decode(kv_dtype == DRT_BF16, q, cache, head_stride, rows, hq, hkv, n_keys,
                       nullptr, ranges, o_part, out, nullptr, ofmt, as_stream(stream), nullptr,
                       false);
    } else {
      const AttnPlan p = plan_attention(rows, hq, hkv, n_keys, (size_t)256 << 20);
      float* ml_part = o_part + (size_t)p.splits * hkv * rows * (hq / hkv) * 128;
      attention(kv_dtype == DRT_BF16, q, cache, head_stride, rows, hq, hkv, n_keys, row_pos0,
                fa.mask_kind, mask_prompt_len, fa.mask_block, p, o_part, ml_part, out, nullptr,
                ofmt, as_stream(stream), nullptr, false);
    }
  });
}

int32_t drt_op_rms_norm(const float* x, const void* weight, float eps, float* y, int32_t rows,
                        int32_t d, void* stream) {
  return guarded([&] {
    require(x && weight && y && rows > 0 && d > 0, "bad rms_norm arguments");
    rms_norm_rows(x, (const uint16_t*)weight, eps, y, rows, d, as_stream(stream));
  });
}

int32_t drt_op_rope(const float* x, const float* cos_t, const float* sin_t, float* y,
                    int32_t rows, int32_t h, int32_t hd, void* stream) {
  return guarded([&] {
    require(x && cos_t && sin_t && y && rows > 0 && h > 0 && hd > 0 && hd % 2 == 0,
            "bad rope arguments");
    rope_rows(x, cos_t, sin_t, y, rows, h, hd, as_stream(stream));
  });
}

int32_t drt_op_swiglu(const float* gate, const float* up, float* y, int64_t n, void* stream) {
  return guarded([&] {
    require(gate && up && y && n > 0, "bad swiglu arguments");
    swiglu_rows(gate, up, y, n, as_stream(stream));
  });
}

size_t drt_op_lm_head_workspace_bytes(int32_t rows, int32_t n, int32_t k) {
  if (rows <= 0 || n <= 0 || k <= 0) return 0;
  return (size_t)2 * rows * k * 2 + (size_t)rows * (k / 64) * 4 + lmhead_stats_bytes(rows, n) + 512;
}

int32_t drt_op_lm_head_score(const void* qw, const void* sb, const void* wb, int32_t rows,
                             int32_t n, int32_t k, const float* x, float temperature,
                             uint64_t seed, int32_t step, const int32_t* positions,
                             double* scores, int32_t* tokens, float* logits, void* workspace,
                             size_t workspace_bytes, void* stream) {
  return guarded([&] {
    const bool q4 = qw && sb;
    require(q4 || wb, "lm_head needs q4 (qw, sb) or bf16 (wb) weights");
    require(x && scores && tokens && rows > 0 && n > 0 && k > 0, "bad lm_head arguments");
    require(n % 64 == 0 && k % 64 == 0, "lm_head needs n % 64 == 0 and k % 64 == 0");
    require(!(temperature > 0.f) || positions, "sampling needs positions");
    require(workspace && workspace_bytes >= drt_op_lm_head_workspace_bytes(rows, n, k),
            "lm_head workspace too small");
    LinearW w;
    w.N = n;
    w.K = k;
    w.q4 = q4;
    if (q4) {
      w.qw.p = const_cast<void*>(qw);
      w.sb.p = const_cast<void*>(sb);
    } else {
      w.wb.p = const_cast<void*>(wb);
    }
    char* ws = (char*)workspace;
    void* act = ws;
    float* xs = (float*)(ws + (size_t)2 * rows * k * 2);  // after the hi and lo planes
    void* stats = ws + (size_t)2 * rows * k * 2 + (size_t)rows * (k / 64) * 4;
    stats = (void*)(((uintptr_t)stats + 255) & ~(uintptr_t)255);
    hipStream_t st = as_stream(stream);
    auto release = [&] { w.qw.p = nullptr; w.sb.p = nullptr; w.wb.p = nullptr; };
    try {
      if (q4) q4_act_prep(x, false, rows, k, (_Float16*)act, xs, st);
      else to_bf16(x, (uint16_t*)act, (int64_t)rows * k, st);
      lmhead(w, act, xs, rows, logits, stats, temperature, seed, step, positions, scores, tokens,
             st);
    } catch (...) {
      release();
      throw;
    }
    release();
  });
}

}  // extern "C"
